"""The optimizer step that refreshes an FFI layer's transposed weights
(haste_sgd_sr_step_wt, used by SRSgd for weights whose backward keeps an index
plan): bit-identical to the plain SGD step, and the next backward, which reuses
the refreshed W^T instead of gathering it, bit-identical to one that gathers."""
import numpy as np
import pytest
import torch

import oracle
from haste_amd import _C, _lib, bindings
from haste_amd.optim_sr import SRSgd
from haste_amd.rewire import GroupFixedFanIn

pytestmark = pytest.mark.gpu


def bits(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("B,D,O,G,F,gdt,use_mom,do_sr", [
    (64, 768, 4133, 32, 32, torch.bfloat16, False, True),
    (100, 300, 2001, 64, 128, torch.float32, True, True),
    (37, 200, 700, 128, 64, torch.float16, False, False),
    (96, 512, 1000, 16, 48, torch.bfloat16, True, True),
])
def test_sgd_wt_matches_sgd_and_gather(dev, B, D, O, G, F, gdt, use_mom, do_sr):
    g = torch.Generator(device=dev).manual_seed(O)
    Gc = (O + G - 1) // G
    W = ((torch.rand(O, F, generator=g, device=dev) * 2 - 1) / F ** 0.5).to(torch.bfloat16)
    grad = (torch.randn(O, F, generator=g, device=dev) * 0.05).to(gdt)
    m = torch.randn(O, F, generator=g, device=dev) * 0.01
    idx = torch.randint(0, D, (Gc, F), generator=g, device=dev, dtype=torch.int32)
    dY = (torch.randn(B, O, generator=g, device=dev) * 0.1).to(torch.bfloat16)
    lr, wd, mu, seed = 0.05, 1e-4, 0.9, 1234
    st = _C.stream_of(W)
    # plain SGD
    W1, m1 = W.clone(), m.clone()
    _lib.call("haste_sgd_sr_step", W1.data_ptr(), grad.data_ptr(), _C.dtype_code(gdt),
              m1.data_ptr() if use_mom else None, W1.numel(), lr, wd, mu, int(use_mom),
              int(do_sr), seed, 0, st)
    # SGD + W^T refresh into a planned workspace
    ws = _C.bwd_features_workspace(B, D, F, O, G, torch.bfloat16, dev)
    _lib.call("haste_ffi_bwd_features_plan", idx.data_ptr(), ws.data_ptr(), ws.numel(), B, D, F,
              O, G, _lib.DTYPE_BF16, st)
    W2, m2 = W.clone(), m.clone()
    _lib.call("haste_sgd_sr_step_wt", W2.data_ptr(), grad.data_ptr(), _C.dtype_code(gdt),
              m2.data_ptr() if use_mom else None, lr, wd, mu, int(use_mom), int(do_sr), seed,
              ws.data_ptr(), ws.numel(), B, D, F, O, G, _lib.DTYPE_BF16, st)
    torch.cuda.synchronize()
    assert np.array_equal(bits(W1), bits(W2))
    if use_mom:
        assert torch.equal(m1.view(torch.int32), m2.view(torch.int32))
    # bwd-features reusing the refreshed W^T (plan_ready 2) == gathering it (1)
    outs = []
    for ready in (2, 1):
        dxt = torch.empty(D, B, dtype=torch.float32, device=dev)
        _lib.call("haste_ffi_bwd_features", idx.data_ptr(), W2.data_ptr(), dY.data_ptr(), O,
                  dxt.data_ptr(), ws.data_ptr(), ws.numel(), B, D, F, O, G, _lib.DTYPE_BF16,
                  ready, st)
        outs.append(dxt)
    torch.cuda.synchronize()
    assert torch.equal(outs[0].view(torch.int32), outs[1].view(torch.int32))
    torch.testing.assert_close(outs[0].cpu(), oracle.ffi_backward_features(
        idx.cpu(), W2.cpu(), dY.cpu(), G, D), rtol=1e-4, atol=1e-5)


@pytest.mark.parametrize("B,D,O,G,F,gdt,bdt,use_mom,do_sr", [
    (64, 768, 4133, 32, 32, torch.bfloat16, torch.bfloat16, True, True),
    (100, 300, 2001, 64, 128, torch.float32, torch.float32, False, True),
    (37, 200, 700, 128, 64, torch.float16, torch.bfloat16, True, False),
    (96, 512, 1000, 16, 48, torch.bfloat16, torch.float32, True, True),
])
def test_sgd_wt_bias_matches_separate_steps(dev, B, D, O, G, F, gdt, bdt, use_mom, do_sr):
    """haste_sgd_sr_step_wt_bias == haste_sgd_sr_step_wt on the weights plus
    haste_sgd_sr_step on the bias (same seed, offsets from 0), bit for bit,
    momentum buffers included."""
    g = torch.Generator(device=dev).manual_seed(O + 7)
    Gc = (O + G - 1) // G
    W = ((torch.rand(O, F, generator=g, device=dev) * 2 - 1) / F ** 0.5).to(torch.bfloat16)
    grad = (torch.randn(O, F, generator=g, device=dev) * 0.05).to(gdt)
    m = torch.randn(O, F, generator=g, device=dev) * 0.01
    bias = (torch.randn(O, generator=g, device=dev) * 0.1).to(torch.bfloat16)
    gb = (torch.randn(O, generator=g, device=dev) * 0.05).to(bdt)
    mb = torch.randn(O, generator=g, device=dev) * 0.01
    idx = torch.randint(0, D, (Gc, F), generator=g, device=dev, dtype=torch.int32)
    lr, wd, mu, seed = 0.05, 1e-4, 0.9, 99
    st = _C.stream_of(W)
    ws = _C.bwd_features_workspace(B, D, F, O, G, torch.bfloat16, dev)
    _lib.call("haste_ffi_bwd_features_plan", idx.data_ptr(), ws.data_ptr(), ws.numel(), B, D, F,
              O, G, _lib.DTYPE_BF16, st)
    mp = (lambda t: t.data_ptr() if use_mom else None)
    W1, m1, b1, mb1 = W.clone(), m.clone(), bias.clone(), mb.clone()
    _lib.call("haste_sgd_sr_step_wt", W1.data_ptr(), grad.data_ptr(), _C.dtype_code(gdt), mp(m1),
              lr, wd, mu, int(use_mom), int(do_sr), seed, ws.data_ptr(), ws.numel(), B, D, F, O,
              G, _lib.DTYPE_BF16, st)
    _lib.call("haste_sgd_sr_step", b1.data_ptr(), gb.data_ptr(), _C.dtype_code(bdt), mp(mb1), O,
              lr, wd, mu, int(use_mom), int(do_sr), seed, 0, st)
    torch.cuda.synchronize()
    wt1 = ws.clone()
    W2, m2, b2, mb2 = W.clone(), m.clone(), bias.clone(), mb.clone()
    _lib.call("haste_sgd_sr_step_wt_bias", W2.data_ptr(), grad.data_ptr(), _C.dtype_code(gdt),
              mp(m2), b2.data_ptr(), gb.data_ptr(), _C.dtype_code(bdt), mp(mb2), lr, wd, mu,
              int(use_mom), int(do_sr), seed, ws.data_ptr(), ws.numel(), B, D, F, O, G,
              _lib.DTYPE_BF16, st)
    torch.cuda.synchronize()
    assert np.array_equal(bits(W1), bits(W2))
    assert np.array_equal(bits(b1), bits(b2))
    assert not np.array_equal(bits(b2), bits(bias))
    assert torch.equal(wt1, ws)
    if use_mom:
        assert torch.equal(m1.view(torch.int32), m2.view(torch.int32))
        assert torch.equal(mb1.view(torch.int32), mb2.view(torch.int32))


def test_training_loop_with_refresh_matches_without(dev):
    """Three SRSgd steps of a drop-in layer: refreshing W^T in the optimizer
    (and skipping the gather in the backward) gives the same weights, bias and
    input gradients, bit for bit, as the plain path; an in-place change of the
    weights between steps is seen (the backward gathers again)."""
    B, D, O, G, F = 64, 300, 3001, 64, 64

    def run(refresh):
        bindings._WS_CACHE.clear()
        torch.manual_seed(0)
        layer = GroupFixedFanIn(D, O, F, group_size=G, rewire_threshold=0.0,
                                dtype=torch.bfloat16).to(dev)
        opt = SRSgd(layer.parameters(), lr=0.05, weight_decay=1e-4, momentum=0.9, seed=42,
                    refresh_transposed=refresh)
        gx = []
        gen = torch.Generator(device=dev).manual_seed(1)
        for step in range(3):
            x = torch.randn(B, D, generator=gen, device=dev).to(torch.bfloat16).requires_grad_(True)
            dY = (torch.randn(B, O, generator=gen, device=dev) * 0.1).to(torch.bfloat16)
            opt.zero_grad()
            layer(x).backward(dY)
            gx.append(x.grad.clone())
            opt.step()
            if step == 1:
                with torch.no_grad():
                    layer.weights.mul_(0.75)   # a change the optimizer did not make
        torch.cuda.synchronize()
        return layer, gx

    a, gxa = run(True)
    b, gxb = run(False)
    for u, v in zip(gxa, gxb):
        assert torch.equal(u.view(torch.int16), v.view(torch.int16))
    for (ka, va), (kb, vb) in zip(a.state_dict().items(), b.state_dict().items()):
        assert torch.equal(va, vb), ka


@pytest.mark.parametrize("clear", [True, False])
def test_edit_through_data_needs_clear_wt_refreshed(dev, clear):
    """An edit through ``W.data`` does not move the weights' version counter, so
    the refreshed W^T would be reused: ``bindings.clear_wt_refreshed(W)``, called
    as documented, makes the next backward gather again (input gradients then
    equal the plain path's bit for bit); without it they differ."""
    B, D, O, G, F = 64, 300, 3001, 64, 64

    def run(refresh, clear_after_edit):
        bindings._WS_CACHE.clear()
        torch.manual_seed(0)
        layer = GroupFixedFanIn(D, O, F, group_size=G, rewire_threshold=0.0,
                                dtype=torch.bfloat16).to(dev)
        opt = SRSgd(layer.parameters(), lr=0.05, weight_decay=1e-4, momentum=0.9, seed=42,
                    refresh_transposed=refresh)
        gen = torch.Generator(device=dev).manual_seed(1)
        gx = []
        for step in range(3):
            x = torch.randn(B, D, generator=gen, device=dev).to(torch.bfloat16).requires_grad_(True)
            dY = (torch.randn(B, O, generator=gen, device=dev) * 0.1).to(torch.bfloat16)
            opt.zero_grad()
            layer(x).backward(dY)
            gx.append(x.grad.clone())
            opt.step()
            if step == 1:
                layer.weights.data.mul_(0.75)
                if clear_after_edit:
                    bindings.clear_wt_refreshed(layer.weights)
        torch.cuda.synchronize()
        return gx

    a = run(True, clear)
    b = run(False, False)
    assert torch.equal(a[1].view(torch.int16), b[1].view(torch.int16))
    same = torch.equal(a[2].view(torch.int16), b[2].view(torch.int16))
    assert same == clear


def test_same_shape_layers_keep_their_own_plans(dev):
    """Two FFI layers of one shape each keep their own workspace: after
    alternating backwards both index plans are still valid (none is rebuilt)."""
    B, D, O, G, F = 32, 256, 2000, 32, 32
    bindings._WS_CACHE.clear()
    torch.manual_seed(3)
    layers = [GroupFixedFanIn(D, O, F, group_size=G, rewire_threshold=0.0,
                              dtype=torch.bfloat16).to(dev) for _ in range(2)]
    gen = torch.Generator(device=dev).manual_seed(4)
    for _ in range(2):
        for layer in layers:
            x = torch.randn(B, D, generator=gen, device=dev).to(torch.bfloat16).requires_grad_(True)
            layer(x).backward(torch.ones(B, O, device=dev, dtype=torch.bfloat16))
    torch.cuda.synchronize()
    assert len(bindings._WS_CACHE) == 2
    for layer in layers:
        locs = layer.group_locations
        assert sum(ent.plan_valid(locs) for ent in bindings._WS_CACHE.values()) == 1
