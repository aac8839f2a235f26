"""GPU tests of the drop-in Python API (ops / bindings / optim_sr / rewire / step)."""
import math

import numpy as np
import pytest
import torch

import oracle
from haste_amd import backward_features, backward_weights, ffi_forward, ops
from haste_amd.optim_sr import SGD_SR, SRSgd
from haste_amd.rewire import GroupFixedFanIn
from haste_amd.step import FFITrainStep

pytestmark = pytest.mark.gpu
TOL16 = dict(rtol=1e-2, atol=1e-3)


def bits(t):
    return t.detach().cpu().view(torch.int16).numpy().view(np.uint16)


def test_module_level_functions(dev):
    B, D, O, G, F = 32, 256, 1000, 32, 64
    g = torch.Generator().manual_seed(0)
    x = torch.randn(B, D, generator=g).to(torch.bfloat16)
    W = (torch.randn(O, F, generator=g) * 0.1).to(torch.bfloat16)
    idx = torch.randint(0, D, ((O + G - 1) // G, F), generator=g, dtype=torch.int32)
    dY = (torch.randn(B, O, generator=g) * 0.1).to(torch.bfloat16)
    xT = x.t().contiguous()
    out = ffi_forward(idx.to(dev), xT.to(dev), W.to(dev), None, G)
    torch.testing.assert_close(out.float().cpu(), oracle.ffi_forward(idx, xT, W, None, G), **TOL16)
    dxt = backward_features(xT.to(dev), W.to(dev), idx.to(dev), dY.to(dev), G)
    torch.testing.assert_close(dxt.cpu(), oracle.ffi_backward_features(idx, W, dY, G, D), rtol=1e-4, atol=1e-5)
    dw = backward_weights(xT.to(dev), W.to(dev), idx.to(dev), dY.to(dev), G)
    torch.testing.assert_close(dw.float().cpu(), oracle.ffi_backward_weights(idx, xT, dY, G), **TOL16)


@pytest.mark.parametrize("B,D,O,G,F", [(64, 768, 4096, 32, 32), (50, 300, 1001, 64, 128)])
def test_autograd_matches_oracle(dev, B, D, O, G, F):
    torch.manual_seed(1)
    layer = GroupFixedFanIn(D, O, F, group_size=G, prune_mode="fraction", rewire_fraction=0.15,
                            dtype=torch.bfloat16)
    with torch.no_grad():
        layer.bias.copy_(torch.randn(O) * 0.1)
    W, bias, idx = layer.weights.detach().clone(), layer.bias.detach().clone(), layer.group_locations.clone()
    layer = layer.to(dev)
    x = torch.randn(B, D).to(torch.bfloat16)
    dY = (torch.randn(B, O) * 0.1).to(torch.bfloat16)
    xd = x.to(dev).requires_grad_(True)
    out = layer(xd)
    out.backward(dY.to(dev))
    xT = x.t().contiguous()
    torch.testing.assert_close(out.detach().float().cpu(), oracle.ffi_forward(idx, xT, W, bias, G), **TOL16)
    ref_dx = oracle.ffi_backward_features(idx, W, dY, G, D).t().contiguous()
    torch.testing.assert_close(xd.grad.float().cpu(), ref_dx, **TOL16)
    # grad_X is SR-rounded with seed 123 (bindings.py:48): check the bits against the
    # oracle SR of the GPU's own fp32 feature gradient
    dxt = backward_features(xT.to(dev), W.to(dev), idx.to(dev), dY.to(dev), G)
    exp = oracle.sr_round_bf16(dxt.t().contiguous().cpu().numpy(), 123)
    assert np.array_equal(bits(xd.grad), exp)
    torch.testing.assert_close(layer.weights.grad.float().cpu(), oracle.ffi_backward_weights(idx, xT, dY, G), **TOL16)
    torch.testing.assert_close(layer.bias.grad.float().cpu(), oracle.bias_grad(dY), **TOL16)
    assert layer.weights.grad.dtype == torch.bfloat16 and layer.bias.grad.dtype == torch.bfloat16


def test_autograd_3d_input_and_no_bias(dev):
    torch.manual_seed(2)
    layer = GroupFixedFanIn(128, 512, 32, bias=False, group_size=16, rewire_threshold=0.01,
                            dtype=torch.bfloat16).to(dev)
    x = torch.randn(3, 5, 128, device=dev).to(torch.bfloat16).requires_grad_(True)
    out = layer(x)
    assert out.shape == (3, 5, 512)
    out.float().sum().backward()
    assert x.grad.shape == x.shape and layer.weights.grad is not None


def test_srsgd_matches_oracle_and_increments_seed(dev):
    torch.manual_seed(3)
    W = torch.nn.Parameter(((torch.rand(1000, 64) - 0.5) * 0.2).to(torch.bfloat16).to(dev))
    b = torch.nn.Parameter(torch.zeros(1000, dtype=torch.bfloat16, device=dev))
    opt = SRSgd([W, b], lr=0.05, weight_decay=1e-4, momentum=0.0, seed=42)
    for step in range(2):
        W.grad = (torch.randn(1000, 64, device=dev) * 0.01).to(torch.bfloat16)
        b.grad = (torch.randn(1000, device=dev) * 0.01).to(torch.bfloat16)
        w0, g0, b0, gb0 = bits(W), bits(W.grad), bits(b), bits(b.grad)
        opt.step()
        ref_w, _ = oracle.sgd_sr_step(w0, g0, None, 0.05, 1e-4, 0.0, False, True, 42 + step)
        ref_b, _ = oracle.sgd_sr_step(b0, gb0, None, 0.05, 1e-4, 0.0, False, True, 42 + step)
        assert np.array_equal(bits(W), ref_w.reshape(1000, 64))
        assert np.array_equal(bits(b), ref_b)
    assert opt.param_groups[0]["seed"] == 44
    assert SGD_SR is SRSgd


def test_srsgd_momentum_and_fp32_params(dev):
    torch.manual_seed(4)
    W = torch.nn.Parameter(((torch.rand(256, 32) - 0.5) * 0.2).to(torch.bfloat16).to(dev))
    P = torch.nn.Parameter(torch.randn(100, device=dev))
    opt = SRSgd([W, P], lr=0.1, weight_decay=1e-3, momentum=0.9, seed=5)
    W.grad_dtype = torch.float32  # fp32 gradient for a bf16 parameter
    W.grad = torch.randn(256, 32, device=dev) * 0.01
    P.grad = torch.randn(100, device=dev)
    w0, g0 = bits(W), W.grad.cpu().numpy()
    p0 = P.detach().clone()
    opt.step()
    ref_w, ref_m = oracle.sgd_sr_step(w0, g0, np.zeros(256 * 32, np.float32), 0.1, 1e-3, 0.9, True, True, 5)
    assert np.array_equal(bits(W), ref_w.reshape(256, 32))
    assert np.array_equal(opt.state[W]["momentum_buf"].cpu().numpy().reshape(-1).view(np.uint32),
                          ref_m.view(np.uint32))
    exp_p = p0 - 0.1 * (P.grad + 1e-3 * p0)
    torch.testing.assert_close(P.detach(), exp_p, rtol=1e-6, atol=1e-6)


def test_fp32_grads_mode(dev):
    """fp32_grads=True: weight/bias gradients come out of the kernel in fp32."""
    torch.manual_seed(7)
    B, D, O, G, F = 64, 768, 4096, 32, 32
    layer = GroupFixedFanIn(D, O, F, group_size=G, rewire_threshold=0.0, dtype=torch.bfloat16,
                            fp32_grads=True)
    W, idx = layer.weights.detach().clone(), layer.group_locations.clone()
    layer = layer.to(dev)
    x = torch.randn(B, D).to(torch.bfloat16)
    dY = (torch.randn(B, O) * 0.1).to(torch.bfloat16)
    layer(x.to(dev)).backward(dY.to(dev))
    assert layer.weights.grad.dtype == torch.float32 and layer.bias.grad.dtype == torch.float32
    torch.testing.assert_close(layer.weights.grad.cpu(),
                               oracle.ffi_backward_weights(idx, x.t().contiguous(), dY, G),
                               rtol=1e-4, atol=1e-5)
    torch.testing.assert_close(layer.bias.grad.cpu(), oracle.bias_grad(dY), rtol=1e-4, atol=1e-5)
    w0, g0 = bits(layer.weights), layer.weights.grad.cpu().numpy()
    SRSgd(layer.parameters(), lr=0.05, weight_decay=1e-4, seed=42).step()
    ref_w, _ = oracle.sgd_sr_step(w0, g0, None, 0.05, 1e-4, 0.0, False, True, 42)
    assert np.array_equal(bits(layer.weights), ref_w.reshape(O, F))


def test_module_rewire_matches_oracle(dev):
    torch.manual_seed(5)
    layer = GroupFixedFanIn(768, 5000, 64, group_size=64, prune_mode="fraction", rewire_fraction=0.15,
                            init_mode="zero", dtype=torch.bfloat16)
    w0 = bits(layer.weights)
    idx0 = layer.group_locations.numpy().copy()
    layer = layer.to(dev)
    layer.rewire(seed=99)
    ref_w, ref_idx, n, _, _ = oracle.rewire(w0, idx0, 64, 768, prune_mode=oracle.PRUNE_FRACTION,
                                            k=int(64 * 0.15), init_mode=oracle.INIT_ZERO,
                                            bound=1 / math.sqrt(64), seed=99)
    assert np.array_equal(layer.group_locations.cpu().numpy(), ref_idx)
    assert np.array_equal(bits(layer.weights), ref_w)
    assert layer.pruned_total == n == 79 * 9
    sd = layer.state_dict()
    assert set(sd) == {"weights", "bias", "group_locations"}
    assert sd["group_locations"].dtype == torch.int32


def test_train_step_matches_api(dev):
    """FFITrainStep (fp32 grads) agrees with the autograd path + oracle SGD."""
    torch.manual_seed(6)
    B, D, O, G, F = 64, 768, 4096, 32, 32
    layer = GroupFixedFanIn(D, O, F, group_size=G, rewire_threshold=0.0, dtype=torch.bfloat16).to(dev)
    x = torch.randn(B, D, device=dev).to(torch.bfloat16)
    dY = (torch.randn(B, O, device=dev) * 0.1).to(torch.bfloat16)
    w0 = bits(layer.weights)
    st = FFITrainStep(layer.weights.data, layer.bias.data, layer.group_locations, B, D, G, 0.05, 1e-4, seed=42)
    logits = st.forward(x)
    ref = oracle.ffi_forward(layer.group_locations.cpu(), x.t().contiguous().cpu(),
                             layer.weights.detach().cpu(), layer.bias.detach().cpu(), G)
    torch.testing.assert_close(logits.float().cpu(), ref, **TOL16)
    st.backward(dY, dY.stride(0))
    torch.cuda.synchronize()
    ref_dw = oracle.ffi_backward_weights(layer.group_locations.cpu(), x.t().contiguous().cpu(), dY.cpu(), G)
    torch.testing.assert_close(st.dW.cpu(), ref_dw, rtol=1e-4, atol=1e-5)
    dw_np = st.dW.cpu().numpy()
    st.sgd()
    torch.cuda.synchronize()
    ref_w, _ = oracle.sgd_sr_step(w0, dw_np, None, 0.05, 1e-4, 0.0, False, True, 42)
    assert np.array_equal(bits(layer.weights), ref_w.reshape(O, F))
    assert st.seed == 43


def test_train_step_replans_after_rewire(dev):
    """FFITrainStep reuses its index plan across steps and rebuilds it when
    rewire() changes group_locations."""
    torch.manual_seed(8)
    B, D, O, G, F = 96, 768, 5000, 64, 64
    layer = GroupFixedFanIn(D, O, F, group_size=G, prune_mode="fraction", rewire_fraction=0.25,
                            dtype=torch.bfloat16).to(dev)
    x = torch.randn(B, D, device=dev).to(torch.bfloat16)
    st = FFITrainStep(layer.weights.data, layer.bias.data, layer.group_locations, B, D, G, 0.05,
                      1e-4, seed=1)
    dY = torch.zeros(B, st.ldo, dtype=torch.bfloat16, device=dev)
    dY[:, :O] = (torch.randn(B, O, device=dev) * 0.1).to(torch.bfloat16)

    def check():
        st.backward_features(dY, st.ldo)
        torch.cuda.synchronize()
        ref = oracle.ffi_backward_features(layer.group_locations.cpu(), layer.weights.detach().cpu(),
                                           dY[:, :O].cpu(), G, D)
        # bf16 SR of the fp32 gradient: within one bf16 ulp (2^-7 relative at
        # most) of the oracle's values, inside the north star's 1e-2 / 1e-3
        torch.testing.assert_close(st.dX.float().cpu(), ref.t(), **TOL16)

    check()
    check()  # plan reused
    v0 = layer.group_locations._version
    layer.rewire(seed=3)
    assert layer.group_locations._version != v0
    check()  # plan rebuilt for the new indices


@pytest.mark.parametrize("H", [1000, 1001])
def test_head_tail_logits_match_cat(dev, H):
    """ops.head_tail_logits equals torch.cat((head(x), group_ffi_mul(x, ...)), 1) of
    src/model.py:245-248 in values and gradients; the tail lands in place on
    16-byte aligned rows of the concatenated buffer."""
    B, D, O, G, F = 64, 256, 3000, 32, 64
    torch.manual_seed(3)
    x = torch.randn(B, D, device=dev).to(torch.bfloat16)
    head = torch.nn.Linear(D, H).to(dev).to(torch.bfloat16)
    W = (torch.randn(O, F, device=dev) * 0.1).to(torch.bfloat16)
    bias = (torch.randn(O, device=dev) * 0.1).to(torch.bfloat16)
    idx = torch.randint(0, D, ((O + G - 1) // G, F), dtype=torch.int32, device=dev)
    g_out = (torch.randn(B, H + O, device=dev) * 0.1).to(torch.bfloat16)

    def run(fused):
        xr = x.clone().requires_grad_(True)
        hd = torch.nn.Linear(D, H).to(dev).to(torch.bfloat16)
        hd.load_state_dict(head.state_dict())
        Wr, br = W.clone().requires_grad_(True), bias.clone().requires_grad_(True)
        if fused:
            out = ops.head_tail_logits(xr, hd, xr, Wr, idx, br, G)
        else:
            out = torch.cat((hd(xr), ops.group_ffi_mul(xr, Wr, idx, br, G)), dim=1)
        out.backward(g_out)
        return out.detach(), xr.grad, hd.weight.grad, hd.bias.grad, Wr.grad, br.grad

    o_ref, gx_ref, ghw_ref, ghb_ref, gw_ref, gb_ref = run(False)
    o, gx, ghw, ghb, gw, gb = run(True)
    assert o.shape == (B, H + O)
    # the tail and its gradients against the CPU oracle
    xc, Wc, bc, idxc = x.cpu(), W.cpu(), bias.cpu(), idx.cpu()
    gt = g_out[:, H:].cpu()
    xT = xc.t().contiguous()
    torch.testing.assert_close(o[:, H:].float().cpu(), oracle.ffi_forward(idxc, xT, Wc, bc, G), **TOL16)
    torch.testing.assert_close(gw.float().cpu(), oracle.ffi_backward_weights(idxc, xT, gt, G), **TOL16)
    torch.testing.assert_close(gb.float().cpu(), oracle.bias_grad(gt), **TOL16)
    # grad of x = the head's dense gradient (fp32 here) + the tail's.  On the GPU
    # each half is rounded to bf16 (the tail stochastically, up to one ulp) and
    # autograd adds them in bf16.  The halves reach |0.5| here (bf16 ulp 2^-9
    # below 0.5) while their sum can cancel to ~0, so the error bound is
    # absolute: half an ulp + one ulp + half an ulp of terms below 0.5 < 4e-3
    gx_exp = (g_out[:, :H].float().cpu() @ head.weight.float().cpu()
              + oracle.ffi_backward_features(idxc, Wc, gt, G, D).t())
    torch.testing.assert_close(gx.float().cpu(), gx_exp, rtol=1e-2, atol=4e-3)
    assert (o[:, H:].data_ptr() % 16 == 0) and o.stride(0) % 8 == 0
    assert np.array_equal(bits(o), bits(o_ref))
    assert np.array_equal(bits(gw), bits(gw_ref)) and np.array_equal(bits(gb), bits(gb_ref))
    torch.testing.assert_close(ghw.float(), ghw_ref.float(), **TOL16)
    torch.testing.assert_close(ghb.float(), ghb_ref.float(), **TOL16)
    torch.testing.assert_close(gx.float(), gx_ref.float(), **TOL16)


def test_autograd_reuses_plan_until_indices_change(dev):
    """The drop-in backward keeps the index plan of its workspace across calls and
    rebuilds it after the indices change (rewire, in-place edit): gradients match
    the oracle every time."""
    B, D, O, G, F = 64, 300, 1000, 32, 64
    torch.manual_seed(5)
    layer = GroupFixedFanIn(D, O, F, group_size=G, prune_mode="fraction", rewire_fraction=0.2,
                            dtype=torch.bfloat16).to(dev)
    x = torch.randn(B, D).to(torch.bfloat16)
    dY = (torch.randn(B, O) * 0.1).to(torch.bfloat16)

    def check():
        xd = x.to(dev).requires_grad_(True)
        layer.zero_grad()
        layer(xd).backward(dY.to(dev))
        idx = layer.group_locations.cpu()
        W = layer.weights.detach().cpu()
        ref = oracle.ffi_backward_features(idx, W, dY, G, D).t().contiguous()
        torch.testing.assert_close(xd.grad.float().cpu(), ref, **TOL16)

    check()
    check()                         # plan reused
    layer.rewire(seed=1)            # indices change (version bump)
    check()
    with torch.no_grad():
        layer.group_locations[0].copy_(torch.arange(F, dtype=torch.int32, device=dev))
    check()


@pytest.mark.parametrize("O,in_place", [(1024, True), (1003, True), (12, False)])
def test_autograd_grad_output_layout(dev, monkeypatch, O, in_place):
    """The backward reads autograd's [B, O] grad_output in place whatever its row
    alignment (O = 1003: rows on 2-byte boundaries) and copies it only when the
    kernels' unaligned-row path does not apply (O < 16 with unaligned rows);
    the gradients match the oracle either way."""
    from haste_amd import _C

    B, D, G, F = 48, 300, 64, 64
    torch.manual_seed(9)
    layer = GroupFixedFanIn(D, O, F, group_size=G, rewire_threshold=0.0, dtype=torch.bfloat16)
    W, idx = layer.weights.detach().clone(), layer.group_locations.clone()
    layer = layer.to(dev)
    x = torch.randn(B, D).to(torch.bfloat16)
    dY = (torch.randn(B, O) * 0.1).to(torch.bfloat16)
    seen = []
    orig = _C.grad_rows

    def spy(t):
        out = orig(t)
        seen.append(out[0].data_ptr() == t.data_ptr())
        return out

    monkeypatch.setattr(_C, "grad_rows", spy)
    xd = x.to(dev).requires_grad_(True)
    layer(xd).backward(dY.to(dev))
    assert seen == [in_place]
    torch.testing.assert_close(xd.grad.float().cpu(),
                               oracle.ffi_backward_features(idx, W, dY, G, D).t(), **TOL16)
    torch.testing.assert_close(layer.weights.grad.float().cpu(),
                               oracle.ffi_backward_weights(idx, x.t().contiguous(), dY, G), **TOL16)
    torch.testing.assert_close(layer.bias.grad.float().cpu(), oracle.bias_grad(dY), **TOL16)


def test_train_step_sees_weight_changes_made_outside(dev):
    """FFITrainStep keys the reuse of its transposed weights on the version
    counter of the tensor it was given (here the Parameter): after its own
    fused update the reuse is valid; after an in-place change through the
    Parameter it gathers them again, so dX follows the new weights."""
    torch.manual_seed(10)
    B, D, O, G, F = 64, 300, 2000, 64, 64
    layer = GroupFixedFanIn(D, O, F, group_size=G, rewire_threshold=0.0, dtype=torch.bfloat16).to(dev)
    x = torch.randn(B, D, device=dev).to(torch.bfloat16)
    st = FFITrainStep(layer.weights, layer.bias, layer.group_locations, B, D, G, 0.05, 1e-4, seed=3)
    dY = torch.zeros(B, st.ldo, dtype=torch.bfloat16, device=dev)
    dY[:, :O] = (torch.randn(B, O, device=dev) * 0.1).to(torch.bfloat16)

    def check():
        st.backward_features(dY, st.ldo)
        torch.cuda.synchronize()
        ref = oracle.ffi_backward_features(layer.group_locations.cpu(), layer.weights.detach().cpu(),
                                           dY[:, :O].cpu(), G, D)
        torch.testing.assert_close(st.dX.float().cpu(), ref.t(), **TOL16)

    st.forward(x)
    check()
    v0 = layer.weights._version
    st.backward_weights_sgd(dY, st.ldo)        # writes W and its transpose
    assert layer.weights._version > v0
    check()
    with torch.no_grad():
        layer.weights.mul_(-0.5)               # a change the step did not make
    check()
