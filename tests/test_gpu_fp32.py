"""GPU tests of fp32 FFI layers (the reference's float instantiations:
shared_ffi/ffi_forward_kernels.cu:289-485, ffi_backward_features.cu:225-415,
ffi_backward_weights.cu:273-470).  Those kernels round the fp32 features,
weights and grad of the logits to fp16 (to nearest) as they load them and
accumulate in fp32, so the oracle is fed the fp16-rounded operands and the
results are compared in fp32: products of fp16 values are exact in fp32, only
the order of the fp32 sums differs (tolerance rtol 1e-5 / atol 1e-5 for sums of
up to 256 terms, rtol 1e-4 / atol 1e-5 for the feature gradient, whose
duplicated indices add a hi/lo split of their summed weights).  The bias
gradient is the reference's torch.sum(grad_output, 0) on the fp32 grad
(bindings.py:40), compared bit for bit with that op."""
import numpy as np
import pytest
import torch

import oracle
from haste_amd import _C, ops
from haste_amd.optim_sr import SRSgd
from haste_amd.rewire import GroupFixedFanIn

pytestmark = pytest.mark.gpu
TOL32 = dict(rtol=1e-5, atol=1e-5)
TOL32_DX = dict(rtol=1e-4, atol=1e-5)

CASES = [(64, 768, 4096, 32, 32), (128, 768, 8193, 64, 128), (37, 200, 513, 16, 64),
         (70, 300, 1000, 128, 128), (20, 512, 777, 16, 256), (24, 256, 1034, 32, 64)]


def _inputs(B, D, O, G, F, seed):
    g = torch.Generator().manual_seed(seed)
    Gc = (O + G - 1) // G
    xT = torch.randn(D, B, generator=g)
    W = (torch.rand(O, F, generator=g) * 2 - 1) / F ** 0.5
    bias = torch.randn(O, generator=g) * 0.1
    idx = torch.randint(0, D, (Gc, F), generator=g, dtype=torch.int32)  # with duplicates
    dY = torch.randn(B, O, generator=g) * 0.1
    return xT, W, bias, idx, dY


def h(t):
    """The fp16 rounding the reference's fp32 kernels apply, back in fp32."""
    return t.half().float()


@pytest.mark.parametrize("B,D,O,G,F", CASES)
def test_f32_kernels_match_oracle(dev, B, D, O, G, F):
    xT, W, bias, idx, dY = _inputs(B, D, O, G, F, seed=B + O)
    out = _C.ffi_forward_cuda(idx.to(dev), xT.to(dev), W.to(dev), bias.to(dev), B, D, F, O, G)
    assert out.dtype == torch.float32 and out.shape == (B, O)
    torch.testing.assert_close(out.cpu(), oracle.ffi_forward(idx, h(xT), h(W), bias, G), **TOL32)
    # without bias, and the padding columns of the last group are not written past O
    out0 = _C.ffi_forward_cuda(idx.to(dev), xT.to(dev), W.to(dev), None, B, D, F, O, G)
    torch.testing.assert_close(out0.cpu(), oracle.ffi_forward(idx, h(xT), h(W), None, G), **TOL32)
    dxt = _C.ffi_backward_features_cuda(xT.to(dev), W.to(dev), idx.to(dev), dY.to(dev), B, D,
                                        F, O, G)
    assert dxt.dtype == torch.float32 and dxt.shape == (D, B)
    torch.testing.assert_close(dxt.cpu(), oracle.ffi_backward_features(idx, h(W), h(dY), G, D),
                               **TOL32_DX)
    dw = _C.ffi_backward_weights_cuda(xT.to(dev), W.to(dev), idx.to(dev), dY.to(dev), B, D, F,
                                      O, G)
    assert dw.dtype == torch.float32 and dw.shape == (O, F)
    torch.testing.assert_close(dw.cpu(), oracle.ffi_backward_weights(idx, h(xT), h(dY), G),
                               **TOL32)


def test_f32_forward_rounds_operands_to_fp16(dev):
    """The fp32 layer computes with fp16 operands, as the reference: operands that
    fp16 cannot hold exactly give the fp16 product, not the fp32 one."""
    B, D, O, G, F = 16, 64, 64, 32, 32
    xT = torch.full((D, B), 1.0 + 2.0 ** -12)    # rounds to 1.0 in fp16
    W = torch.full((O, F), 1.0 / 32)
    idx = torch.arange(F, dtype=torch.int32).repeat(O // G, 1)
    out = _C.ffi_forward_cuda(idx.to(dev), xT.to(dev), W.to(dev), None, B, D, F, O, G)
    assert torch.equal(out.cpu(), torch.ones(B, O))


@pytest.mark.parametrize("B,D,O,G,F", [(64, 768, 4096, 32, 32), (50, 300, 1001, 64, 128)])
def test_f32_autograd_and_sgd(dev, B, D, O, G, F):
    torch.manual_seed(5)
    layer = GroupFixedFanIn(D, O, F, group_size=G, prune_mode="fraction", rewire_fraction=0.15,
                            dtype=torch.float32)
    with torch.no_grad():
        layer.bias.copy_(torch.randn(O) * 0.1)
    W, bias, idx = layer.weights.detach().clone(), layer.bias.detach().clone(), layer.group_locations.clone()
    layer = layer.to(dev)
    x = torch.randn(B, D)
    dY = torch.randn(B, O) * 0.1
    xd = x.to(dev).requires_grad_(True)
    out = layer(xd)
    assert out.dtype == torch.float32
    dYd = dY.to(dev)
    out.backward(dYd)
    xT = x.t().contiguous()
    torch.testing.assert_close(out.detach().cpu(), oracle.ffi_forward(idx, h(xT), h(W), bias, G),
                               **TOL32)
    ref_dx = oracle.ffi_backward_features(idx, h(W), h(dY), G, D).t().contiguous()
    assert xd.grad.dtype == torch.float32
    torch.testing.assert_close(xd.grad.cpu(), ref_dx, **TOL32_DX)
    assert layer.weights.grad.dtype == torch.float32
    torch.testing.assert_close(layer.weights.grad.cpu(),
                               oracle.ffi_backward_weights(idx, h(xT), h(dY), G), **TOL32)
    assert torch.equal(layer.bias.grad, dYd.sum(0))
    # SRSgd on fp32 parameters is the reference's torch update (optim_sr.py:73-84):
    # with momentum 0, p.add_(g + wd * p, alpha=-lr), bit for bit
    w0 = layer.weights.detach().clone()
    g0 = layer.weights.grad.clone()
    opt = SRSgd(layer.parameters(), lr=0.05, weight_decay=1e-4, momentum=0.0)
    opt.step()
    assert torch.equal(layer.weights.detach(), w0.add(g0.add(w0, alpha=1e-4), alpha=-0.05))


def test_f32_head_tail_logits(dev):
    B, D, O, G, F, H = 32, 256, 1500, 32, 64, 1000
    torch.manual_seed(6)
    x = torch.randn(B, D, device=dev)
    head = torch.nn.Linear(D, H).to(dev)
    W = (torch.randn(O, F, device=dev) * 0.1).requires_grad_(True)
    bias = (torch.randn(O, device=dev) * 0.1).requires_grad_(True)
    idx = torch.randint(0, D, ((O + G - 1) // G, F), dtype=torch.int32, device=dev)
    out = ops.head_tail_logits(x, head, x, W, idx, bias, G)
    g_out = torch.randn(B, H + O, device=dev) * 0.1
    out.backward(g_out)
    xT = x.t().contiguous().cpu()
    Wc, bc, idxc, gt = W.detach().cpu(), bias.detach().cpu(), idx.cpu(), g_out[:, H:].cpu()
    assert out.dtype == torch.float32
    torch.testing.assert_close(out[:, :H].detach(), head(x).detach(), rtol=0, atol=0)
    torch.testing.assert_close(out[:, H:].detach().cpu(), oracle.ffi_forward(idxc, h(xT), h(Wc), bc, G),
                               **TOL32)
    torch.testing.assert_close(W.grad.cpu(), oracle.ffi_backward_weights(idxc, h(xT), h(gt), G),
                               **TOL32)
    assert torch.equal(bias.grad, g_out[:, H:].sum(0))


# ---- rewire of fp16 / fp32 layers (the reference rewires in the weights' dtype,
# shared_ffi/rewire.py:155,224-237): bit-exact against the oracle ----
def _w_np(t):
    t = t.detach().cpu()
    return t.numpy().copy() if t.dtype == torch.float32 else t.view(torch.int16).numpy().view(np.uint16).copy()


_WCODE = {torch.float16: oracle.F16, torch.float32: oracle.F32, torch.bfloat16: oracle.BF16}


@pytest.mark.parametrize("wdt", [torch.float16, torch.float32])
@pytest.mark.parametrize("init", ["zero", "random"])
@pytest.mark.parametrize("O,F,G,D", [(1000, 64, 32, 300), (1001, 13, 16, 50), (130, 256, 128, 900),
                                     (100000, 64, 32, 300)])
def test_rewire_f16_f32_layers_match_oracle(dev, wdt, init, O, F, G, D):
    torch.manual_seed(7)
    layer = GroupFixedFanIn(D, O, F, group_size=G, prune_mode="fraction", rewire_fraction=0.15,
                            init_mode=init, dtype=wdt)
    w, idx = _w_np(layer.weights), layer.group_locations.numpy().copy()
    seed = 0x5EED + O
    ref_w, ref_idx, ref_n, _, _ = oracle.rewire(
        w, idx, G, D, prune_mode=oracle.PRUNE_FRACTION, k=int(F * 0.15),
        init_mode=oracle.INIT_RANDOM if init == "random" else oracle.INIT_ZERO,
        bound=1.0 / F ** 0.5, seed=seed, w_dtype=_WCODE[wdt])
    layer = layer.to(dev)
    layer.rewire(seed=seed)
    torch.cuda.synchronize()
    assert layer.weights.dtype == wdt
    assert layer.pruned_total == ref_n
    assert np.array_equal(layer.group_locations.cpu().numpy(), ref_idx)
    assert np.array_equal(_w_np(layer.weights), ref_w)


@pytest.mark.parametrize("wdt,gdt,score", [(torch.float16, torch.float16, "mean"),
                                           (torch.float16, torch.float32, "max"),
                                           (torch.float32, torch.float32, "mean"),
                                           (torch.float32, None, "max")])
def test_app_rewire_f16_f32_layers_match_oracle(dev, wdt, gdt, score):
    from haste_amd.rewire import GroupFixedFanInReal
    O, F, G, D = 777, 128, 64, 768
    torch.manual_seed(8)
    layer = GroupFixedFanInReal(D, O, F, group_size=G, prune_mode="fraction",
                                rewire_fraction=0.15, init_mode="random", score_mode=score,
                                regrow_mode="unused", dtype=wdt,
                                fp32_grads=gdt == torch.float32 and wdt != torch.float32)
    w, idx = _w_np(layer.weights), layer.group_locations.numpy().copy()
    g_np = None
    if gdt is not None:
        gt = (torch.randn(O, F, generator=torch.Generator().manual_seed(9)) * 1e-2).to(gdt)
        g_np = _w_np(gt)
    Gc = (O + G - 1) // G
    k = int(Gc * F * 0.15)
    seed = 0xFACE + O
    ref_w, ref_idx, ref_n, _, _ = oracle.rewire_ex(
        w, idx, G, D, prune_mode=oracle.PRUNE_GLOBAL_FRACTION,
        score_mode=oracle.SCORE_MAX if score == "max" else oracle.SCORE_MEAN, grad=g_np, k=k,
        regrow_mode=oracle.REGROW_UNUSED, init_mode=oracle.INIT_RANDOM, bound=1.0 / F ** 0.5,
        seed=seed, w_dtype=_WCODE[wdt], grad_dtype=_WCODE[gdt] if gdt is not None else oracle.BF16)
    layer = layer.to(dev)
    if gdt is not None:
        layer.use_grad = True
        layer.weights.grad = gt.to(dev)
    layer.rewire(seed=seed)
    torch.cuda.synchronize()
    assert layer.pruned_total == ref_n == k
    assert np.array_equal(layer.group_locations.cpu().numpy(), ref_idx)
    assert np.array_equal(_w_np(layer.weights), ref_w)
