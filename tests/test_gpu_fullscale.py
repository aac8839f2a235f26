"""Value checks at the full sizes of BASELINE configs 1 to 4 (GPU).

Config 1 (B=512, D=768, O=131073, G=64, F=128) is checked whole against the
CPU oracle: forward, backward to features (fp32 and the SR'd bf16 dX),
backward to weights and bias, plus two size-independent properties -- the
feature gradient is bit-identical run to run, and the two adjoint pairings
<X, dX^T> and <W, dW> (both the trilinear sum over dY, X and W) agree.

Config 4 (B=1024, D=768, O=3,000,000, G=128, F=128) has 6.1 GB of logits, so
B * ldo > 2^31 and every 64-bit offset path is live; the oracle checks three
groups -- the first, the one holding label 2^31 / B, and the last (64
labels) -- with dY zero outside them, so the oracle's result on those groups
alone is exact for dX.  Logits, dX, dW, dbias and the fused SR-SGD bits of
their rows are compared; rows outside them get dW = 0 and the decay-only
update.  Configs 2 and 3 are checked the same way on three groups each,
through the training step's own backward (partials + fused update with dX).

Tolerances as in test_gpu_ffi.py: rtol 1e-2 / atol 1e-3 for bf16 outputs,
rtol 1e-4 / atol 1e-5 for fp32 ones, bit-exact for SR and SR-SGD.
"""
import numpy as np
import pytest
import torch

import oracle
from haste_amd import _C, _lib
from haste_amd.step import FFITrainStep

pytestmark = pytest.mark.gpu

TOL16 = dict(rtol=1e-2, atol=1e-3)
TOL32 = dict(rtol=1e-4, atol=1e-5)
LR, WD = 0.05, 1e-4


def bits(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def make(B, D, O, G, F, dev, seed):
    g = torch.Generator(device=dev).manual_seed(seed)
    Gc = (O + G - 1) // G
    x = torch.randn(B, D, generator=g, device=dev).to(torch.bfloat16)
    W = ((torch.rand(O, F, generator=g, device=dev) * 2 - 1) / F ** 0.5).to(torch.bfloat16)
    bias = (torch.randn(O, generator=g, device=dev) * 0.1).to(torch.bfloat16)
    idx = torch.randint(0, D, (Gc, F), generator=g, device=dev, dtype=torch.int32)
    return x, W, bias, idx


def bwd_features_fp32(idx, W, dY, lddy, B, D, F, O, G):
    ws = _C.bwd_features_workspace(B, D, F, O, G, torch.bfloat16, W.device)
    out = torch.empty(D, B, dtype=torch.float32, device=W.device)
    _lib.call("haste_ffi_bwd_features", idx.data_ptr(), W.data_ptr(), dY.data_ptr(), lddy,
              out.data_ptr(), ws.data_ptr(), ws.numel(), B, D, F, O, G, _lib.DTYPE_BF16, 0,
              _C.stream_of(W))
    return out


def bwd_weights_fp32(idx, xT, ldx, dY, lddy, B, D, F, O, G):
    dW = torch.empty(O, F, dtype=torch.float32, device=xT.device)
    db = torch.empty(O, dtype=torch.float32, device=xT.device)
    _lib.call("haste_ffi_bwd_weights", idx.data_ptr(), xT.data_ptr(), ldx, dY.data_ptr(), lddy,
              dW.data_ptr(), _lib.DTYPE_F32, db.data_ptr(), _lib.DTYPE_F32, B, D, F, O, G,
              _lib.DTYPE_BF16, _C.stream_of(xT))
    return dW, db


def test_config1_full_size(dev):
    B, D, O, G, F = 512, 768, 131073, 64, 128
    x, W, bias, idx = make(B, D, O, G, F, dev, seed=21)
    st = FFITrainStep(W, bias, idx, B, D, G, LR, WD, seed=42)
    logits = st.forward(x)
    xc, Wc, bc, idxc = x.cpu(), W.cpu(), bias.cpu(), idx.cpu()
    xT = xc.t().contiguous()
    ref = oracle.ffi_forward(idxc, xT, Wc, bc, G)
    torch.testing.assert_close(logits.float().cpu(), ref, **TOL16)

    gy = torch.Generator(device=dev).manual_seed(22)
    dY = torch.zeros(B, st.ldo, dtype=torch.bfloat16, device=dev)
    dY[:, :O] = (torch.randn(B, O, generator=gy, device=dev) * 0.1).to(torch.bfloat16)
    dYc = dY[:, :O].cpu()
    dxt = bwd_features_fp32(idx, W, dY, st.ldo, B, D, F, O, G)
    dxt2 = bwd_features_fp32(idx, W, dY, st.ldo, B, D, F, O, G)
    torch.cuda.synchronize()
    assert torch.equal(dxt.view(torch.int32), dxt2.view(torch.int32)), "not deterministic"
    torch.testing.assert_close(dxt.cpu(), oracle.ffi_backward_features(idxc, Wc, dYc, G, D), **TOL32)

    st.backward_features(dY, st.ldo)              # SR'd bf16 dX of the training step
    exp = oracle.sr_round_bf16(dxt.t().contiguous().cpu().numpy(), 123)
    assert np.array_equal(bits(st.dX), exp)

    dW, db = bwd_weights_fp32(idx, st.xT_buf, st.ldx, dY, st.ldo, B, D, F, O, G)
    torch.testing.assert_close(dW.cpu(), oracle.ffi_backward_weights(idxc, xT, dYc, G), **TOL32)
    torch.testing.assert_close(db.cpu(), oracle.bias_grad(dYc), **TOL32)

    # adjoint pairings: <X, dX^T> and <W, dW> are the same trilinear sum
    lhs = (xc.double().t() * dxt.cpu().double()).sum().item()
    rhs = (Wc.double() * dW.cpu().double()).sum().item()
    assert abs(lhs - rhs) <= 1e-5 * (abs(lhs) + abs(rhs)) + 1e-3, (lhs, rhs)


def test_config4_full_size_spot_groups(dev):
    B, D, O, G, F = 1024, 768, 3_000_000, 128, 128
    Gc = (O + G - 1) // G
    x, W, bias, idx = make(B, D, O, G, F, dev, seed=31)
    groups = [0, (2 ** 31 // B) // G, Gc - 1]
    w0 = W.clone()
    b0 = bias.clone()
    st = FFITrainStep(W, bias, idx, B, D, G, LR, WD, seed=7)
    assert B * st.ldo > 2 ** 31
    logits = st.forward(x)
    xT = x.cpu().t().contiguous()
    idxc = idx.cpu()
    spans = [(g * G, min(O, (g + 1) * G)) for g in groups]
    assert spans[-1][1] - spans[-1][0] == 64

    # the three groups as a small problem of their own (the last one partial)
    idx_s = idxc[groups]
    W_s = torch.cat([w0[a:b].cpu() for a, b in spans])
    b_s = torch.cat([b0[a:b].cpu() for a, b in spans])
    got = torch.cat([logits[:, a:b].cpu() for a, b in spans], dim=1)
    torch.testing.assert_close(got.float(), oracle.ffi_forward(idx_s, xT, W_s, b_s, G), **TOL16)

    gy = torch.Generator(device=dev).manual_seed(32)
    dY = torch.zeros(B, st.ldo, dtype=torch.bfloat16, device=dev)
    for a, b in spans:
        dY[:, a:b] = (torch.randn(B, b - a, generator=gy, device=dev) * 0.1).to(torch.bfloat16)
    dY_s = torch.cat([dY[:, a:b].cpu() for a, b in spans], dim=1)

    dxt = bwd_features_fp32(idx, W, dY, st.ldo, B, D, F, O, G)
    torch.testing.assert_close(dxt.cpu(), oracle.ffi_backward_features(idx_s, W_s, dY_s, G, D), **TOL32)
    st.backward_features(dY, st.ldo)
    exp = oracle.sr_round_bf16(dxt.t().contiguous().cpu().numpy(), 123)
    assert np.array_equal(bits(st.dX), exp)

    dW, db = bwd_weights_fp32(idx, st.xT_buf, st.ldx, dY, st.ldo, B, D, F, O, G)
    ref_w = oracle.ffi_backward_weights(idx_s, xT, dY_s, G)
    torch.testing.assert_close(torch.cat([dW[a:b].cpu() for a, b in spans]), ref_w, **TOL32)
    torch.testing.assert_close(torch.cat([db[a:b].cpu() for a, b in spans]), oracle.bias_grad(dY_s), **TOL32)
    others = torch.tensor([200, 5000, 1_000_000, 2_999_800], device=dev)  # outside the groups
    assert not dW[others].any() and not db[others].any()

    # fused weight gradient + SR-SGD (seed 7, offsets l*F + j and l from 0)
    st.backward_weights_sgd(dY, st.ldo)
    torch.cuda.synchronize()
    for (a, b) in spans + [(int(r), int(r) + 1) for r in others.tolist()]:
        ref, _ = oracle.sgd_sr_step(bits(w0[a:b]).reshape(-1), dW[a:b].cpu().numpy().reshape(-1),
                                    None, LR, WD, 0.0, False, True, 7, offset0=a * F)
        assert np.array_equal(bits(W[a:b]).reshape(-1), ref), (a, b)
        ref_b, _ = oracle.sgd_sr_step(bits(b0[a:b]), db[a:b].cpu().numpy(), None, LR, WD, 0.0,
                                      False, True, 7, offset0=a)
        assert np.array_equal(bits(bias[a:b]), ref_b), (a, b)


@pytest.mark.parametrize("cfg", [
    # config 2: 670K labels, F = 64; dY (686 MB) beyond the last-level cache, so
    # bwd-features runs its LDS-ring build
    dict(B=512, D=768, O=670_091, G=64, F=64, relu=False, seed=41),
    # config 3: D = 4096 (many feature ranges, 64-column batch tiles), F = 256,
    # post-ReLU features (about half zeros)
    dict(B=256, D=4096, O=500_000, G=32, F=256, relu=True, seed=51),
])
def test_configs_2_3_full_size_spot_groups(dev, cfg):
    """BASELINE configs 2 and 3 at full size: the training step (forward, bwd-features
    partials finished by the fused update's launch, fused SR-SGD) checked on the
    first, a middle and the last group against the oracle, with dY zero outside
    them (so dX of those groups alone is exact); other rows get dW = 0 and the
    decay-only update."""
    B, D, O, G, F = cfg["B"], cfg["D"], cfg["O"], cfg["G"], cfg["F"]
    Gc = (O + G - 1) // G
    x, W, bias, idx = make(B, D, O, G, F, dev, seed=cfg["seed"])
    if cfg["relu"]:
        x = x.clamp_min(0)
    groups = [0, Gc // 2, Gc - 1]
    spans = [(g * G, min(O, (g + 1) * G)) for g in groups]
    w0, b0 = W.clone(), bias.clone()
    st = FFITrainStep(W, bias, idx, B, D, G, LR, WD, seed=9)
    xT = x.cpu().t().contiguous()
    idx_s = idx.cpu()[groups]
    W_s = torch.cat([w0[a:b].cpu() for a, b in spans])
    b_s = torch.cat([b0[a:b].cpu() for a, b in spans])

    gy = torch.Generator(device=dev).manual_seed(cfg["seed"] + 1)
    dY = torch.zeros(B, st.ldo, dtype=torch.bfloat16, device=dev)
    for a, b in spans:
        dY[:, a:b] = (torch.randn(B, b - a, generator=gy, device=dev) * 0.1).to(torch.bfloat16)
    dY_s = torch.cat([dY[:, a:b].cpu() for a, b in spans], dim=1)
    # the reference values of dW / dbias and the fp32 feature gradient, before the step
    st.forward(x)
    logits = st.logits
    got = torch.cat([logits[:, a:b].cpu() for a, b in spans], dim=1)
    torch.testing.assert_close(got.float(), oracle.ffi_forward(idx_s, xT, W_s, b_s, G), **TOL16)
    dW, db = bwd_weights_fp32(idx, st.xT_buf, st.ldx, dY, st.ldo, B, D, F, O, G)
    ref_w = oracle.ffi_backward_weights(idx_s, xT, dY_s, G)
    torch.testing.assert_close(torch.cat([dW[a:b].cpu() for a, b in spans]), ref_w, **TOL32)
    torch.testing.assert_close(torch.cat([db[a:b].cpu() for a, b in spans]), oracle.bias_grad(dY_s),
                               **TOL32)
    dxt = bwd_features_fp32(idx, W, dY, st.ldo, B, D, F, O, G)
    torch.testing.assert_close(dxt.cpu(), oracle.ffi_backward_features(idx_s, W_s, dY_s, G, D),
                               **TOL32)

    # the training step's backward: partials, then the fused update writes dX too
    st.backward_features(dY, st.ldo, defer_dx=True)
    st.backward_weights_sgd(dY, st.ldo)
    torch.cuda.synchronize()
    exp = oracle.sr_round_bf16(dxt.t().contiguous().cpu().numpy(), 123)
    assert np.array_equal(bits(st.dX), exp)
    others = [G + 1, Gc // 3 * G + 5, O - G - 1]  # rows outside the groups
    assert all(not dW[r].any() and float(db[r]) == 0.0 for r in others)
    for (a, b) in spans + [(r, r + 1) for r in others]:
        ref, _ = oracle.sgd_sr_step(bits(w0[a:b]).reshape(-1), dW[a:b].cpu().numpy().reshape(-1),
                                    None, LR, WD, 0.0, False, True, 9, offset0=a * F)
        assert np.array_equal(bits(W[a:b]).reshape(-1), ref), (a, b)
        ref_b, _ = oracle.sgd_sr_step(bits(b0[a:b]), db[a:b].cpu().numpy(), None, LR, WD, 0.0,
                                      False, True, 9, offset0=a)
        assert np.array_equal(bits(bias[a:b]), ref_b), (a, b)


@pytest.mark.parametrize("cfg", [2, 4])
def test_rewire_full_size(dev, cfg):
    """Rewire at the full sizes that configs 2 and 4 run it every 1000 steps
    (shared_ffi/rewire.py:143-239 with the build's contract): prune the
    int(F * 0.15) smallest mean-|W| slots of every group (k = 9 at config 2,
    19 at config 4), regrow indices unused in the group, zero init.  Scores,
    indices, weights and the pruned count bit-exact against the oracle."""
    O, F, G = {2: (670091, 64, 64), 4: (3_000_000, 128, 128)}[cfg]
    D, k = 768, int(F * 0.15)
    Gc = (O + G - 1) // G
    g = torch.Generator(device=dev).manual_seed(100 + cfg)
    Wd = ((torch.rand(O, F, generator=g, device=dev) * 2 - 1) / F ** 0.5).to(torch.bfloat16)
    idxd = torch.randint(0, D, (Gc, F), generator=g, device=dev, dtype=torch.int32)
    w, idx = bits(Wd), idxd.cpu().numpy()
    seed = 0x5EED0000 + cfg
    ref_w, ref_idx, ref_n, ref_s, _ = oracle.rewire(
        w, idx, G, D, prune_mode=oracle.PRUNE_FRACTION, k=k, regrow_mode=oracle.REGROW_UNUSED,
        init_mode=oracle.INIT_ZERO, bound=1.0 / F ** 0.5, seed=seed)
    scores = torch.empty(Gc, F, device=dev)
    cnt = torch.zeros(1, dtype=torch.int32, device=dev)
    _lib.call("haste_rewire", Wd.data_ptr(), _lib.DTYPE_BF16, idxd.data_ptr(), scores.data_ptr(),
              cnt.data_ptr(), O, F, G, D, _lib.PRUNE_FRACTION, 0.0, k, _lib.REGROW_UNUSED,
              _lib.INIT_ZERO, 1.0 / F ** 0.5, seed, _C.stream_of(Wd))
    torch.cuda.synchronize()
    assert int(cnt.item()) == ref_n
    assert np.array_equal(scores.cpu().numpy().view(np.uint32), ref_s.view(np.uint32))
    assert np.array_equal(idxd.cpu().numpy(), ref_idx)
    assert np.array_equal(bits(Wd), ref_w)
    # every group pruned exactly k slots
    assert ref_n == Gc * k
