"""GPU parity of the fused weight-gradient + SR-SGD kernel
(haste_ffi_bwd_weights_sgd) through the C ABI.

Bar: bit-exact.  The fused kernel must give exactly the bits of
haste_ffi_bwd_weights (fp32 dW, dbias) followed by haste_sgd_sr_step_multi on
{W, bias} (same seed, offsets from 0 per tensor), and that SGD result must be
bit-exact against the CPU oracle's SGD applied to the same fp32 gradients.
The fp32 gradients themselves match the oracle's fp32 contraction within
rtol 1e-4 / atol 1e-5 (summation order only).
"""
import numpy as np
import pytest
import torch

import oracle
from haste_amd import _C, _lib

pytestmark = pytest.mark.gpu

CASES = [
    # B, D, O, G, F, bias, momentum, do_sr
    (64, 768, 4096, 32, 32, True, False, True),
    (128, 768, 8193, 64, 128, True, False, True),    # config 1 shape, 1-label last group
    (100, 300, 1000, 16, 48, True, True, True),      # B % 8 != 0, F % 32 != 0, momentum
    (96, 512, 2050, 64, 64, False, False, True),     # no bias, partial last group
    (40, 768, 2100, 128, 128, True, True, False),    # G = 128, RNE instead of SR
    (130, 768, 3001, 128, 128, True, False, True),   # G = 128, SR: two prefetched epilogue passes
    (70, 768, 2000, 128, 96, True, True, True),      # G = 128, F < 128 slots, momentum
    (33, 200, 700, 128, 256, True, False, True),     # G = 128, F = 256 (several epilogue passes)
    (64, 4096, 3000, 32, 256, True, True, True),     # wide input, F = 256
    (37, 512, 999, 32, 240, True, False, True),      # 32-row chunks: a partial chunk, F < 256 slots
]


def bits(t):
    return t.detach().cpu().view(torch.int16).numpy().view(np.uint16).copy()


def setup(B, D, O, G, F, seed):
    g = torch.Generator().manual_seed(seed)
    Gc = (O + G - 1) // G
    x = torch.randn(B, D, generator=g).to(torch.bfloat16)
    W = ((torch.rand(O, F, generator=g) * 2 - 1) / F ** 0.5).to(torch.bfloat16)
    bias = (torch.randn(O, generator=g) * 0.1).to(torch.bfloat16)
    idx = torch.randint(0, D, (Gc, F), generator=g, dtype=torch.int32)
    lddy = (O + 7) // 8 * 8
    dY = torch.zeros(B, lddy, dtype=torch.bfloat16)
    dY[:, :O] = (torch.randn(B, O, generator=g) * 0.1).to(torch.bfloat16)
    mW = torch.randn(O, F, generator=g) * 0.01
    mb = torch.randn(O, generator=g) * 0.01
    return x, W, bias, idx, dY, lddy, mW, mb


@pytest.mark.parametrize("B,D,O,G,F,has_bias,use_mom,do_sr", CASES)
def test_fused_matches_separate_and_oracle(dev, B, D, O, G, F, has_bias, use_mom, do_sr):
    x, W, bias, idx, dY, lddy, mW, mb = setup(B, D, O, G, F, seed=O + F)
    lr, wd, mu, seed = 0.05, 1e-4, 0.9, 42 + G
    xT, ldx = _C.padded_transpose(x.to(dev))
    idx_d, dY_d = idx.to(dev), dY.to(dev)
    st = _C.stream_of(dY_d)

    # separate path: fp32 gradients, then the multi-tensor SGD kernel
    dW = torch.empty(O, F, dtype=torch.float32, device=dev)
    db = torch.empty(O, dtype=torch.float32, device=dev)
    _lib.call("haste_ffi_bwd_weights", idx_d.data_ptr(), xT.data_ptr(), ldx, dY_d.data_ptr(),
              lddy, dW.data_ptr(), _lib.DTYPE_F32, db.data_ptr(), _lib.DTYPE_F32, B, D, F, O, G,
              _lib.DTYPE_BF16, st)
    W1, b1, mW1, mb1 = W.to(dev), bias.to(dev), mW.to(dev), mb.to(dev)
    ts = [(W1, dW, mW1)] + ([(b1, db, mb1)] if has_bias else [])
    arr = (_lib.SgdTensor * len(ts))(*[_lib.SgdTensor(w.data_ptr(), g_.data_ptr(),
                                                      m.data_ptr() if use_mom else None,
                                                      w.numel(), 0) for w, g_, m in ts])
    _lib.call("haste_sgd_sr_step_multi", arr, len(ts), _lib.DTYPE_F32, lr, wd, mu, int(use_mom),
              int(do_sr), seed, st)

    # fused path (also storing the gradients)
    W2, b2, mW2, mb2 = W.to(dev), bias.to(dev), mW.to(dev), mb.to(dev)
    dW2 = torch.full((O, F), 7.0, dtype=torch.float32, device=dev)
    db2 = torch.full((O,), 7.0, dtype=torch.float32, device=dev)
    _lib.call("haste_ffi_bwd_weights_sgd", idx_d.data_ptr(), xT.data_ptr(), ldx, dY_d.data_ptr(),
              lddy, W2.data_ptr(), b2.data_ptr() if has_bias else None,
              mW2.data_ptr() if use_mom else None, mb2.data_ptr() if use_mom else None,
              dW2.data_ptr(), _lib.DTYPE_F32, db2.data_ptr(), _lib.DTYPE_F32, lr, wd, mu,
              int(use_mom), int(do_sr), seed, None, 0, B, D, F, O, G, _lib.DTYPE_BF16, st)
    torch.cuda.synchronize()

    assert torch.equal(dW2, dW), "fused kernel's fp32 dW differs from haste_ffi_bwd_weights"
    assert torch.equal(db2, db)
    assert np.array_equal(bits(W2), bits(W1)), "fused SGD differs from the separate path"
    if has_bias:
        assert np.array_equal(bits(b2), bits(b1))
    else:
        assert np.array_equal(bits(b2), bits(bias))
    if use_mom:
        assert torch.equal(mW2, mW1)
        if has_bias:
            assert torch.equal(mb2, mb1)

    # oracle: fp32 gradients within summation-order tolerance, SGD bit-exact on them
    ref_dw = oracle.ffi_backward_weights(idx, x.t().contiguous(), dY[:, :O], G)
    torch.testing.assert_close(dW.cpu(), ref_dw, rtol=1e-4, atol=1e-5)
    torch.testing.assert_close(db.cpu(), oracle.bias_grad(dY[:, :O]), rtol=1e-4, atol=1e-5)
    w_ref, m_ref = oracle.sgd_sr_step(bits(W).reshape(-1), dW.cpu().numpy().reshape(-1),
                                      mW.numpy().reshape(-1).copy() if use_mom else None, lr, wd,
                                      mu, use_mom, do_sr, seed)
    assert np.array_equal(bits(W2).reshape(-1), w_ref)
    if use_mom:
        assert np.array_equal(mW2.cpu().numpy().reshape(-1), m_ref)


@pytest.mark.parametrize("B,D,O,G,F", [(128, 768, 8193, 64, 128), (72, 500, 3001, 32, 64),
                                       (512, 768, 270001, 64, 128)])  # dY > 256 MB: streamed
def test_train_step_fused_equals_unfused(dev, B, D, O, G, F):
    """FFITrainStep.step (bwd-features partials, then the fused weight-gradient
    + SGD launch that also writes dX and hands the next step's bwd-features the
    transposed updated weights) gives dX, W and bias
    bit-identical to backward + sgd (which rebuild W^T every step), step by
    step; idx is drawn with replacement, so duplicated indices (hi/lo W^T rows)
    occur."""
    from haste_amd.step import FFITrainStep

    x, W, bias, idx, dY, lddy, _, _ = setup(B, D, O, G, F, seed=5)
    x_d, dY_d, idx_d = x.to(dev), dY.to(dev), idx.to(dev)
    Wa, ba, Wb, bb = W.to(dev), bias.to(dev), W.to(dev), bias.to(dev)
    sa = FFITrainStep(Wa, ba, idx_d, B, D, G, 0.05, 1e-4, seed=9)
    sb = FFITrainStep(Wb, bb, idx_d, B, D, G, 0.05, 1e-4, seed=9)
    for step in range(3):
        sa.step(x_d, dY_d, lddy)
        sb.forward(x_d)
        sb.backward(dY_d, lddy)
        sb.sgd()
        torch.cuda.synchronize()
        assert torch.equal(sa.dX, sb.dX), f"dX differs at step {step}"
        assert np.array_equal(bits(Wa), bits(Wb)), f"W differs at step {step}"
        assert np.array_equal(bits(ba), bits(bb))
    assert sa.seed == sb.seed == 12


DX_CASES = [
    # B, D, O, G, F, bias, momentum, lddy = O (the last dY row ends at label O)
    (64, 768, 4096, 32, 32, True, False, False),
    (128, 768, 8193, 64, 128, True, False, True),    # config 1 shape, 1-label last group
    (100, 300, 1000, 16, 48, True, True, False),     # G = 16, B and D not multiples of 32
    (96, 512, 2050, 64, 64, False, False, False),    # no bias
    (130, 768, 3001, 128, 128, True, True, True),    # G = 128, momentum
    (33, 200, 700, 128, 256, True, False, False),    # F = 256, one batch tile of 33 rows
    (72, 500, 3001, 32, 64, True, False, True),      # several feature ranges and slices
    (37, 512, 999, 32, 240, True, False, True),      # 32-row weight-gradient chunks, F < 256
]


@pytest.mark.parametrize("B,D,O,G,F,has_bias,use_mom,ys", DX_CASES)
def test_weight_update_finishes_dx(dev, B, D, O, G, F, has_bias, use_mom, ys):
    """haste_ffi_bwd_features_partials + haste_ffi_bwd_weights_sgd_dx (the
    final bwd-features pass as trailing workgroups of the weight update) give
    dX, W, bias and momentum bit-identical to haste_ffi_bwd_features_sr +
    haste_ffi_bwd_weights_sgd, and leave W^T of the updated weights in the
    workspace: a following bwd-features call with plan_ready = 2 matches one
    that rebuilds it."""
    x, W, bias, idx, dY, lddy, mW, mb = setup(B, D, O, G, F, seed=3 * O + F)
    if ys:
        dY, lddy = dY[:, :O].contiguous(), O
    lr, wd, mu, seed = 0.05, 1e-4, 0.9, 7 + G
    xT, ldx = _C.padded_transpose(x.to(dev))
    idx_d, dY_d = idx.to(dev), dY.to(dev)
    st = _C.stream_of(dY_d)
    code = _lib.DTYPE_BF16
    out = {}
    for mode in ("separate", "merged"):
        ws = _C.bwd_features_workspace(B, D, F, O, G, torch.bfloat16, dev)
        Wm, bm, mWm, mbm = W.to(dev), bias.to(dev), mW.to(dev), mb.to(dev)
        dX = torch.full((B, D), 3.0, dtype=torch.bfloat16, device=dev)
        bp = bm.data_ptr() if has_bias else None
        mwp, mbp = (mWm.data_ptr(), mbm.data_ptr()) if use_mom else (None, None)
        if mode == "separate":
            _lib.call("haste_ffi_bwd_features_sr", idx_d.data_ptr(), Wm.data_ptr(),
                      dY_d.data_ptr(), lddy, dX.data_ptr(), 123, ws.data_ptr(), ws.numel(), B, D,
                      F, O, G, code, 0, st)
            _lib.call("haste_ffi_bwd_weights_sgd", idx_d.data_ptr(), xT.data_ptr(), ldx,
                      dY_d.data_ptr(), lddy, Wm.data_ptr(), bp, mwp, mbp, None, _lib.DTYPE_F32,
                      None, _lib.DTYPE_F32, lr, wd, mu, int(use_mom), 1, seed, ws.data_ptr(),
                      ws.numel(), B, D, F, O, G, code, st)
        else:
            _lib.call("haste_ffi_bwd_features_partials", idx_d.data_ptr(), Wm.data_ptr(),
                      dY_d.data_ptr(), lddy, ws.data_ptr(), ws.numel(), B, D, F, O, G, code, 0,
                      st)
            _lib.call("haste_ffi_bwd_weights_sgd_dx", idx_d.data_ptr(), xT.data_ptr(), ldx,
                      dY_d.data_ptr(), lddy, Wm.data_ptr(), bp, mwp, mbp, lr, wd, mu,
                      int(use_mom), 1, seed, dX.data_ptr(), 123, ws.data_ptr(), ws.numel(), B, D,
                      F, O, G, code, st)
        # the next step's bwd-features on the workspace's W^T of the updated weights
        dX_next = torch.empty(B, D, dtype=torch.bfloat16, device=dev)
        _lib.call("haste_ffi_bwd_features_sr", idx_d.data_ptr(), Wm.data_ptr(), dY_d.data_ptr(),
                  lddy, dX_next.data_ptr(), 124, ws.data_ptr(), ws.numel(), B, D, F, O, G, code,
                  2, st)
        torch.cuda.synchronize()
        out[mode] = (bits(dX), bits(Wm), bits(bm), mWm.cpu(), mbm.cpu(), bits(dX_next))
    a, b = out["separate"], out["merged"]
    assert np.array_equal(b[0], a[0]), "dX of the merged launch differs"
    assert np.array_equal(b[1], a[1]) and np.array_equal(b[2], a[2]), "W / bias differ"
    assert torch.equal(b[3], a[3]) and torch.equal(b[4], a[4]), "momentum differs"
    assert np.array_equal(b[5], a[5]), "W^T refreshed by the merged launch differs"
    assert not np.array_equal(a[0], bits(torch.full((B, D), 3.0, dtype=torch.bfloat16)))
    # and the refreshed W^T is that of the updated weights: a rebuild agrees
    ws = _C.bwd_features_workspace(B, D, F, O, G, torch.bfloat16, dev)
    Wu = torch.from_numpy(a[1].view(np.int16)).view(torch.bfloat16).to(dev)
    dX_rb = torch.empty(B, D, dtype=torch.bfloat16, device=dev)
    _lib.call("haste_ffi_bwd_features_sr", idx_d.data_ptr(), Wu.data_ptr(), dY_d.data_ptr(), lddy,
              dX_rb.data_ptr(), 124, ws.data_ptr(), ws.numel(), B, D, F, O, G, code, 0, st)
    torch.cuda.synchronize()
    assert np.array_equal(bits(dX_rb), b[5])


@pytest.mark.parametrize("B,D,O,G,F,has_bias,use_mom,ys", DX_CASES)
def test_weight_gradient_finishes_dx(dev, B, D, O, G, F, has_bias, use_mom, ys):
    """haste_ffi_bwd_features_partials + haste_ffi_bwd_weights_dx (the drop-in
    backward: the final bwd-features pass as trailing workgroups of the weight
    gradient) give dX, dW and dbias bit-identical to haste_ffi_bwd_features_sr +
    haste_ffi_bwd_weights, for bf16 and fp32 gradient outputs."""
    x, W, bias, idx, dY, lddy, _, _ = setup(B, D, O, G, F, seed=5 * O + F)
    if ys:
        dY, lddy = dY[:, :O].contiguous(), O
    xT, ldx = _C.padded_transpose(x.to(dev))
    idx_d, dY_d, W_d = idx.to(dev), dY.to(dev), W.to(dev)
    st = _C.stream_of(dY_d)
    code = _lib.DTYPE_BF16
    for gdt, gcode in ((torch.bfloat16, _lib.DTYPE_BF16), (torch.float32, _lib.DTYPE_F32)):
        out = {}
        for mode in ("separate", "merged"):
            ws = _C.bwd_features_workspace(B, D, F, O, G, torch.bfloat16, dev)
            dX = torch.full((B, D), 3.0, dtype=torch.bfloat16, device=dev)
            dW = torch.full((O, F), 5.0, dtype=gdt, device=dev)
            db = torch.full((O,), 5.0, dtype=gdt, device=dev)
            dbp = db.data_ptr() if has_bias else None
            if mode == "separate":
                _lib.call("haste_ffi_bwd_features_sr", idx_d.data_ptr(), W_d.data_ptr(),
                          dY_d.data_ptr(), lddy, dX.data_ptr(), 123, ws.data_ptr(), ws.numel(),
                          B, D, F, O, G, code, 0, st)
                _lib.call("haste_ffi_bwd_weights", idx_d.data_ptr(), xT.data_ptr(), ldx,
                          dY_d.data_ptr(), lddy, dW.data_ptr(), gcode, dbp, gcode, B, D, F, O, G,
                          code, st)
            else:
                _lib.call("haste_ffi_bwd_features_partials", idx_d.data_ptr(), W_d.data_ptr(),
                          dY_d.data_ptr(), lddy, ws.data_ptr(), ws.numel(), B, D, F, O, G, code,
                          0, st)
                _lib.call("haste_ffi_bwd_weights_dx", idx_d.data_ptr(), xT.data_ptr(), ldx,
                          dY_d.data_ptr(), lddy, dW.data_ptr(), gcode, dbp, gcode,
                          dX.data_ptr(), 123, ws.data_ptr(), ws.numel(), B, D, F, O, G, code, st)
            torch.cuda.synchronize()
            out[mode] = (bits(dX), dW.cpu(), db.cpu())
        a, b = out["separate"], out["merged"]
        assert np.array_equal(b[0], a[0]), "dX of the merged launch differs"
        assert torch.equal(b[1], a[1]) and torch.equal(b[2], a[2]), "dW / dbias differ"
        assert not np.array_equal(a[0], bits(torch.full((B, D), 3.0, dtype=torch.bfloat16)))
