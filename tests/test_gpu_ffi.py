"""GPU parity of the FFI kernels (forward, backward to features, backward to
weights + bias) against the CPU oracle, through the C ABI.

Tolerance: bf16/f16 outputs match the fp32-accumulate
oracle within rtol 1e-2 / atol 1e-3.  fp32 outputs (dX^T, dW in fp32 mode) are
checked at rtol 1e-4 / atol 1e-5 (summation order differs only).
"""
import numpy as np
import pytest
import torch

import oracle
from bwdf_cases import RING_CASES, STAGED_CASES, kernel_config
from haste_amd import _C, _lib

pytestmark = pytest.mark.gpu

TOL16 = dict(rtol=1e-2, atol=1e-3)
TOL32 = dict(rtol=1e-4, atol=1e-5)


def make_case(B, D, O, G, F, seed=0, dtype=torch.bfloat16, idx_mode="perm"):
    g = torch.Generator().manual_seed(seed)
    Gc = (O + G - 1) // G
    x = torch.randn(B, D, generator=g).to(dtype)
    bound = 1.0 / F ** 0.5
    W = ((torch.rand(O, F, generator=g) * 2 - 1) * bound).to(dtype)
    bias = (torch.randn(O, generator=g) * 0.1).to(dtype)
    if idx_mode == "perm" and F <= D:
        idx = torch.stack([torch.randperm(D, generator=g)[:F] for _ in range(Gc)]).to(torch.int32)
    else:
        idx = torch.randint(0, D, (Gc, F), generator=g, dtype=torch.int32)
    if idx_mode in ("shared", "same"):
        # consecutive groups share most features (a random walk replacing 30 % of
        # a row's slots per group), or all of them: the staged build's window
        # plan keeps a shared feature on one wave across a window of groups
        for i in range(1, Gc):
            idx[i] = idx[i - 1]
            if idx_mode == "shared":
                m = torch.rand(F, generator=g) < 0.3
                idx[i, m] = torch.randint(0, D, (int(m.sum()),), generator=g, dtype=torch.int32)
    if idx_mode == "dups":
        idx[0, :] = 5                                  # one index for the whole group
        if Gc > 1:
            idx[1, : F // 2] = idx[1, F // 2: 2 * (F // 2)]  # every index twice
        if Gc > 2:
            idx[2, 3:12] = 7                            # a run of 9 equal indices
    dY = (torch.randn(B, O, generator=g) * 0.1).to(dtype)
    return x, W, bias, idx, dY


def gpu_forward(x, W, bias, idx, G, dev):
    B, D = x.shape
    O, F = W.shape
    xT = x.t().contiguous().to(dev)
    return _C.ffi_forward_cuda(idx.to(dev), xT, W.to(dev), None if bias is None else bias.to(dev),
                               B, D, F, O, G)


CASES = [
    # B, D, O, G, F, idx_mode
    (64, 768, 4096, 32, 32, "perm"),
    (64, 768, 4133, 32, 32, "perm"),      # partial last group, O % 8 != 0
    (100, 300, 1000, 16, 16, "random"),   # B % 8 != 0, G = 16
    (7, 50, 130, 16, 48, "random"),       # F % 32 != 0, tiny batch
    (128, 768, 8193, 64, 128, "perm"),    # config 1 shape at reduced O, 1-label last group
    (96, 512, 2000, 64, 64, "dups"),      # duplicate indices, runs of equal indices
    (64, 4096, 3000, 32, 256, "random"),  # wide input, F = 256 (config 3 family)
    (40, 768, 2100, 128, 128, "random"),  # G = 128 (config 4 family)
    (33, 200, 700, 128, 256, "dups"),
    (200, 768, 3000, 128, 128, "dups"),   # G = 128, batch tiles of 128 (8 waves), 4 ranges
    (150, 200, 1500, 128, 256, "random"), # G = 128, 8 waves, one range: rounds past the ring
    (256, 768, 5000, 64, 64, "dups"),     # 2-tile ring (config 2 family); duplicates overflow it
    (160, 4096, 1000, 32, 256, "random"), # 2-tile ring, 15 ranges (config 3 family), 8 waves
    (1, 64, 64, 64, 64, "random"),
    (5, 20, 5, 16, 32, "random"),         # O < G (one partial group), D < F (forced duplicates)
]


@pytest.mark.parametrize("B,D,O,G,F,mode", CASES)
def test_forward(dev, B, D, O, G, F, mode):
    x, W, bias, idx, _ = make_case(B, D, O, G, F, idx_mode=mode)
    out = gpu_forward(x, W, bias, idx, G, dev)
    assert out.shape == (B, O)
    ref = oracle.ffi_forward(idx, x.t().contiguous(), W, bias, G)
    torch.testing.assert_close(out.float().cpu(), ref, **TOL16)
    out_nb = gpu_forward(x, W, None, idx, G, dev)
    torch.testing.assert_close(out_nb.float().cpu(), oracle.ffi_forward(idx, x.t().contiguous(), W, None, G), **TOL16)


@pytest.mark.parametrize("O,G", [(1027, 32), (1034, 32), (4133, 32), (2000, 64)])
def test_forward_bias_alignment_and_last_group(dev, O, G):
    """The bias is loaded four labels at a time where it is 8-byte aligned and
    label by label where it is not, and in the last group (3, 10 and 5 labels at
    O = 1027, 1034, 4133): every way gives the same logits, bit for bit."""
    B, D, F = 48, 256, 64
    x, W, bias, idx, _ = make_case(B, D, O, G, F, idx_mode="random", seed=5)
    out = gpu_forward(x, W, bias, idx, G, dev)
    torch.testing.assert_close(out.float().cpu(), oracle.ffi_forward(idx, x.t().contiguous(), W, bias, G),
                               **TOL16)
    big = torch.zeros(O + 1, dtype=bias.dtype, device=dev)
    big[1:] = bias.to(dev)
    xT = x.t().contiguous().to(dev)
    out_u = _C.ffi_forward_cuda(idx.to(dev), xT, W.to(dev), big[1:], B, D, F, O, G)
    assert torch.equal(out_u.cpu(), out.cpu())


def test_forward_f16(dev):
    x, W, bias, idx, _ = make_case(64, 768, 4133, 32, 64, dtype=torch.float16)
    out = gpu_forward(x, W, bias, idx, 32, dev)
    torch.testing.assert_close(out.float().cpu(), oracle.ffi_forward(idx, x.t().contiguous(), W, bias, 32), **TOL16)


@pytest.mark.parametrize("B,D,O,G,F,mode", CASES)
def test_backward_features(dev, B, D, O, G, F, mode):
    x, W, bias, idx, dY = make_case(B, D, O, G, F, idx_mode=mode, seed=1)
    xT = x.t().contiguous().to(dev)
    dXT = _C.ffi_backward_features_cuda(xT, W.to(dev), idx.to(dev), dY.to(dev), B, D, F, O, G)
    ref = oracle.ffi_backward_features(idx, W, dY, G, D)
    torch.testing.assert_close(dXT.cpu(), ref, **TOL32)


# every (G, BT, RT) case under the LDS-ring build (1) and, where it exists
# (G = 32, 64), the direct build (2); every staged (G, BT) case and the ring
# cases with G >= 32 under the staged build (3)
# Index rows shared between consecutive groups, under the staged build: one or
# several feature ranges, duplicates within a row (D < F), F = 256, and more
# ranges than the window plan pins (every group then laid out on its own).
WINDOW_CASES = [(96, 300, 20000, 64, 128, "shared", 3), (64, 768, 20000, 128, 256, "shared", 3),
                (64, 1500, 20000, 32, 64, "shared", 3), (64, 9000, 20000, 64, 128, "shared", 3),
                (64, 200, 6000, 64, 64, "same", 3), (48, 100, 9000, 128, 128, "shared", 3)]
BUILD_CASES = ([c + (1,) for c in RING_CASES] + [c + (2,) for c in RING_CASES if c[3] in (32, 64)]
               + [c + (3,) for c in STAGED_CASES] + [c + (3,) for c in RING_CASES if c[3] >= 32]
               + WINDOW_CASES)


@pytest.mark.parametrize("B,D,O,G,F,mode,build", BUILD_CASES)
def test_backward_features_every_build(dev, B, D, O, G, F, mode, build):
    """One shape per (G, batch tile, ring tiles) build of the main kernel (the
    coverage of RING_CASES is checked on the CPU in test_abi.py), under each
    main-kernel build."""
    x, W, bias, idx, dY = make_case(B, D, O, G, F, idx_mode=mode, seed=11)
    prev = _lib.lib().haste_ffi_bwd_features_set_build(build)
    try:
        BT, RT, _, _ = kernel_config(_lib.lib(), B, D, O, G, F)
        dXT = _C.ffi_backward_features_cuda(x.t().contiguous().to(dev), W.to(dev), idx.to(dev),
                                            dY.to(dev), B, D, F, O, G)
        torch.cuda.synchronize()
    finally:
        _lib.lib().haste_ffi_bwd_features_set_build(prev)
    ref = oracle.ffi_backward_features(idx, W, dY, G, D)
    torch.testing.assert_close(dXT.cpu(), ref, **TOL32,
                               msg=lambda m: f"G={G} BT={BT} RT={RT} build={build}: {m}")


@pytest.mark.parametrize("B,D,O,G,F,mode", CASES[:6])
def test_backward_features_sr_fused(dev, oracle_mod, B, D, O, G, F, mode):
    """Fused SR output == oracle SR (seed 123, offset b*D+d) of the GPU's own fp32
    dX, bit for bit; and within tolerance of the fp32 oracle."""
    x, W, bias, idx, dY = make_case(B, D, O, G, F, idx_mode=mode, seed=2)
    Wd, idxd = W.to(dev), idx.to(dev)
    dYd, lddy = _C.rows_aligned(dY.to(dev))
    dXT = _C.ffi_backward_features_cuda(x.t().contiguous().to(dev), Wd, idxd, dYd, B, D, F, O, G)
    ws = _C.bwd_features_workspace(B, D, F, O, G, torch.bfloat16, dev)
    dX = torch.empty(B, D, dtype=torch.bfloat16, device=dev)
    _lib.call("haste_ffi_bwd_features_sr", idxd.data_ptr(), Wd.data_ptr(), dYd.data_ptr(),
              lddy, dX.data_ptr(), 123, ws.data_ptr(), ws.numel(), B, D, F, O, G,
              _lib.DTYPE_BF16, 0, _C.stream_of(Wd))
    torch.cuda.synchronize()
    exp = oracle_mod.sr_round_bf16(dXT.t().contiguous().cpu().numpy(), seed=123)
    got = dX.cpu().view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, exp)
    ref = oracle.ffi_backward_features(idx, W, dY, G, D).t()
    torch.testing.assert_close(dX.float().cpu(), ref, **TOL16)


@pytest.mark.parametrize("B,D,O,G,F,mode", CASES)
def test_backward_weights_and_bias(dev, B, D, O, G, F, mode):
    x, W, bias, idx, dY = make_case(B, D, O, G, F, idx_mode=mode, seed=3)
    xT, ldx = _C.padded_transpose(x.to(dev))
    dYd, lddy = _C.rows_aligned(dY.to(dev))
    idxd = idx.to(dev)
    ref_w = oracle.ffi_backward_weights(idx, x.t().contiguous(), dY, G)
    ref_b = oracle.bias_grad(dY)
    for wcode, tol in ((_lib.DTYPE_F32, TOL32), (_lib.DTYPE_BF16, TOL16)):
        dW = torch.empty(O, F, dtype=torch.float32 if wcode == _lib.DTYPE_F32 else torch.bfloat16, device=dev)
        db = torch.empty(O, dtype=dW.dtype, device=dev)
        _lib.call("haste_ffi_bwd_weights", idxd.data_ptr(), xT.data_ptr(), ldx, dYd.data_ptr(),
                  lddy, dW.data_ptr(), wcode, db.data_ptr(), wcode, B, D, F, O, G,
                  _lib.DTYPE_BF16, _C.stream_of(dYd))
        torch.testing.assert_close(dW.float().cpu(), ref_w, **tol)
        torch.testing.assert_close(db.float().cpu(), ref_b, **tol)


def test_backward_weights_reference_api(dev):
    x, W, bias, idx, dY = make_case(64, 768, 4133, 32, 32, seed=4)
    dW = _C.ffi_backward_weights_cuda(x.t().contiguous().to(dev), W.to(dev), idx.to(dev),
                                      dY.to(dev), 64, 768, 32, 4133, 32)
    assert dW.dtype == torch.bfloat16 and dW.shape == (4133, 32)
    torch.testing.assert_close(dW.float().cpu(), oracle.ffi_backward_weights(idx, x.t().contiguous(), dY, 32), **TOL16)


def test_backward_f16(dev):
    x, W, bias, idx, dY = make_case(64, 768, 2048, 64, 64, dtype=torch.float16, seed=5)
    dXT = _C.ffi_backward_features_cuda(x.t().contiguous().to(dev), W.to(dev), idx.to(dev),
                                        dY.to(dev), 64, 768, 64, 2048, 64)
    torch.testing.assert_close(dXT.cpu(), oracle.ffi_backward_features(idx, W, dY, 64, 768), **TOL32)
    dW = _C.ffi_backward_weights_cuda(x.t().contiguous().to(dev), W.to(dev), idx.to(dev),
                                      dY.to(dev), 64, 768, 64, 2048, 64)
    torch.testing.assert_close(dW.float().cpu(), oracle.ffi_backward_weights(idx, x.t().contiguous(), dY, 64), **TOL16)


def test_backward_features_deterministic(dev):
    """Same inputs -> bitwise identical fp32 output (no float atomics on global memory)."""
    x, W, bias, idx, dY = make_case(256, 768, 20000, 64, 128, seed=6, idx_mode="dups")
    args = (x.t().contiguous().to(dev), W.to(dev), idx.to(dev), dY.to(dev), 256, 768, 128, 20000, 64)
    a = _C.ffi_backward_features_cuda(*args)
    b = _C.ffi_backward_features_cuda(*args)
    assert torch.equal(a.view(torch.int32), b.view(torch.int32))


def test_out_of_range_indices_are_clamped(dev):
    x, W, bias, idx, dY = make_case(16, 64, 128, 32, 32, seed=7, idx_mode="random")
    bad = idx.clone()
    bad[0, 0] = 10**6
    bad[1, 1] = -5
    clamped = bad.clamp(0, 63)
    out = gpu_forward(x, W, bias, bad, 32, dev)
    torch.testing.assert_close(out.float().cpu(), oracle.ffi_forward(clamped, x.t().contiguous(), W, bias, 32), **TOL16)


@pytest.mark.parametrize("B,O,G,F", [(70, 1001, 64, 128), (64, 4133, 32, 32), (65, 700, 128, 64)])
def test_forward_leaves_columns_past_O_untouched(dev, B, O, G, F):
    """The logits may sit inside a wider row (e.g. a head/tail concat at a column
    offset): columns >= O of an ld-padded output, and rows past B, keep their
    contents."""
    D = 256
    x, W, bias, idx, _ = make_case(B, D, O, G, F, idx_mode="random")
    ldo = (O + 63) // 64 * 64 + 64
    out = torch.full((B + 3, ldo), 7.0, dtype=torch.bfloat16, device=dev)
    xT, ldx = _C.padded_transpose(x.to(dev))
    idx_d, W_d, b_d = idx.to(dev), W.to(dev), bias.to(dev)  # alive until the kernel ran
    _lib.call("haste_ffi_forward", idx_d.data_ptr(), xT.data_ptr(), ldx, W_d.data_ptr(),
              b_d.data_ptr(), out.data_ptr(), ldo, B, D, F, O, G, _lib.DTYPE_BF16,
              _C.stream_of(out))
    torch.cuda.synchronize()
    ref = oracle.ffi_forward(idx, x.t().contiguous(), W, bias, G)
    torch.testing.assert_close(out[:B, :O].float().cpu(), ref, **TOL16)
    assert bool((out[:B, O:] == 7.0).all()), "columns >= O were written"
    assert bool((out[B:] == 7.0).all()), "rows >= B were written"


@pytest.mark.parametrize("B", [37, 64, 100, 130])
def test_forward_g16_rows_written_once(dev, B):
    """G = 16: every wave stores only the rows it staged (an instruction spans 32
    rows, a wave stages 16); each call rewrites a NaN-filled output the same."""
    D, O, G, F = 200, 513, 16, 64
    x, W, bias, idx, _ = make_case(B, D, O, G, F)
    ref = oracle.ffi_forward(idx, x.t().contiguous(), W, bias, G)
    ldx, ldo = (B + 7) // 8 * 8, (O + 7) // 8 * 8
    xT = torch.zeros(D, ldx, dtype=torch.bfloat16)
    xT[:, :B] = x.t()
    xT, idx_d, W_d, bias_d = xT.to(dev), idx.to(dev), W.to(dev), bias.to(dev)
    for _ in range(3):
        out = torch.full((B, ldo), float("nan"), dtype=torch.bfloat16, device=dev)
        _lib.call("haste_ffi_forward", idx_d.data_ptr(), xT.data_ptr(), ldx, W_d.data_ptr(),
                  bias_d.data_ptr(), out.data_ptr(), ldo, B, D, F, O, G, _lib.DTYPE_BF16,
                  torch.cuda.current_stream().cuda_stream)
        torch.testing.assert_close(out[:, :O].float().cpu(), ref, **TOL16)


def test_backward_weights_streaming_dY(dev):
    """dY above 256 MB (the MI355X last-level cache) is read with non-temporal
    loads, a separate instantiation of the weight-gradient kernel: dW and dbias
    of the first, a middle and the last (partial) group match the oracle."""
    B, D, O, G, F = 512, 768, 270001, 64, 128
    g = torch.Generator(device=dev).manual_seed(12)
    x = torch.randn(B, D, generator=g, device=dev).to(torch.bfloat16)
    Gc = (O + G - 1) // G
    idx = torch.randint(0, D, (Gc, F), generator=g, device=dev, dtype=torch.int32)
    lddy = (O + 7) // 8 * 8
    assert B * lddy * 2 > 256 << 20
    dY = torch.zeros(B, lddy, dtype=torch.bfloat16, device=dev)
    dY[:, :O] = torch.randn(B, O, generator=g, device=dev).mul_(0.1).to(torch.bfloat16)
    xT, ldx = _C.padded_transpose(x)
    dW = torch.empty(O, F, dtype=torch.float32, device=dev)
    db = torch.empty(O, dtype=torch.float32, device=dev)
    _lib.call("haste_ffi_bwd_weights", idx.data_ptr(), xT.data_ptr(), ldx, dY.data_ptr(), lddy,
              dW.data_ptr(), _lib.DTYPE_F32, db.data_ptr(), _lib.DTYPE_F32, B, D, F, O, G,
              _lib.DTYPE_BF16, _C.stream_of(dY))
    torch.cuda.synchronize()
    x_t = x.t().contiguous().cpu()
    for grp in (0, Gc // 2, Gc - 1):
        l0, l1 = grp * G, min(O, (grp + 1) * G)
        dy = dY[:, l0:l1].cpu()
        ref_w = oracle.ffi_backward_weights(idx[grp:grp + 1].cpu(), x_t, dy, G)
        torch.testing.assert_close(dW[l0:l1].cpu(), ref_w, **TOL32)
        torch.testing.assert_close(db[l0:l1].cpu(), oracle.bias_grad(dy), **TOL32)


@pytest.mark.parametrize("build", [1, 2, 3])  # bwd-features main kernel: ring, direct, staged
@pytest.mark.parametrize("B,D,O,G,F,pad,col0", [
    (37, 300, 2003, 64, 64, 0, 0),    # [B, O] contiguous, O odd
    (64, 768, 4133, 32, 32, 4, 0),    # odd row stride past O
    (7, 50, 130, 16, 48, 5, 0),       # tiny batch
    (100, 768, 2100, 128, 128, 0, 0),
    (65, 200, 1001, 16, 32, 1, 0),    # B = 65: the last row sits alone in a 64-row chunk
    (1, 64, 67, 64, 64, 0, 0),        # one row, last group of 3 labels
    (130, 300, 5000, 64, 64, 3, 5),   # the view starts 5 columns into a row of 5008
    (70, 300, 3001, 32, 32, 0, 1001), # the tail columns of a head/tail concat
])
def test_backward_reads_rows_at_any_stride(dev, oracle_mod, B, D, O, G, F, pad, col0, build):
    """The backward kernels read grad-of-logits rows in place whatever their
    alignment (rows start on 2-byte boundaries) and read nothing past label O
    of the last row: the tensor here ends there, with NaN in the rest of each
    row.  Results are bit-identical to the same data in 16-byte aligned rows,
    and match the oracle, under each bwd-features main-kernel build."""
    prev = _lib.lib().haste_ffi_bwd_features_set_build(build)
    try:
        _any_stride_case(dev, B, D, O, G, F, pad, col0)
    finally:
        _lib.lib().haste_ffi_bwd_features_set_build(prev)


def _any_stride_case(dev, B, D, O, G, F, pad, col0):
    x, W, bias, idx, dY = make_case(B, D, O, G, F, idx_mode="random", seed=13)
    lddy = col0 + O + pad
    buf = torch.full(((B - 1) * lddy + col0 + O,), float("nan"), dtype=torch.bfloat16, device=dev)
    dYo = buf.as_strided((B, O), (lddy, 1), col0)
    dYo.copy_(dY.to(dev))
    dYa, ldda = _C.rows_aligned(dY.to(dev))            # aligned copy, stride % 8 == 0
    assert (lddy % 8 != 0 or col0 % 8 != 0) and ldda % 8 == 0
    idx_d, W_d = idx.to(dev), W.to(dev)
    xT, ldx = _C.padded_transpose(x.to(dev))
    st = _C.stream_of(W_d)

    def bwdf(y, ld):
        ws = _C.bwd_features_workspace(B, D, F, O, G, torch.bfloat16, dev)
        out = torch.empty(D, B, dtype=torch.float32, device=dev)
        _lib.call("haste_ffi_bwd_features", idx_d.data_ptr(), W_d.data_ptr(), y.data_ptr(), ld,
                  out.data_ptr(), ws.data_ptr(), ws.numel(), B, D, F, O, G, _lib.DTYPE_BF16, 0,
                  st)
        dx = torch.empty(B, D, dtype=torch.bfloat16, device=dev)
        _lib.call("haste_ffi_bwd_features_sr", idx_d.data_ptr(), W_d.data_ptr(), y.data_ptr(),
                  ld, dx.data_ptr(), 123, ws.data_ptr(), ws.numel(), B, D, F, O, G,
                  _lib.DTYPE_BF16, 1, st)
        return out, dx

    def bwdw(y, ld):
        dW = torch.empty(O, F, dtype=torch.float32, device=dev)
        db = torch.empty(O, dtype=torch.float32, device=dev)
        _lib.call("haste_ffi_bwd_weights", idx_d.data_ptr(), xT.data_ptr(), ldx, y.data_ptr(),
                  ld, dW.data_ptr(), _lib.DTYPE_F32, db.data_ptr(), _lib.DTYPE_F32, B, D, F, O, G,
                  _lib.DTYPE_BF16, st)
        W2, b2 = W.to(dev), bias.to(dev)
        _lib.call("haste_ffi_bwd_weights_sgd", idx_d.data_ptr(), xT.data_ptr(), ldx,
                  y.data_ptr(), ld, W2.data_ptr(), b2.data_ptr(), None, None, None,
                  _lib.DTYPE_F32, None, _lib.DTYPE_F32, 0.05, 1e-4, 0.0, 0, 1, 42, None, 0, B, D,
                  F, O, G, _lib.DTYPE_BF16, st)
        return dW, db, W2, b2

    f_o, sr_o = bwdf(dYo, lddy)
    f_a, sr_a = bwdf(dYa, ldda)
    w_o = bwdw(dYo, lddy)
    w_a = bwdw(dYa, ldda)
    torch.cuda.synchronize()
    assert torch.equal(f_o.view(torch.int32), f_a.view(torch.int32))
    assert torch.equal(sr_o.view(torch.int16), sr_a.view(torch.int16))
    for a, b in zip(w_o, w_a):
        assert torch.equal(a.view(torch.int32 if a.dtype == torch.float32 else torch.int16),
                           b.view(torch.int32 if b.dtype == torch.float32 else torch.int16))
    torch.testing.assert_close(f_o.cpu(), oracle.ffi_backward_features(idx, W, dY, G, D), **TOL32)
    torch.testing.assert_close(w_o[0].cpu(), oracle.ffi_backward_weights(idx, x.t().contiguous(), dY, G), **TOL32)
    torch.testing.assert_close(w_o[1].cpu(), oracle.bias_grad(dY), **TOL32)
