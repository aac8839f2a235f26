"""Pins the oracle's fp16 / fp8 outputs of stochastic rounding and its fp8
weight update (shared_ffi/sr_triton.py:18-25,43-46,146,167-168): fp8 decoding
of every code against torch's float8 types, in-range encodings against torch's
round-to-nearest-even conversions, saturation by closed forms, the 20-bit
rounding to e4m3 by exact unbiasedness over all 2^20 random words, and the
bf16-then-store outputs on bf16-exact inputs (which stochastic rounding leaves
unchanged) against torch's conversions.  NaN and overflow results of the
reference (Triton's float8 conversions on NVIDIA GPUs) are not pinned."""
import numpy as np
import pytest
import torch

import oracle

FMTS = {oracle.F8E4M3: torch.float8_e4m3fn, oracle.F8E5M2: torch.float8_e5m2}
MAXF = {oracle.F8E4M3: 448.0, oracle.F8E5M2: 57344.0}
MAXC = {oracle.F8E4M3: 0x7E, oracle.F8E5M2: 0x7B}


def torch_decode(codes, tdt):
    return torch.from_numpy(codes).view(tdt).float().numpy()


def torch_encode(x, tdt):
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(tdt).view(torch.uint8).numpy()


@pytest.mark.parametrize("fmt", list(FMTS))
def test_decode_every_code(fmt):
    codes = np.arange(256, dtype=np.uint8)
    got, want = oracle.f8_to_f32(codes, fmt), torch_decode(codes, FMTS[fmt])
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))
    assert oracle.f8_to_f32(np.array([MAXC[fmt]], np.uint8), fmt)[0] == MAXF[fmt]


@pytest.mark.parametrize("fmt", list(FMTS))
def test_encode_in_range_matches_torch(fmt):
    """Every finite value, the midpoints between neighbours (ties) and the
    fp32 values either side of them, and random values in range."""
    codes = np.arange(256, dtype=np.uint8)
    v = oracle.f8_to_f32(codes, fmt)
    v = np.unique(v[np.isfinite(v)]).astype(np.float32)
    mid = ((v[:-1].astype(np.float64) + v[1:]) / 2).astype(np.float32)
    near = np.concatenate([np.nextafter(mid, np.float32(-np.inf)), mid,
                           np.nextafter(mid, np.float32(np.inf))])
    rng = np.random.default_rng(fmt)
    rnd = (rng.standard_normal(200_000) * rng.choice([1e-3, 1e-1, 1, 30, 300], 200_000)).astype(np.float32)
    x = np.concatenate([v, near, rnd, (rnd * 1e-3).astype(np.float32)])
    x = x[np.abs(x) <= MAXF[fmt]]
    assert np.array_equal(oracle.f32_to_f8(x, fmt), torch_encode(x, FMTS[fmt]))


def test_encode_closed_forms():
    E, F = oracle.F8E4M3, oracle.F8E5M2
    cases = [
        (E, 448.0, 0x7E), (E, 464.0, 0x7E), (E, 1e6, 0x7E), (E, -1e6, 0xFE), (E, np.inf, 0x7E),
        (E, -np.inf, 0xFE), (E, 2.0 ** -9, 0x01), (E, 2.0 ** -10, 0x00), (E, 1.5 * 2.0 ** -10, 0x01),
        (E, 1.0, 0x38), (E, -0.0, 0x80),
        (F, 57344.0, 0x7B), (F, 1e9, 0x7B), (F, np.inf, 0x7B), (F, -np.inf, 0xFB),
        (F, 2.0 ** -16, 0x01), (F, 2.0 ** -17, 0x00), (F, 1.0, 0x3C),
    ]
    for fmt, x, code in cases:
        assert oracle.f32_to_f8(np.array([x], np.float32), fmt)[0] == code, (fmt, x)
    for fmt in (E, F):
        got = oracle.f32_to_f8(np.array([np.nan, -np.nan], np.float32), fmt)
        assert np.isnan(oracle.f8_to_f32(got, fmt)).all()


@pytest.mark.parametrize("x", [1.0, 1.0 + 2 ** -5, -3.3, 0.0172, 200.5, -2 ** -6 * 1.37, 447.9])
def test_sr_e4m3_unbiased_over_every_word(x):
    """stochastic_rounding_to_fp8 in e4m3's normal range: over all 2^20
    random words the mean of the rounded values is exactly the fp32 input, and
    every result is one of its two e4m3 neighbours (only the input itself when
    it is an e4m3 value)."""
    xf = np.float32(x)
    words = np.arange(1 << 20, dtype=np.uint32)
    got = oracle.f8_to_f32(oracle.sr_e4m3_words(float(xf), words), oracle.F8E4M3).astype(np.float64)
    assert got.mean() == float(xf)
    lo = float(torch.tensor([float(xf)]).to(torch.float8_e4m3fn).float())
    vals = set(np.unique(got).tolist())
    assert len(vals) <= 2 and all(abs(v - float(xf)) < 2 ** -3 * max(abs(float(xf)), 2 ** -6) for v in vals)
    if lo == float(xf):
        assert vals == {float(xf)}


@pytest.mark.parametrize("out_dtype,tdt", [(oracle.F16, torch.float16),
                                           (oracle.F8E5M2, torch.float8_e5m2),
                                           (oracle.BF16, torch.bfloat16)])
def test_sr_outputs_on_bf16_exact_inputs(out_dtype, tdt):
    """Inputs exactly representable in bf16 are left unchanged by the bf16
    rounding, so the output is torch's conversion of the input."""
    rng = np.random.default_rng(7)
    x = torch.from_numpy(rng.standard_normal(50_000).astype(np.float32) * 10).to(torch.bfloat16)
    x = x[x.float().abs() <= 57344].float().numpy()
    got = oracle.sr_round(x, out_dtype, seed=5)
    want = torch.from_numpy(x).to(tdt)
    want = want.view(torch.uint8 if out_dtype == oracle.F8E5M2 else torch.int16).numpy()
    assert np.array_equal(got.view(want.dtype), want)


@pytest.mark.parametrize("fmt", list(FMTS))
def test_sgd_f8w_closed_forms(fmt):
    tdt = FMTS[fmt]
    codes = np.arange(256, dtype=np.uint8)
    v = oracle.f8_to_f32(codes, fmt)
    ok = np.isfinite(v)
    codes = codes[ok]
    g = np.zeros(codes.size, np.float32)
    # lr = 0: every weight unchanged (fp8 values are exact in bf16), with and without SR
    for sr in (False, True):
        out, _ = oracle.sgd_sr_step_f8w(codes, fmt, g, None, 0.0, 0.0, 0.0, False, sr, seed=3)
        assert np.array_equal(out, codes)
    # round to nearest: w - lr*g with exactly representable products, against torch
    w = v[ok]
    gg = np.full(w.size, 0.75, np.float32)
    out, _ = oracle.sgd_sr_step_f8w(codes, fmt, gg, None, 0.5, 0.0, 0.0, False, False, seed=3)
    ref = torch.from_numpy(w - np.float32(0.5) * gg).to(torch.bfloat16).float()
    ref = ref.clamp(-MAXF[fmt], MAXF[fmt]).to(tdt).view(torch.uint8).numpy()
    assert np.array_equal(out, ref)
