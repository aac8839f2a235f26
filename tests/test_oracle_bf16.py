"""Pins the oracle's fp32 -> bf16 round-to-nearest-even conversions to torch's
own `.to(torch.bfloat16)`, the conversion the reference's bf16 tensors go
through (`shared_ffi/rewire.py:109-112,235`; the RNE store of `_sgd_m_wd_sr`
with stochastic rounding off, `shared_ffi/sr_triton.py:165-166`).

Both oracle forms are checked: the C function `ho_f32_to_bf16_rne` (SGD without
SR, rewire's new weights) and the numpy `f32_to_bf16_bits` (test inputs)."""
import numpy as np
import pytest
import torch

from oracle import f32_to_bf16_bits, f32_to_bf16_rne


def torch_bf16_bits(x: np.ndarray) -> np.ndarray:
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(torch.bfloat16) \
        .view(torch.int16).numpy().view(np.uint16)


def _every_bf16_with_neighbours() -> np.ndarray:
    """Every bf16 pattern as fp32, and fp32 values at and around its half-ulp
    points: the patterns +0x7FFF, +0x8000 (the tie) and +0x8001 below and above."""
    hi = np.arange(1 << 16, dtype=np.uint32) << 16
    u = np.concatenate([hi, hi + 0x7FFF, hi + 0x8000, hi + 0x8001, hi + 1, hi + 0xFFFF,
                        hi - 0x8000, hi - 0x7FFF])
    return u.view(np.float32)


@pytest.mark.parametrize("conv", [f32_to_bf16_rne, f32_to_bf16_bits], ids=["c", "numpy"])
def test_bf16_rne_matches_torch_everywhere(conv):
    x = _every_bf16_with_neighbours()
    got, want = conv(x), torch_bf16_bits(x)
    nan = np.isnan(x)
    assert np.array_equal(got[~nan], want[~nan])
    # NaN stays NaN (torch gives the canonical quiet NaN, the oracle keeps the
    # sign and sets the quiet bit: both are NaN patterns)
    assert np.all((got[nan] & 0x7F80) == 0x7F80) and np.all((got[nan] & 0x7F) != 0)
    # sanity: the tie cases really were there, both ways
    ties = x.view(np.uint32) & 0xFFFF == 0x8000
    assert ties.sum() > 60000
    assert np.any(got[ties & ~nan] & 1 == 0)


@pytest.mark.parametrize("conv", [f32_to_bf16_rne, f32_to_bf16_bits], ids=["c", "numpy"])
def test_bf16_rne_matches_torch_random(conv):
    rng = np.random.default_rng(123)
    with np.errstate(over="ignore"):
        big = (rng.standard_normal(100_000) * 3e38).astype(np.float32)   # overflow to inf
    parts = [
        rng.integers(0, 1 << 32, 200_000, dtype=np.uint64).astype(np.uint32).view(np.float32),
        rng.standard_normal(100_000).astype(np.float32),
        (rng.standard_normal(100_000) * 1e-38).astype(np.float32),   # subnormals
        big,
    ]
    x = np.concatenate(parts)
    got, want = conv(x), torch_bf16_bits(x)
    ok = ~np.isnan(x)
    assert np.array_equal(got[ok], want[ok])


def test_bf16_rne_closed_forms():
    """Hand-derived cases: ties go to the even pattern, the largest finite bf16
    plus half an ulp overflows to inf, and the smallest subnormal tie rounds to 0."""
    cases = {
        0x3F808000: 0x3F80,   # 1 + 2^-8: tie, 0x3F80 is even
        0x3F818000: 0x3F82,   # 1 + 3*2^-8: tie, rounds up to the even 0x3F82
        0x3F807FFF: 0x3F80,
        0x3F808001: 0x3F81,
        0x7F7F8000: 0x7F80,   # max finite + half ulp -> +inf (tie to even 0x7F80)
        0x7F7F7FFF: 0x7F7F,
        0x00008000: 0x0000,   # half the smallest subnormal: tie to +0
        0x00018000: 0x0002,
        0x80008000: 0x8000,   # -0 side
        0xFF800000: 0xFF80,   # -inf
    }
    x = np.array(list(cases), dtype=np.uint32).view(np.float32)
    want = np.array(list(cases.values()), dtype=np.uint16)
    assert np.array_equal(f32_to_bf16_rne(x), want)
    assert np.array_equal(f32_to_bf16_bits(x), want)
    assert np.array_equal(torch_bf16_bits(x), want)
