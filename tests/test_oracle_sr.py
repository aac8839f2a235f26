"""Pins the oracle's stochastic rounding (shared_ffi/sr_triton.py:9-16) by
properties that the definition of unbiased stochastic rounding fixes."""
import numpy as np
import pytest

from oracle import bf16_bits_to_f32


def _sr(oracle_mod, x, r):
    return int(oracle_mod.lib().ho_sr_bf16(np.float32(x), int(r)))


def test_exact_values_unchanged(oracle_mod):
    rng = np.random.default_rng(0)
    vals = (rng.standard_normal(200) * 10).astype(np.float32)
    vals = bf16_bits_to_f32((vals.view(np.uint32) >> 16).astype(np.uint16))  # exactly bf16
    for v in vals:
        for r in (0, 1, 0x7FFF, 0xFFFF, 0xDEADFFFF):
            assert _sr(oracle_mod, v, r) == int(np.float32(v).view(np.uint32) >> 16)


@pytest.mark.parametrize("x", [1.0 + 2**-9, -3.14159, 1e-30, 65504.3, 2.0 - 2**-20, -7.77e20])
def test_unbiased_over_all_random_words(oracle_mod, x):
    """Averaging SR(x) over all 2^16 random low words reproduces x exactly:
    SR rounds to one of the two bf16 neighbours of x with probability
    proportional to the distance to the other one."""
    x = np.float32(x)
    lib = oracle_mod.lib()
    outs = np.array([lib.ho_sr_bf16(x, r) for r in range(1 << 16)], dtype=np.uint16)
    trunc = np.uint16(x.view(np.uint32) >> 16)
    assert set(np.unique(outs).tolist()) <= {int(trunc), int(trunc) + 1}
    vals = bf16_bits_to_f32(outs).astype(np.float64)
    assert vals.mean() == np.float64(x)


def test_round_up_iff_carry(oracle_mod):
    """The result is the upper neighbour exactly when low16(x) + r16 carries."""
    rng = np.random.default_rng(1)
    xs = rng.standard_normal(300).astype(np.float32)
    rs = rng.integers(0, 2**32, 300, dtype=np.uint64)
    for x, r in zip(xs, rs):
        u = int(np.float32(x).view(np.uint32))
        trunc = u >> 16
        up = (u & 0xFFFF) + (int(r) & 0xFFFF) >= 0x10000
        assert _sr(oracle_mod, x, r) == trunc + int(up)


def test_sign_symmetry(oracle_mod):
    rng = np.random.default_rng(2)
    for x, r in zip(rng.standard_normal(200).astype(np.float32), rng.integers(0, 2**32, 200)):
        assert _sr(oracle_mod, -x, r) == _sr(oracle_mod, x, r) ^ 0x8000


def test_specials(oracle_mod):
    assert _sr(oracle_mod, np.inf, 0xFFFF) == 0x7F80
    assert _sr(oracle_mod, -np.inf, 0xFFFF) == 0xFF80
    assert _sr(oracle_mod, 0.0, 0xFFFF) == 0x0000
    n = _sr(oracle_mod, np.float32("nan"), 0xFFFF)
    assert (n & 0x7F80) == 0x7F80 and (n & 0x7F) != 0
    # the largest finite bf16-truncated values round up to inf when they carry
    big = np.float32(3.4e38)
    assert _sr(oracle_mod, big, 0xFFFF) in (0x7F7F, 0x7F80)


def test_array_matches_scalar(oracle_mod):
    rng = np.random.default_rng(3)
    x = rng.standard_normal(4096).astype(np.float32)
    out = oracle_mod.sr_round_bf16(x, seed=123, offset0=7)
    r = oracle_mod.randint(123, 7, 4096)
    lib = oracle_mod.lib()
    ref = np.array([lib.ho_sr_bf16(a, int(b)) for a, b in zip(x, r)], dtype=np.uint16)
    assert np.array_equal(out, ref)
