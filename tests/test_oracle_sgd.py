"""Pins the oracle's fused SGD step (shared_ffi/sr_triton.py:109-168) by an
exact-rational evaluation of the FMA contract on small arrays."""
from fractions import Fraction

import numpy as np
import pytest

from oracle import bf16_bits_to_f32, f32_to_bf16_bits


def f32_round(q: Fraction) -> np.float32:
    """Correctly rounded (nearest-even) float32 of an exact rational."""
    c = np.float32(float(q))
    best = None
    for cand in (np.nextafter(c, np.float32(-np.inf)), c, np.nextafter(c, np.float32(np.inf))):
        if not np.isfinite(cand):
            continue
        err = abs(Fraction(float(cand)) - q)
        key = (err, int(cand.view(np.uint32)) & 1)
        if best is None or key < best[0]:
            best = (key, cand)
    return best[1]


def fma_exact(a, b, c) -> np.float32:
    return f32_round(Fraction(float(a)) * Fraction(float(b)) + Fraction(float(c)))


def sgd_reference(w_bits, g, m, lr, wd, mu, use_mom, do_sr, seed, oracle_mod):
    lr, wd, mu = np.float32(lr), np.float32(wd), np.float32(mu)
    r = oracle_mod.randint(seed, 0, len(w_bits))
    out = np.empty_like(w_bits)
    m_out = None if m is None else m.copy()
    for i in range(len(w_bits)):
        w = bf16_bits_to_f32(w_bits[i])
        gi = fma_exact(wd, w, np.float32(g[i]))
        upd = gi
        if use_mom:
            upd = fma_exact(mu, m[i], gi)
            m_out[i] = upd
        nw = fma_exact(-lr, upd, w)
        if do_sr:
            u = int(np.float32(nw).view(np.uint32))
            out[i] = ((u + (int(r[i]) & 0xFFFF)) & 0xFFFFFFFF) >> 16
        else:
            out[i] = f32_to_bf16_bits(np.array([nw], dtype=np.float32))[0]
    return out, m_out


def _inputs(n, seed=0):
    rng = np.random.default_rng(seed)
    w = f32_to_bf16_bits((rng.uniform(-0.2, 0.2, n)).astype(np.float32))
    g = (rng.standard_normal(n) * 0.05).astype(np.float32)
    m = (rng.standard_normal(n) * 0.01).astype(np.float32)
    return w, g, m


@pytest.mark.parametrize("use_mom,do_sr", [(False, True), (True, True), (False, False), (True, False)])
def test_sgd_matches_exact_fma_chain(oracle_mod, use_mom, do_sr):
    w, g, m = _inputs(600)
    got, gm = oracle_mod.sgd_sr_step(w, g, m if use_mom else None, 0.05, 1e-4, 0.9, use_mom,
                                     do_sr, seed=42)
    ref, rm = sgd_reference(w, g, m if use_mom else None, 0.05, 1e-4, 0.9, use_mom, do_sr, 42,
                            oracle_mod)
    assert np.array_equal(got, ref)
    if use_mom:
        assert np.array_equal(gm.view(np.uint32), rm.view(np.uint32))


def test_fma_contract_is_observable(oracle_mod):
    """Rounding after each product (no FMA) changes the fp32 update on some
    inputs, so the exact-chain test above discriminates the contract."""
    w, g, _ = _inputs(800, seed=5)
    lr, wd = np.float32(0.05), np.float32(1e-4)
    wf = bf16_bits_to_f32(w)
    unfused = (wf - (lr * (g + wd * wf).astype(np.float32)).astype(np.float32)).astype(np.float32)
    diffs = sum(fma_exact(-lr, fma_exact(wd, a, b), a) != u for a, b, u in zip(wf, g, unfused))
    assert diffs > 0


def test_lr_zero_keeps_weights(oracle_mod):
    w, g, _ = _inputs(1000, seed=2)
    got, _ = oracle_mod.sgd_sr_step(w, g, None, 0.0, 0.0, 0.0, False, True, seed=7)
    assert np.array_equal(got, w)


def test_grad_dtypes_equivalent(oracle_mod):
    """bf16 gradients (as uint16 bits) give the same result as their exact fp32 values."""
    w, g, _ = _inputs(1000, seed=3)
    gb = f32_to_bf16_bits(g)
    a, _ = oracle_mod.sgd_sr_step(w, gb, None, 0.05, 1e-4, 0.0, False, True, seed=9)
    b, _ = oracle_mod.sgd_sr_step(w, bf16_bits_to_f32(gb), None, 0.05, 1e-4, 0.0, False, True, seed=9)
    assert np.array_equal(a, b)


def test_seed_changes_rounding(oracle_mod):
    w, g, _ = _inputs(5000, seed=4)
    a, _ = oracle_mod.sgd_sr_step(w, g, None, 0.05, 1e-4, 0.0, False, True, seed=42)
    b, _ = oracle_mod.sgd_sr_step(w, g, None, 0.05, 1e-4, 0.0, False, True, seed=43)
    assert (a != b).sum() > 100
    # every output is one of the two bf16 neighbours of the RNE result
    c, _ = oracle_mod.sgd_sr_step(w, g, None, 0.05, 1e-4, 0.0, False, False, seed=0)
    assert np.all(np.abs(a.astype(np.int32) - c.astype(np.int32)) <= 1)
