"""Pins the oracle's fused SGD step (shared_ffi/sr_triton.py:109-168):

* torch.optim.SGD's update on inputs where every operation is exact, which fixes
  the terms, their signs and their order independently of the oracle;
* hand-derived closed forms;
* an exact-rational evaluation of the FMA contraction on general inputs, which
  fixes the rounding (where fused and unfused evaluation differ)."""
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


# ---- independent pins of the update's terms, signs and order ----------------
# torch.optim.SGD (dampening 0, no Nesterov) performs d = g + wd*p;
# buf = mu*buf + d; p = p - lr*buf.  On dyadic inputs with short numerators
# every product and sum is exact in fp32 (so fusing or not cannot matter) and
# every result is exact in bf16 (so RNE and SR are the identity): the oracle
# must then equal torch's fp32 update bit for bit.  A swapped sign, a weight
# decay applied to the wrong operand or momentum applied in the wrong order
# changes the value.

def _exact_inputs(n, seed):
    rng = np.random.default_rng(seed)
    w = rng.integers(-15, 16, n).astype(np.float32) / 16      # a / 16
    g = rng.integers(-31, 32, n).astype(np.float32) / 64      # b / 64
    m = rng.integers(-31, 32, n).astype(np.float32) / 32      # c / 32
    return w, g, m


@pytest.mark.parametrize("use_mom", [False, True])
@pytest.mark.parametrize("do_sr", [False, True])
def test_sgd_equals_torch_optim_sgd_on_exact_inputs(oracle_mod, use_mom, do_sr):
    import torch

    lr, wd, mu = 0.5, 0.25, 0.5
    w, g, m = _exact_inputs(4096, seed=11 + use_mom)
    p = torch.nn.Parameter(torch.from_numpy(w.copy()))
    opt = torch.optim.SGD([p], lr=lr, momentum=mu if use_mom else 0.0, dampening=0.0,
                          weight_decay=wd)
    p.grad = torch.from_numpy(g.copy())
    if use_mom:
        opt.state[p]["momentum_buffer"] = torch.from_numpy(m.copy())
    opt.step()
    exp = p.detach().numpy()
    w_bits = f32_to_bf16_bits(w)
    assert np.array_equal(bf16_bits_to_f32(w_bits), w)  # inputs exact in bf16
    got, gm = oracle_mod.sgd_sr_step(w_bits, g, m.copy() if use_mom else None, lr, wd, mu,
                                     use_mom, do_sr, seed=42)
    assert np.array_equal(bf16_bits_to_f32(got), exp)
    if use_mom:
        assert np.array_equal(gm, opt.state[p]["momentum_buffer"].numpy())


def test_sgd_closed_forms(oracle_mod):
    """Hand-derived single-element updates (all values exact in bf16)."""
    def one(w, g, m, lr, wd, mu, use_mom):
        wb = f32_to_bf16_bits(np.array([w], np.float32))
        out, mo = oracle_mod.sgd_sr_step(wb, np.array([g], np.float32),
                                         np.array([m], np.float32) if use_mom else None,
                                         lr, wd, mu, use_mom, False, seed=0)
        return float(bf16_bits_to_f32(out)[0]), (None if mo is None else float(mo[0]))

    # w' = w - lr*(g + wd*w) = 1 - 0.5*(0.5 + 0.25) = 0.625
    assert one(1.0, 0.5, 0.0, 0.5, 0.25, 0.0, False) == (0.625, None)
    # m' = mu*m + (g + wd*w) = 0.25 + 0.75 = 1; w' = 1 - 0.5*1 = 0.5
    assert one(1.0, 0.5, 0.5, 0.5, 0.25, 0.5, True) == (0.5, 1.0)
    # the decay term scales w, not g: w = 2, g = 0 -> w' = 2 - 0.5*0.5 = 1.75
    assert one(2.0, 0.0, 0.0, 0.5, 0.25, 0.0, False) == (1.75, None)
    # a negative gradient raises the weight: w' = 0 - 0.25*(-1) = 0.25
    assert one(0.0, -1.0, 0.0, 0.25, 0.0, 0.0, False) == (0.25, None)
    # momentum scales the old buffer, not the new gradient: m = 1, g = 1, mu = 0.25
    # -> m' = 1.25, w' = 0 - 1 * 1.25
    assert one(0.0, 1.0, 1.0, 1.0, 0.0, 0.25, True) == (-1.25, 1.25)


def test_f32_to_f16_matches_numpy():
    """The oracle's fp32 -> fp16 conversion (used for fp16 weights) is numpy's
    round-to-nearest-even conversion: on every bf16 value (the inputs it gets),
    on random fp32 values, and around the subnormal, overflow and halfway cases."""
    import oracle
    bf = np.arange(65536, dtype=np.uint32)
    xs = [(bf << 16).view(np.float32)]
    rng = np.random.default_rng(5)
    xs.append(rng.standard_normal(100000).astype(np.float32) * np.float32(2.0) ** rng.integers(-30, 18, 100000).astype(np.float32))
    edges = np.array([65504, 65519.99, 65520, 65536, 2.0 ** -14, 2.0 ** -24, 2.0 ** -25,
                      1.5 * 2.0 ** -25, 3 * 2.0 ** -26, 1 + 2.0 ** -11, 1 + 3 * 2.0 ** -11],
                     dtype=np.float32)
    xs.append(np.concatenate([edges, -edges]))
    for x in xs:
        finite = ~np.isnan(x)
        got = oracle.f32_to_f16_rne(x[finite])
        with np.errstate(over="ignore"):
            ref = x[finite].astype(np.float16).view(np.uint16)
        assert np.array_equal(got, ref)


@pytest.mark.parametrize("gdt", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("use_mom,do_sr", [(False, True), (True, True), (False, False)])
def test_sgd_f16_weights_is_bf16_step_then_fp16_store(gdt, use_mom, do_sr):
    """On fp16 weights the step is the bf16-weight step on the same fp32 values
    (fp16 -> fp32 is exact), followed by the store's fp16 conversion (numpy's):
    checked where the weights are bf16-representable, so both oracles take the
    same inputs; with lr = 0 and no SR the weights are fp16(RNE_bf16(w))."""
    import oracle
    rng = np.random.default_rng(11)
    n = 4099
    w16 = (rng.random(n, dtype=np.float32) - 0.5).astype(np.float16)
    wbf = f32_to_bf16_bits(w16.astype(np.float32))      # bf16 of the fp16 value
    w16 = bf16_bits_to_f32(wbf).astype(np.float16)       # fp16 values that are bf16 exact
    g32 = (rng.standard_normal(n) * 0.05).astype(np.float32)
    g = {"f32": g32, "bf16": f32_to_bf16_bits(g32), "f16": g32.astype(np.float16)}[gdt]
    m = (rng.standard_normal(n) * 0.01).astype(np.float32)
    got_w, got_m = oracle.sgd_sr_step_f16w(w16, g, m if use_mom else None, 0.05, 1e-4, 0.9,
                                           use_mom, do_sr, 2**33 + 7)
    ref_b, ref_m = oracle.sgd_sr_step(wbf, g, m if use_mom else None, 0.05, 1e-4, 0.9, use_mom,
                                      do_sr, 2**33 + 7)
    assert np.array_equal(got_w.view(np.uint16), bf16_bits_to_f32(ref_b).astype(np.float16).view(np.uint16))
    if use_mom:
        assert np.array_equal(got_m.view(np.uint32), ref_m.view(np.uint32))
    # lr = 0, no SR: fp16 of the bf16 rounding of an arbitrary fp16 weight
    w_any = (rng.standard_normal(n) * 3).astype(np.float16)
    out, _ = oracle.sgd_sr_step_f16w(w_any, g, None, 0.0, 0.0, 0.0, False, False, 1)
    expect = bf16_bits_to_f32(f32_to_bf16_bits(w_any.astype(np.float32))).astype(np.float16)
    assert np.array_equal(out.view(np.uint16), expect.view(np.uint16))
