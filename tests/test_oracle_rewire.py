"""Pins the oracle's rewire contract (restating shared_ffi/rewire.py:143-239)."""
import math

import numpy as np
import pytest
import torch

import oracle
from oracle import bf16_bits_to_f32, f32_to_bf16_bits


def _layer(O, F, G, D, seed=0):
    rng = np.random.default_rng(seed)
    b = 1 / math.sqrt(F)
    w = f32_to_bf16_bits(rng.uniform(-b, b, (O, F)).astype(np.float32))
    idx = rng.integers(0, D, ((O + G - 1) // G, F)).astype(np.int32)
    return w, idx


def _scores_brute(w, G):
    O, F = w.shape
    Gc = (O + G - 1) // G
    wf = bf16_bits_to_f32(w)
    s = np.zeros((Gc, F), dtype=np.float32)
    for g in range(Gc):
        rows = range(g * G, min(O, g * G + G))
        for j in range(F):
            acc = np.float32(0)
            for l in rows:
                acc = np.float32(acc + np.float32(abs(wf[l, j])))
            s[g, j] = np.float32(acc / np.float32(len(rows)))
    return s


def test_scores_sequential_mean():
    w, _ = _layer(37, 8, 16, 50)
    assert np.array_equal(oracle.rewire_scores(w, 16), _scores_brute(w, 16))


@pytest.mark.parametrize("k", [1, 3, 8])
def test_fraction_prunes_k_smallest(k):
    O, F, G, D = 70, 8, 16, 40
    w, idx = _layer(O, F, G, D, seed=1)
    w[3, :] = 0  # ties: group 0 rows with equal |W| contributions
    w2, idx2, n, scores, mask = oracle.rewire(w, idx, G, D, prune_mode=oracle.PRUNE_FRACTION, k=k,
                                              seed=11)
    Gc = idx.shape[0]
    assert n == Gc * k
    for g in range(Gc):
        order = sorted(range(F), key=lambda j: (scores[g, j], j))
        assert set(np.nonzero(mask[g])[0].tolist()) == set(order[:k])


def test_threshold_mode():
    O, F, G, D = 64, 16, 32, 100
    w, idx = _layer(O, F, G, D, seed=2)
    thr = float(np.median(oracle.rewire_scores(w, G)))
    w2, idx2, n, scores, mask = oracle.rewire(w, idx, G, D, prune_mode=oracle.PRUNE_THRESHOLD,
                                              threshold=thr, seed=3)
    assert np.array_equal(mask, scores < np.float32(thr))
    assert n == int(mask.sum())


def test_zero_init_and_untouched_elsewhere():
    O, F, G, D = 50, 8, 16, 30
    w, idx = _layer(O, F, G, D, seed=4)
    w2, idx2, n, _, mask = oracle.rewire(w, idx, G, D, prune_mode=oracle.PRUNE_FRACTION, k=2,
                                         init_mode=oracle.INIT_ZERO, seed=5)
    rowmask = mask[np.arange(O) // G]
    assert np.all(w2[rowmask] == 0)
    assert np.array_equal(w2[~rowmask], w[~rowmask])
    assert np.array_equal(idx2[~mask], idx[~mask])
    assert idx2.min() >= 0 and idx2.max() < D


def test_random_regrow_indices_are_philox_draws():
    O, F, G, D = 40, 8, 16, 768
    w, idx = _layer(O, F, G, D, seed=6)
    seed = 987654321012
    _, idx2, _, _, mask = oracle.rewire(w, idx, G, D, prune_mode=oracle.PRUNE_FRACTION, k=3,
                                        seed=seed)
    for g, j in zip(*np.nonzero(mask)):
        blk = oracle.philox4x32([g * F + j, 1, 0, 0], [seed & 0xFFFFFFFF, seed >> 32], 10)
        assert idx2[g, j] == (int(blk[0]) * D) >> 32


def test_unused_regrow_avoids_group_indices():
    O, F, G, D = 64 * 6, 48, 64, 64  # small D: collisions are frequent
    w, idx = _layer(O, F, G, D, seed=7)
    _, idx2, _, _, mask = oracle.rewire(w, idx, G, D, prune_mode=oracle.PRUNE_FRACTION, k=10,
                                        regrow_mode=oracle.REGROW_UNUSED, seed=8)
    for g in range(idx.shape[0]):
        kept = set(idx[g][~mask[g]].tolist())
        new = idx2[g][mask[g]].tolist()
        assert not (set(new) & kept)
        assert len(set(new)) == len(new)


def test_random_init_bounds():
    O, F, G, D = 32, 16, 16, 20
    w, idx = _layer(O, F, G, D, seed=9)
    b = 1 / math.sqrt(F)
    w2, _, _, _, mask = oracle.rewire(w, idx, G, D, prune_mode=oracle.PRUNE_FRACTION, k=4,
                                      init_mode=oracle.INIT_RANDOM, bound=b, seed=10)
    vals = bf16_bits_to_f32(w2[mask[np.arange(O) // G]])
    assert np.all(np.abs(vals) <= b * (1 + 2**-8)) and np.unique(vals).size > 10


# ---- the application's variant (GroupFixedFanInReal.rewire, src/group_fanin_real.py:150-286) ----
def _app_case(O=300, F=32, G=16, seed=11):
    g = torch.Generator().manual_seed(seed)
    W = (torch.rand(O, F, generator=g) * 2 - 1).to(torch.bfloat16)
    grad = (torch.randn(O, F, generator=g) * 1e-2).to(torch.bfloat16)
    return W, grad


def _ref_scores(W, grad, G, mode):
    """The reference's own steps in torch: |w| or (w * grad).abs() in the tensors'
    dtype, then index_add_ (mean) or scatter_reduce amax (max) per group."""
    O, F = W.shape
    Gc = (O + G - 1) // G
    gid = torch.arange(O) // G
    val = (W.abs() if grad is None else (W * grad).abs()).to(torch.float32)
    if mode == "mean":
        s = torch.zeros(Gc, F).index_add_(0, gid, val)
        cnt = torch.zeros(Gc).index_add_(0, gid, torch.ones(O)).clamp_min(1).unsqueeze(1)
        return s / cnt
    s = torch.full((Gc, F), -float("inf"))
    return s.scatter_reduce(0, gid[:, None].expand(-1, F), val, reduce="amax", include_self=True)


@pytest.mark.parametrize("mode", ["mean", "max"])
@pytest.mark.parametrize("gkind", [None, "bf16", "f32"])
def test_app_scores_match_reference_steps(mode, gkind):
    W, grad = _app_case()
    if gkind == "f32":
        grad = grad.float() * 1.37
    g_np = None if gkind is None else (grad.view(torch.int16).numpy().view(np.uint16)
                                       if gkind == "bf16" else grad.numpy())
    wb = W.view(torch.int16).numpy().view(np.uint16)
    sm = oracle.SCORE_MEAN if mode == "mean" else oracle.SCORE_MAX
    got = torch.from_numpy(oracle.rewire_scores_ex(wb, 16, sm, g_np))
    ref = _ref_scores(W, None if gkind is None else grad, 16, mode)
    if mode == "max":
        assert torch.equal(got, ref)            # a max does not depend on the order
    else:
        torch.testing.assert_close(got, ref, rtol=2e-6, atol=0)  # summation order differs
    if gkind is None and mode == "mean":
        assert np.array_equal(got.numpy(), oracle.rewire_scores(wb, 16))


def test_app_global_fraction_selects_k_smallest():
    """GLOBAL_FRACTION prunes exactly k = int(Gc*F*fraction) slots of the layer: the
    smallest scores (torch.topk(largest=False) when scores are distinct), ties to
    the lower flat slot (brute-force lexicographic order)."""
    W, _ = _app_case(O=250, F=16, G=16)
    wb = W.view(torch.int16).numpy().view(np.uint16)
    Gc = 16
    idx = np.zeros((Gc, 16), dtype=np.int32)
    k = int(Gc * 16 * 0.15)
    _, _, n, scores, mask = oracle.rewire_ex(wb, idx, 16, 100, prune_mode=oracle.PRUNE_GLOBAL_FRACTION,
                                             score_mode=oracle.SCORE_MAX, k=k, seed=3)
    assert n == k and mask.sum() == k
    flat = scores.reshape(-1)
    order = np.lexsort((np.arange(flat.size), flat))
    assert set(np.flatnonzero(mask.reshape(-1))) == set(order[:k].tolist())
    if len(np.unique(flat)) == flat.size:
        _, ti = torch.topk(torch.from_numpy(flat), k, largest=False)
        assert set(ti.tolist()) == set(order[:k].tolist())
    # ties: all scores equal -> the k lowest flat slots
    z = np.zeros_like(wb)
    _, _, n, _, mask = oracle.rewire_ex(z, idx, 16, 100, prune_mode=oracle.PRUNE_GLOBAL_FRACTION, k=k)
    assert np.array_equal(np.flatnonzero(mask.reshape(-1)), np.arange(k))


def test_app_rewire_invariants():
    """Zero init: every row of a pruned slot is zero, other weights untouched; new
    indices in [0, D); kept indices unchanged."""
    W, grad = _app_case(O=200, F=32, G=16, seed=5)
    wb = W.view(torch.int16).numpy().view(np.uint16)
    Gc, D = 13, 77
    idx = np.random.default_rng(0).integers(0, D, (Gc, 32)).astype(np.int32)
    g_np = grad.view(torch.int16).numpy().view(np.uint16)
    w2, ix2, n, _, mask = oracle.rewire_ex(wb, idx, 16, D, prune_mode=oracle.PRUNE_GLOBAL_FRACTION,
                                           score_mode=oracle.SCORE_MEAN, grad=g_np, k=60, seed=9)
    assert n == 60
    rows_mask = np.repeat(mask, 16, axis=0)[:200]
    assert np.all(w2[rows_mask] == 0) and np.array_equal(w2[~rows_mask], wb[~rows_mask])
    assert np.array_equal(ix2[~mask], idx[~mask]) and ix2.min() >= 0 and ix2.max() < D


# ---- fp16 and fp32 weights (the reference's rewire works in the weights' dtype,
# shared_ffi/rewire.py:155,169-185,224-237; group_fanin_real.py:199-204) ----
def _np_of(t):
    """A tensor as the oracle takes it: uint16 bit patterns (bf16 / fp16) or fp32."""
    if t.dtype == torch.float32:
        return t.numpy()
    return t.view(torch.int16).numpy().view(np.uint16)


_CODE = {torch.bfloat16: oracle.BF16, torch.float16: oracle.F16, torch.float32: oracle.F32}


@pytest.mark.parametrize("mode", ["mean", "max"])
@pytest.mark.parametrize("wdt,gdt", [(torch.float16, None), (torch.float16, torch.float16),
                                     (torch.float16, torch.float32),
                                     (torch.float16, torch.bfloat16),
                                     (torch.float32, None), (torch.float32, torch.float32),
                                     (torch.float32, torch.bfloat16)])
def test_app_scores_other_weight_dtypes_match_reference_steps(mode, wdt, gdt):
    """Scores of fp16 / fp32 weights, with or without a gradient of any dtype,
    equal the reference's torch steps on the same tensors (the product W * grad in
    torch's promoted dtype: fp16 for two fp16 tensors, else fp32)."""
    Wb, gb = _app_case(seed=12)
    W = (Wb.float() * 1.7).to(wdt)
    grad = None if gdt is None else (gb.float() * 0.9).to(gdt)
    sm = oracle.SCORE_MEAN if mode == "mean" else oracle.SCORE_MAX
    got = torch.from_numpy(oracle.rewire_scores_ex(
        _np_of(W), 16, sm, None if grad is None else _np_of(grad), w_dtype=_CODE[wdt],
        grad_dtype=_CODE[gdt] if gdt is not None else oracle.BF16))
    ref = _ref_scores(W, grad, 16, mode)
    if mode == "max":
        assert torch.equal(got, ref)
    else:
        torch.testing.assert_close(got, ref, rtol=2e-6, atol=0)
    if grad is None and mode == "mean":
        assert np.array_equal(got.numpy(), oracle.rewire_scores(_np_of(W), 16, w_dtype=_CODE[wdt]))


@pytest.mark.parametrize("init_mode", ["zero", "random"])
def test_rewire_weight_dtypes_agree(init_mode):
    """Weights that bf16, fp16 and fp32 all hold exactly give the same scores, mask
    and indices in every format; the re-initialised weights are the fp32 draws
    stored in each format (RNE to bf16 / fp16, as is for fp32), every other
    weight unchanged."""
    O, F, G, D = 96, 16, 32, 60
    w, idx = _layer(O, F, G, D, seed=4)
    wf = bf16_bits_to_f32(w)                   # |w| <= 1/4: exact in fp16 too
    b = 1 / math.sqrt(F)
    im = oracle.INIT_ZERO if init_mode == "zero" else oracle.INIT_RANDOM
    kw = dict(prune_mode=oracle.PRUNE_FRACTION, k=5, regrow_mode=oracle.REGROW_UNUSED,
              init_mode=im, bound=b, seed=21)
    wh = wf.astype(np.float16).view(np.uint16)
    r_bf = oracle.rewire(w, idx, G, D, **kw)
    r_h = oracle.rewire(wh, idx, G, D, w_dtype=oracle.F16, **kw)
    r_f = oracle.rewire(wf.copy(), idx, G, D, **kw)
    for r in (r_h, r_f):
        assert np.array_equal(r[1], r_bf[1]) and r[2] == r_bf[2]
        assert np.array_equal(r[3], r_bf[3]) and np.array_equal(r[4], r_bf[4])
    rows = r_bf[4][np.arange(O) // G]
    assert np.array_equal(r_f[0][~rows], wf[~rows]) and np.array_equal(r_h[0][~rows], wh[~rows])
    assert np.array_equal(f32_to_bf16_bits(r_f[0]), r_bf[0])
    assert np.array_equal(r_f[0].astype(np.float16).view(np.uint16), r_h[0])
    if init_mode == "zero":
        assert np.all(r_f[0][rows] == 0)
    else:
        v = r_f[0][rows]
        assert np.all(np.abs(v) <= b) and np.unique(v).size == v.size  # fp32 draws, unrounded
