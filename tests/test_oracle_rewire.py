"""Pins the oracle's rewire contract (restating shared_ffi/rewire.py:143-239)."""
import math

import numpy as np
import pytest

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
