"""CPU oracle for the HASTE FFI hot path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import this package, and only as the checker (or as the timed CPU
baseline).  The product package ``haste_amd`` never imports it; on a machine
without the HIP library the product raises instead of falling back here.

Two halves:

* ``ffi.py`` -- the reference's layer math restated as a PyTorch-CPU gather + bmm
  formulation in fp32 (forward, backward-to-features, backward-to-weights,
  bias gradient).
* ``haste_oracle.c`` (built to ``libhaste_oracle.so`` by ``oracle/Makefile``) --
  Philox4x32-10 / ``tl.randint``, stochastic rounding, the fused SGD step and
  the rewire contract, bound here through ctypes.

Parity pins for every function are listed in each function's docstring; the
tests that apply them live in ``tests/test_oracle_*.py``.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

from .ffi import (  # noqa: F401  (re-exported)
    ffi_forward,
    ffi_backward_features,
    ffi_backward_weights,
    bias_grad,
    pad_groups,
)

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libhaste_oracle.so")
_lib = None

BF16, F16, F32 = 0, 1, 2
F8E4M3, F8E5M2 = 3, 4   # OCP float8 e4m3fn / e5m2 (torch.float8_e4m3fn / float8_e5m2)
PRUNE_THRESHOLD, PRUNE_FRACTION = 0, 1
REGROW_RANDOM, REGROW_UNUSED = 0, 1
INIT_ZERO, INIT_RANDOM = 0, 1


def build() -> str:
    """Compile the oracle C library with oracle/Makefile; returns its path."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        P = ctypes.c_void_p
        i64, u64, f32, c_int = ctypes.c_int64, ctypes.c_uint64, ctypes.c_float, ctypes.c_int
        L.ho_philox4x32.argtypes = [P, P, c_int, P]
        L.ho_randint.argtypes = [u64, u64]
        L.ho_randint.restype = ctypes.c_uint32
        L.ho_randint_array.argtypes = [u64, u64, i64, P]
        L.ho_sr_bf16.argtypes = [f32, ctypes.c_uint32]
        L.ho_sr_bf16.restype = ctypes.c_uint16
        L.ho_f32_to_bf16_rne.argtypes = [f32]
        L.ho_f32_to_bf16_rne.restype = ctypes.c_uint16
        L.ho_sr_round_bf16.argtypes = [P, P, i64, u64, u64]
        L.ho_sgd_sr_step.argtypes = [P, P, c_int, P, i64, f32, f32, f32, c_int, c_int, u64, u64]
        L.ho_sgd_sr_step_f16w.argtypes = [P, P, c_int, P, i64, f32, f32, f32, c_int, c_int, u64,
                                          u64]
        L.ho_f32_to_f16_rne_arr.argtypes = [P, P, i64]
        L.ho_sr_round.argtypes = [P, P, c_int, i64, u64, u64]
        L.ho_sgd_sr_step_f8w.argtypes = [P, c_int, P, c_int, P, i64, f32, f32, f32, c_int, c_int,
                                         u64, u64]
        L.ho_f8_to_f32_arr.argtypes = [P, c_int, P, i64]
        L.ho_f32_to_f8_arr.argtypes = [P, c_int, P, i64]
        L.ho_sr_e4m3_words.argtypes = [f32, P, P, i64]
        L.ho_f32_to_bf16_rne_arr.argtypes = [P, P, i64]
        L.ho_rewire_scores.argtypes = [P, c_int, P, i64, i64, i64]
        L.ho_rewire.argtypes = [P, c_int, P, i64, i64, i64, i64, c_int, f32, i64, c_int, c_int,
                                f32, u64, P, P]
        L.ho_rewire.restype = i64
        L.ho_rewire_scores_ex.argtypes = [P, c_int, P, c_int, c_int, P, i64, i64, i64]
        L.ho_rewire_ex.argtypes = [P, c_int, P, P, c_int, c_int, i64, i64, i64, i64, c_int, f32,
                                   i64, c_int, c_int, f32, u64, P, P]
        L.ho_rewire_ex.restype = i64
        L.ho_num_threads.restype = c_int
        L.ho_set_num_threads.argtypes = [c_int]
        _lib = L
    return _lib


def _ptr(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def philox4x32(ctr, key, rounds: int = 10) -> np.ndarray:
    """Philox4x32-R block function.  Pinned by Random123 KATs."""
    c = np.ascontiguousarray(np.asarray(ctr, dtype=np.uint32))
    k = np.ascontiguousarray(np.asarray(key, dtype=np.uint32))
    out = np.zeros(4, dtype=np.uint32)
    lib().ho_philox4x32(_ptr(c), _ptr(k), rounds, _ptr(out))
    return out


def randint(seed: int, offset0: int, n: int) -> np.ndarray:
    """tl.randint(seed, offset0 + arange(n)) (Triton random.py randint4x word 0).
    Pinned by tests/golden/randint_vectors.json."""
    out = np.empty(n, dtype=np.uint32)
    lib().ho_randint_array(seed, offset0, n, _ptr(out))
    return out


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 round-to-nearest-even, as uint16 bit patterns."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    lsb = (u >> 16) & 1
    r = ((u + 0x7FFF + lsb) >> 16).astype(np.uint16)
    nan = np.isnan(x)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def bf16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    return (np.asarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def sr_round_bf16(x: np.ndarray, seed: int, offset0: int = 0) -> np.ndarray:
    """stochastic_rounding(x, out, seed) (shared_ffi/sr_triton.py:51-59); returns
    bf16 bit patterns (uint16)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().ho_sr_round_bf16(_ptr(x), _ptr(out), x.size, seed, offset0)
    return out


def sgd_sr_step(w_bits: np.ndarray, g: np.ndarray, m: np.ndarray | None, lr: float, wd: float,
                mu: float, use_mom: bool, do_sr: bool, seed: int, offset0: int = 0):
    """_sgd_m_wd_sr (shared_ffi/sr_triton.py:109-168) on bf16 weights given as
    uint16 bit patterns.  ``g`` is float32, or uint16 bf16 bit patterns.
    Returns (new weight bits, new momentum or None); inputs are not modified."""
    w = np.array(w_bits, dtype=np.uint16, copy=True, order="C")
    if g.dtype == np.uint16:
        g_dtype = BF16
    elif g.dtype == np.float16:
        g_dtype = F16
    else:
        g_dtype = F32
        g = g.astype(np.float32)
    g = np.ascontiguousarray(g)
    mm = None if m is None else np.array(m, dtype=np.float32, copy=True, order="C")
    lib().ho_sgd_sr_step(_ptr(w), _ptr(g), g_dtype, None if mm is None else _ptr(mm), w.size,
                         np.float32(lr), np.float32(wd), np.float32(mu), int(bool(use_mom)),
                         int(bool(do_sr)), seed, offset0)
    return w, mm


def sgd_sr_step_f16w(w: np.ndarray, g: np.ndarray, m: np.ndarray | None, lr: float, wd: float,
                     mu: float, use_mom: bool, do_sr: bool, seed: int, offset0: int = 0):
    """_sgd_m_wd_sr on fp16 weights (shared_ffi/sr_triton.py:109-168 with an fp16
    w_ptr: the bf16 result of the update is stored as fp16).  ``w`` is float16;
    ``g`` as for sgd_sr_step.  Returns (new float16 weights, new momentum or None)."""
    wb = np.array(np.asarray(w, dtype=np.float16).view(np.uint16), copy=True, order="C")
    if g.dtype == np.uint16:
        g_dtype = BF16
    elif g.dtype == np.float16:
        g_dtype = F16
    else:
        g_dtype = F32
        g = g.astype(np.float32)
    g = np.ascontiguousarray(g)
    mm = None if m is None else np.array(m, dtype=np.float32, copy=True, order="C")
    lib().ho_sgd_sr_step_f16w(_ptr(wb), _ptr(g), g_dtype, None if mm is None else _ptr(mm),
                              wb.size, np.float32(lr), np.float32(wd), np.float32(mu),
                              int(bool(use_mom)), int(bool(do_sr)), seed, offset0)
    return wb.view(np.float16), mm


def f32_to_f16_rne(x: np.ndarray) -> np.ndarray:
    """The oracle's fp32 -> fp16 conversion (round to nearest even), as uint16 bits."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().ho_f32_to_f16_rne_arr(_ptr(x), _ptr(out), x.size)
    return out


def f32_to_bf16_rne(x: np.ndarray) -> np.ndarray:
    """The C oracle's fp32 -> bf16 conversion (ho_f32_to_bf16_rne: round to nearest
    even, NaN kept quiet with its sign), as uint16 bits.  It rounds the SGD result
    when stochastic rounding is off and the rewire's new weights."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().ho_f32_to_bf16_rne_arr(_ptr(x), _ptr(out), x.size)
    return out


# element types of the rewire functions' weights and gradients (haste_oracle.c HO_*)
BF16, F16, F32 = 0, 1, 2


def _weights(w: np.ndarray, w_dtype: int, copy: bool):
    """(C-contiguous weights, dtype code): fp32 arrays are F32; uint16 arrays hold
    the bit patterns of w_dtype (BF16 or F16)."""
    if w.dtype == np.float32:
        return np.array(w, dtype=np.float32, copy=copy, order="C"), F32
    assert w_dtype in (BF16, F16), "uint16 weights are bf16 or fp16 bit patterns"
    return np.array(w, dtype=np.uint16, copy=copy, order="C"), w_dtype


def rewire_scores(w_bits: np.ndarray, G: int, w_dtype: int = BF16) -> np.ndarray:
    O, F = w_bits.shape
    Gc = (O + G - 1) // G
    w, wd = _weights(w_bits, w_dtype, copy=False)
    s = np.empty((Gc, F), dtype=np.float32)
    lib().ho_rewire_scores(_ptr(w), wd, _ptr(s), O, F, G)
    return s


def rewire(w_bits: np.ndarray, idx: np.ndarray, G: int, D: int, *, prune_mode: int,
           threshold: float = 0.0, k: int = 0, regrow_mode: int = REGROW_RANDOM,
           init_mode: int = INIT_ZERO, bound: float = 0.0, seed: int = 0, w_dtype: int = BF16):
    """Rewire contract of haste_oracle.c (restating shared_ffi/rewire.py:143-239).
    w_bits: bf16 / fp16 bit patterns (uint16, w_dtype) or fp32 weights.
    Returns (new weights in the same form, new idx, n_pruned, scores, mask)."""
    w, wd = _weights(w_bits, w_dtype, copy=True)
    ix = np.array(idx, dtype=np.int32, copy=True, order="C")
    O, F = w.shape
    Gc = ix.shape[0]
    scores = np.empty((Gc, F), dtype=np.float32)
    mask = np.empty((Gc, F), dtype=np.uint8)
    n = lib().ho_rewire(_ptr(w), wd, _ptr(ix), O, F, G, D, prune_mode, np.float32(threshold), k,
                        regrow_mode, init_mode, np.float32(bound), seed, _ptr(scores), _ptr(mask))
    return w, ix, int(n), scores, mask.astype(bool)


PRUNE_GLOBAL_FRACTION = 2
SCORE_MEAN, SCORE_MAX = 0, 1


def _grad_f32(grad, grad_dtype: int, wd: int):
    """(grad as an fp32 array, the dtype of the product W * grad): grad is None,
    bit patterns (uint16) of grad_dtype (BF16 or F16) or fp32.  The product's
    dtype is torch's promotion of the two: one 16-bit format for both, else fp32."""
    if grad is None:
        return None, F32
    if grad.dtype == np.uint16:
        assert grad_dtype in (BF16, F16), "uint16 gradients are bf16 or fp16 bit patterns"
        gf = (bf16_bits_to_f32(grad) if grad_dtype == BF16 else
              np.asarray(grad, dtype=np.uint16).view(np.float16).astype(np.float32))
        gd = grad_dtype
    else:
        gf, gd = grad, F32
    return np.ascontiguousarray(gf, dtype=np.float32), (gd if gd == wd else F32)


def rewire_scores_ex(w_bits: np.ndarray, G: int, score_mode: int = SCORE_MEAN,
                     grad: np.ndarray | None = None, w_dtype: int = BF16,
                     grad_dtype: int = BF16) -> np.ndarray:
    """Scores of the application's rewire variant (haste_oracle.c:ho_rewire_scores_ex);
    weights and grad are None (grad only), bit patterns (uint16) of w_dtype /
    grad_dtype, or fp32."""
    O, F = w_bits.shape
    Gc = (O + G - 1) // G
    w, wd = _weights(w_bits, w_dtype, copy=False)
    gf, pd = _grad_f32(grad, grad_dtype, wd)
    s = np.empty((Gc, F), dtype=np.float32)
    lib().ho_rewire_scores_ex(_ptr(w), wd, None if gf is None else _ptr(gf), pd, score_mode,
                              _ptr(s), O, F, G)
    return s


def rewire_ex(w_bits: np.ndarray, idx: np.ndarray, G: int, D: int, *, prune_mode: int,
              score_mode: int = SCORE_MEAN, grad: np.ndarray | None = None,
              threshold: float = 0.0, k: int = 0, regrow_mode: int = REGROW_RANDOM,
              init_mode: int = INIT_ZERO, bound: float = 0.0, seed: int = 0,
              w_dtype: int = BF16, grad_dtype: int = BF16):
    """The application's rewire variant (GroupFixedFanInReal.rewire,
    src/group_fanin_real.py:150-286) under the contract of haste_oracle.c;
    k is per group for PRUNE_FRACTION and for the whole layer for
    PRUNE_GLOBAL_FRACTION.  Weights and grad as rewire_scores_ex.
    Returns (weights in the same form, idx, n_pruned, scores, mask)."""
    w, wd = _weights(w_bits, w_dtype, copy=True)
    ix = np.array(idx, dtype=np.int32, copy=True, order="C")
    O, F = w.shape
    Gc = ix.shape[0]
    gf, pd = _grad_f32(grad, grad_dtype, wd)
    scores = np.empty((Gc, F), dtype=np.float32)
    mask = np.empty((Gc, F), dtype=np.uint8)
    n = lib().ho_rewire_ex(_ptr(w), wd, _ptr(ix), None if gf is None else _ptr(gf), pd, score_mode,
                           O, F, G, D, prune_mode, np.float32(threshold), k, regrow_mode,
                           init_mode, np.float32(bound), seed, _ptr(scores), _ptr(mask))
    return w, ix, int(n), scores, mask.astype(bool)


def set_num_threads(n: int) -> None:
    lib().ho_set_num_threads(int(n))


def num_threads() -> int:
    return int(lib().ho_num_threads())


def f8_to_f32(codes: np.ndarray, fmt: int) -> np.ndarray:
    """fp8 codes (uint8) of format fmt (F8E4M3 / F8E5M2) -> fp32, exact
    (ho_f8_to_f32)."""
    c = np.ascontiguousarray(codes, dtype=np.uint8)
    out = np.empty(c.shape, dtype=np.float32)
    lib().ho_f8_to_f32_arr(_ptr(c), fmt, _ptr(out), c.size)
    return out


def f32_to_f8(x: np.ndarray, fmt: int) -> np.ndarray:
    """fp32 -> fp8 codes, round to nearest even, saturating (ho_f32_to_f8)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint8)
    lib().ho_f32_to_f8_arr(_ptr(x), fmt, _ptr(out), x.size)
    return out


def sr_e4m3_words(x: float, words: np.ndarray) -> np.ndarray:
    """stochastic_rounding_to_fp8 of one value under each random word (uint32)."""
    w = np.ascontiguousarray(words, dtype=np.uint32)
    out = np.empty(w.shape, dtype=np.uint8)
    lib().ho_sr_e4m3_words(float(x), _ptr(w), _ptr(out), w.size)
    return out


def sr_round(x: np.ndarray, out_dtype: int, seed: int, offset0: int = 0) -> np.ndarray:
    """stochastic_rounding(x, output, seed) (sr_triton.py:27-59) for an output of
    dtype out_dtype (BF16 / F16: uint16 bit patterns; F8E4M3 / F8E5M2: uint8 codes)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint8 if out_dtype in (F8E4M3, F8E5M2) else np.uint16)
    lib().ho_sr_round(_ptr(x), _ptr(out), out_dtype, x.size, seed, offset0)
    return out


def sgd_sr_step_f8w(w: np.ndarray, fmt: int, g: np.ndarray, m: np.ndarray | None, lr: float,
                    wd: float, mu: float, use_mom: bool, do_sr: bool, seed: int,
                    offset0: int = 0):
    """_sgd_m_wd_sr (sr_triton.py:109-168) on fp8 weights (uint8 codes of fmt):
    the bf16 result of the update stored as fp8.  ``g`` is float32, or uint16
    bf16 bit patterns, or float16.  Returns (new codes, new momentum or None)."""
    wc = np.ascontiguousarray(w, dtype=np.uint8).copy()
    if g.dtype == np.float32:
        g_dtype = F32
    elif g.dtype == np.uint16:
        g_dtype = BF16
    else:
        g_dtype = F16
    g = np.ascontiguousarray(g)
    mm = None if m is None else np.ascontiguousarray(m, dtype=np.float32).copy()
    lib().ho_sgd_sr_step_f8w(_ptr(wc), fmt, _ptr(g), g_dtype, None if mm is None else _ptr(mm),
                             wc.size, lr, wd, mu, int(use_mom), int(do_sr), seed, offset0)
    return wc, mm
