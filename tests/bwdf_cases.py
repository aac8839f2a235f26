"""Shapes that reach every build of the bwd-features main kernel.

The LDS-ring build (haste_ffi_bwd_features_set_build(1)) is compiled per
(group size G, batch tile BT, ring tiles RT): BT is 64 or 128 batch columns,
and RT is 2, 3 or the per-G maximum (8, 6, 4, 3 for G = 16, 32, 64, 128),
chosen per shape by the library's plan.  RING_CASES holds one shape per build
(B, D, O, G, F, idx_mode), each with two feature ranges.

The staged build (the default for G >= 32, set_build(3)) is compiled per
(G, BT) with G in {32, 64, 128} and BT in {32, 64}.  STAGED_CASES holds one
shape per (G, BT, more than one feature range); G = 128 takes 64 batch columns
only where the whole of D fits one range.

tests/test_abi.py checks on the CPU that the library maps the cases onto
every build, tests/test_gpu_ffi.py runs them against the oracle.
"""
import ctypes

MAX_RING = {16: 8, 32: 6, 64: 4, 128: 3}


def all_variants():
    return {(G, BT, RT) for G, r in MAX_RING.items() for BT in (64, 128)
            for RT in sorted({2, 3, r})}


RING_CASES = [
    (37, 768, 2000, 16, 16, "random"), (37, 768, 2003, 16, 64, "dups"),
    (37, 768, 2000, 16, 128, "random"), (100, 300, 2000, 16, 16, "dups"),
    (100, 300, 1999, 16, 64, "random"), (100, 300, 2000, 16, 128, "dups"),
    (37, 768, 2000, 32, 16, "dups"), (37, 768, 2005, 32, 64, "random"),
    (37, 768, 2000, 32, 128, "dups"), (100, 300, 2000, 32, 16, "random"),
    (100, 300, 2000, 32, 64, "dups"), (100, 300, 2001, 32, 128, "random"),
    (37, 768, 2000, 64, 16, "random"), (37, 768, 2000, 64, 64, "dups"),
    (37, 768, 2007, 64, 128, "random"), (100, 300, 2000, 64, 16, "dups"),
    (100, 300, 2000, 64, 64, "random"), (100, 300, 2000, 64, 128, "dups"),
    (37, 768, 2000, 128, 16, "dups"), (37, 768, 1993, 128, 64, "random"),
    (100, 300, 2000, 128, 16, "random"), (100, 300, 2000, 128, 64, "dups"),
]


STAGED_CASES = [
    (37, 768, 2000, 32, 16, "random"), (37, 1500, 2000, 32, 256, "dups"),
    (37, 300, 2000, 32, 16, "dups"), (37, 1500, 2000, 32, 16, "random"),
    (37, 768, 2000, 64, 16, "dups"), (37, 4096, 2000, 64, 16, "random"),
    (37, 300, 2000, 64, 16, "random"), (37, 1000, 2000, 64, 16, "dups"),
    (37, 768, 2000, 128, 16, "random"), (37, 1500, 2000, 128, 16, "dups"),
    (37, 200, 2000, 128, 16, "dups"),
]


def staged_variants():
    """(G, BT, several feature ranges) of every staged build the cases reach."""
    v = {(G, BT, multi) for G in (32, 64, 128) for BT in (32, 64) for multi in (False, True)}
    return v - {(128, 64, True)}


def kernel_config(lib, B, D, O, G, F, dtype_code=0):
    """(BT, RT, feature ranges, slices) the library plans for these sizes."""
    cfg = (ctypes.c_int64 * 4)()
    rc = lib.haste_ffi_bwd_features_config(B, D, F, O, G, dtype_code, cfg)
    assert rc == 0, rc
    return tuple(int(v) for v in cfg)
