"""C-ABI library: loads, exports every declared symbol, and rejects bad
arguments on the host (these calls return before any HIP call)."""
import ctypes
import os
import re

import pytest
import torch

from haste_amd import _lib

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include",
                      "haste_ffi.h")


def _declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(haste_[a-z0-9_]+)\s*\(", text)))


def test_header_and_binding_agree():
    assert set(_declared_symbols()) == set(_lib.SIGNATURES)


def test_library_exports_every_symbol():
    L = ctypes.CDLL(_lib.LIB_PATH)
    for name in _declared_symbols():
        assert hasattr(L, name), name


def test_version_and_error_string():
    assert _lib.lib().haste_abi_version() == 2
    assert isinstance(_lib.last_error(), str)


def _fwd(**kw):
    args = dict(idx=8, xT=16, ldx=64, W=32, bias=None, out=48, ldo=4096, B=64, D=768, F=32,
                O=4096, G=32, dtype=_lib.DTYPE_BF16, stream=None)
    args.update(kw)
    return _lib.lib().haste_ffi_forward(*args.values())


def test_forward_rejects_bad_group_size():
    assert _fwd(G=48) == _lib.HASTE_ERR_UNSUPPORTED
    assert "group size" in _lib.last_error()


def test_forward_rejects_bad_fanin():
    assert _fwd(F=24) == _lib.HASTE_ERR_INVALID_ARG
    assert "FANIN size should be multiple of 16" in _lib.last_error()
    assert _fwd(F=512) == _lib.HASTE_ERR_UNSUPPORTED


def test_forward_rejects_bad_strides_and_dtype():
    assert _fwd(ldx=60) == _lib.HASTE_ERR_INVALID_ARG
    assert _fwd(ldo=4095) == _lib.HASTE_ERR_INVALID_ARG
    assert _fwd(dtype=_lib.DTYPE_F32) == _lib.HASTE_ERR_UNSUPPORTED
    assert _fwd(B=0) == _lib.HASTE_ERR_INVALID_ARG
    assert _fwd(xT=18) == _lib.HASTE_ERR_INVALID_ARG  # misaligned


def test_forward_f32out_rejects_bad_arguments():
    def call(**kw):
        args = dict(idx=8, xT=16, ldx=64, W=32, bias=None, out=48, ldo=4096, B=64, D=768, F=32,
                    O=4096, G=32, stream=None)
        args.update(kw)
        return _lib.lib().haste_ffi_forward_f16_f32out(*args.values())

    assert call(G=48) == _lib.HASTE_ERR_UNSUPPORTED
    assert call(F=24) == _lib.HASTE_ERR_INVALID_ARG
    assert call(ldo=4092) == _lib.HASTE_ERR_INVALID_ARG
    assert call(out=52) == _lib.HASTE_ERR_INVALID_ARG   # fp32 logits need 16-byte alignment
    assert call(bias=50) == _lib.HASTE_ERR_INVALID_ARG  # fp32 bias, 4-byte alignment
    assert call(idx=None) == _lib.HASTE_ERR_INVALID_ARG
    assert "haste_ffi_forward_f16_f32out" in _lib.last_error()


def test_bwd_features_workspace_size():
    L = _lib.lib()
    n = L.haste_ffi_bwd_features_workspace_size(512, 768, 128, 131073, 64, _lib.DTYPE_BF16)
    assert n > 0 and n % 4 == 0
    assert L.haste_ffi_bwd_features_workspace_size(512, 768, 128, 131073, 48, 0) < 0


def test_bwd_features_rejects_small_workspace():
    L = _lib.lib()
    rc = L.haste_ffi_bwd_features(16, 32, 48, 4096, 64, 256, 16, 64, 768, 32, 4096, 32,
                                  _lib.DTYPE_BF16, 0, None)
    assert rc == _lib.HASTE_ERR_WORKSPACE
    assert "workspace too small" in _lib.last_error()


def test_sgd_rejects_bad_dtype_and_missing_momentum():
    L = _lib.lib()
    assert L.haste_sgd_sr_step(16, 32, 7, None, 100, 0.1, 0.0, 0.0, 0, 1, 1, 0, None) == \
        _lib.HASTE_ERR_UNSUPPORTED
    assert L.haste_sgd_sr_step(16, 32, 0, None, 100, 0.1, 0.0, 0.9, 1, 1, 1, 0, None) == \
        _lib.HASTE_ERR_INVALID_ARG
    assert L.haste_sgd_sr_step(16, 32, 0, None, 0, 0.1, 0.0, 0.0, 0, 1, 1, 0, None) == _lib.HASTE_OK


def test_rewire_rejects_bad_modes():
    L = _lib.lib()
    bf16 = _lib.DTYPE_BF16
    assert L.haste_rewire(16, bf16, 32, None, None, 100, 8, 16, 50, 5, 0.0, 0, 0, 0, 0.1, 1,
                          None) == _lib.HASTE_ERR_INVALID_ARG
    assert L.haste_rewire(16, bf16, 32, None, None, 100, 8, 16, 50, 1, 0.0, 9, 0, 0, 0.1, 1,
                          None) == _lib.HASTE_ERR_INVALID_ARG
    # weights must be bf16, fp16 or fp32
    assert L.haste_rewire(16, 7, 32, None, None, 100, 8, 16, 50, 1, 0.0, 2, 0, 0, 0.1, 1,
                          None) == _lib.HASTE_ERR_INVALID_ARG
    assert "bf16, fp16 or fp32" in _lib.last_error()
    assert L.haste_rewire_scores(16, 7, None, 0, 0, 32, 100, 8, 16, None) == \
        _lib.HASTE_ERR_INVALID_ARG


def test_check_raises_haste_error():
    assert _fwd(G=48) != 0
    with pytest.raises(_lib.HasteError, match="group size"):
        _lib.check(_fwd(G=48))


def test_python_api_rejects_cpu_tensors():
    """The product path has no CPU implementation: CPU tensors raise."""
    from haste_amd import ops, sr
    x = torch.randn(4, 16).to(torch.bfloat16)
    W = torch.randn(32, 16).to(torch.bfloat16)
    idx = torch.zeros(1, 16, dtype=torch.int32)
    with pytest.raises(RuntimeError, match="HIP device"):
        ops.group_ffi_mul(x, W, idx, None, gsize=32)
    with pytest.raises(RuntimeError, match="HIP device"):
        sr.stochastic_rounding(torch.randn(8), torch.empty(8, dtype=torch.bfloat16), 1)


def _bwdw_sgd(**kw):
    args = dict(idx=16, xT=16, ldx=64, dY=32, lddy=4096, W=48, bias=None, mW=None, mb=None,
                dW=None, dW_dtype=_lib.DTYPE_F32, dbias=None, dbias_dtype=_lib.DTYPE_F32,
                lr=0.05, wd=1e-4, mu=0.0, use_mom=0, do_sr=1, seed=42, ws=None, ws_bytes=0, B=64, D=768, F=32, O=4096,
                G=32, dtype=_lib.DTYPE_BF16, stream=None)
    args.update(kw)
    return _lib.lib().haste_ffi_bwd_weights_sgd(*args.values())


def test_bwd_weights_sgd_rejects_bad_arguments():
    assert _bwdw_sgd(dtype=_lib.DTYPE_F16) == _lib.HASTE_ERR_INVALID_ARG
    assert "bf16 weights only" in _lib.last_error()
    assert _bwdw_sgd(use_mom=1) == _lib.HASTE_ERR_INVALID_ARG  # no momentum buffers
    assert _bwdw_sgd(W=None) == _lib.HASTE_ERR_INVALID_ARG
    assert _bwdw_sgd(G=48) == _lib.HASTE_ERR_UNSUPPORTED
    assert _bwdw_sgd(lddy=4092) == _lib.HASTE_ERR_INVALID_ARG
    assert _bwdw_sgd(ws=64, ws_bytes=16) == _lib.HASTE_ERR_INVALID_ARG  # workspace too small


def test_bwd_weights_sgd_dx_requires_dx_and_workspace():
    args = dict(idx=16, xT=16, ldx=64, dY=32, lddy=4096, W=48, bias=None, mW=None, mb=None,
                lr=0.05, wd=1e-4, mu=0.0, use_mom=0, do_sr=1, seed=42, dX=64, dx_seed=123,
                ws=256, ws_bytes=1 << 30, B=64, D=768, F=32, O=4096, G=32,
                dtype=_lib.DTYPE_BF16, stream=None)
    f = _lib.lib().haste_ffi_bwd_weights_sgd_dx
    assert f(*dict(args, dX=None).values()) == _lib.HASTE_ERR_INVALID_ARG
    assert "dX and the bwd-features workspace" in _lib.last_error()
    assert f(*dict(args, ws=None).values()) == _lib.HASTE_ERR_INVALID_ARG
    assert f(*dict(args, ws_bytes=16).values()) == _lib.HASTE_ERR_INVALID_ARG
    assert "workspace too small" in _lib.last_error()
    assert f(*dict(args, dtype=_lib.DTYPE_F16).values()) == _lib.HASTE_ERR_INVALID_ARG


def test_bwd_weights_dx_requires_dx_workspace_and_bf16():
    args = dict(idx=16, xT=16, ldx=64, dY=32, lddy=4096, dW=48, dW_dtype=_lib.DTYPE_F32,
                dbias=None, dbias_dtype=0, dX=64, dx_seed=123, ws=256, ws_bytes=1 << 30, B=64,
                D=768, F=32, O=4096, G=32, dtype=_lib.DTYPE_BF16, stream=None)
    f = _lib.lib().haste_ffi_bwd_weights_dx
    assert f(*dict(args, dX=None).values()) == _lib.HASTE_ERR_INVALID_ARG
    assert "dX and the bwd-features workspace" in _lib.last_error()
    assert f(*dict(args, ws=None).values()) == _lib.HASTE_ERR_INVALID_ARG
    assert f(*dict(args, ws_bytes=16).values()) == _lib.HASTE_ERR_INVALID_ARG
    assert "workspace too small" in _lib.last_error()
    assert f(*dict(args, dW=None).values()) == _lib.HASTE_ERR_INVALID_ARG
    assert f(*dict(args, dtype=_lib.DTYPE_F16).values()) == _lib.HASTE_ERR_INVALID_ARG
    assert "must be bf16" in _lib.last_error()


def test_sgd_wt_bias_rejects_bad_arguments():
    args = dict(W=16, g=32, g_dtype=_lib.DTYPE_BF16, m=None, bias=48, gb=64,
                gb_dtype=_lib.DTYPE_F32, mb=None, lr=0.05, wd=1e-4, mu=0.0, use_mom=0, do_sr=1,
                seed=42, ws=256, ws_bytes=1 << 30, B=64, D=768, F=32, O=4096, G=32,
                dtype=_lib.DTYPE_BF16, stream=None)
    f = _lib.lib().haste_sgd_sr_step_wt_bias
    assert f(*dict(args, bias=None).values()) == _lib.HASTE_ERR_INVALID_ARG
    assert "null bias" in _lib.last_error()
    assert f(*dict(args, gb=None).values()) == _lib.HASTE_ERR_INVALID_ARG
    assert "bias needs its gradient" in _lib.last_error()
    assert f(*dict(args, use_mom=1, m=80).values()) == _lib.HASTE_ERR_INVALID_ARG
    assert f(*dict(args, gb_dtype=7).values()) == _lib.HASTE_ERR_INVALID_ARG
    assert "bad bias gradient dtype" in _lib.last_error()
    assert f(*dict(args, ws_bytes=16).values()) == _lib.HASTE_ERR_WORKSPACE
    assert f(*dict(args, dtype=_lib.DTYPE_F16).values()) == _lib.HASTE_ERR_INVALID_ARG


def test_ring_cases_reach_every_bwd_features_build():
    """tests/bwdf_cases.RING_CASES maps onto every (G, BT, RT) build of the
    bwd-features main kernel, each with more than one feature range, so the GPU
    parity test over them covers every build (no GPU call: the plan's shape
    is computed on the host)."""
    from bwdf_cases import RING_CASES, all_variants, kernel_config

    seen = set()
    prev = _lib.lib().haste_ffi_bwd_features_set_build(1)
    try:
        for B, D, O, G, F, _ in RING_CASES:
            BT, RT, ndr, _S = kernel_config(_lib.lib(), B, D, O, G, F)
            assert ndr >= 2, (B, D, O, G, F)
            seen.add((G, BT, RT))
    finally:
        _lib.lib().haste_ffi_bwd_features_set_build(prev)
    assert seen == all_variants()


def test_staged_cases_reach_every_staged_build():
    """tests/bwdf_cases.STAGED_CASES maps onto every (G, BT) build of the staged
    main kernel, with one and with several feature ranges; the default build
    (0) is the staged one for G >= 32 and the ring build for G = 16."""
    from bwdf_cases import STAGED_CASES, kernel_config, staged_variants

    L = _lib.lib()
    seen = set()
    prev = L.haste_ffi_bwd_features_set_build(3)
    try:
        for B, D, O, G, F, _ in STAGED_CASES:
            BT, RT, ndr, _S = kernel_config(L, B, D, O, G, F)
            assert RT == 0, (B, D, O, G, F)
            seen.add((G, BT, ndr >= 2))
    finally:
        L.haste_ffi_bwd_features_set_build(prev)
    assert seen == staged_variants()
    assert kernel_config(L, 512, 768, 131073, 64, 128)[1] == 0   # default: staged
    assert kernel_config(L, 100, 300, 1000, 16, 16)[1] > 0        # G = 16: ring


def test_sr_words_fold_rejects_bad_arguments():
    L = _lib.lib()
    assert L.haste_sr_words_fold(None, -1, 0, None) == _lib.HASTE_ERR_INVALID_ARG
    assert L.haste_sr_words_fold(None, 10, 0, None) == _lib.HASTE_ERR_INVALID_ARG
    assert L.haste_sr_words_fold(None, 0, 0, None) == 0


def test_forward_bce_noalloc_rejects_shapes_beyond_its_scratch():
    """The no-allocation forward+loss refuses, before any HIP call, a shape whose
    workspace exceeds the library's fixed per-GPU scratch (64 MiB): BASELINE
    config 4's label bitmap alone is 384 MB."""
    L = _lib.lib()
    B, D, F, O, G = 1024, 768, 128, 3_000_000, 128
    assert L.haste_ffi_forward_bce_workspace_size(B, O, G) > 64 << 20
    rc = L.haste_ffi_forward_bce_noalloc(16, 16, 1024, 16, None, 16, 10, 16, 3000064, None, 16,
                                         B, D, F, O, G, _lib.DTYPE_BF16, None)
    assert rc == _lib.HASTE_ERR_WORKSPACE
    assert "scratch" in _lib.last_error()
    # config 2 fits
    assert L.haste_ffi_forward_bce_workspace_size(512, 670091, 64) <= 64 << 20


def test_bwd_features_set_build():
    L = _lib.lib()
    assert L.haste_ffi_bwd_features_set_build(4) == _lib.HASTE_ERR_INVALID_ARG
    assert L.haste_ffi_bwd_features_set_build(-1) == _lib.HASTE_ERR_INVALID_ARG
    prev = L.haste_ffi_bwd_features_set_build(1)
    assert prev == 0
    assert L.haste_ffi_bwd_features_set_build(2) == 1
    assert L.haste_ffi_bwd_features_set_build(3) == 2
    assert L.haste_ffi_bwd_features_set_build(prev) == 3


def test_sr_round_and_f8_sgd_reject_bad_arguments():
    """Checked before any HIP call: output / weight dtypes outside the supported
    ones, negative sizes, null pointers."""
    L = _lib.lib()
    E = _lib.HASTE_ERR_INVALID_ARG
    assert L.haste_sr_round(None, None, _lib.DTYPE_F32, 10, 1, 0, None) == E
    assert L.haste_sr_round(None, None, _lib.DTYPE_F16, -1, 1, 0, None) == E
    assert L.haste_sr_round(None, None, _lib.DTYPE_F8E4M3, 10, 1, 0, None) == E
    assert L.haste_sr_round(None, None, _lib.DTYPE_F8E5M2, 0, 1, 0, None) == 0
    args = (0.1, 0.0, 0.0, 0, 1, 5, 0, None)
    assert L.haste_sgd_sr_step_f8(None, _lib.DTYPE_BF16, None, _lib.DTYPE_F32, None, 10, *args) == E
    assert L.haste_sgd_sr_step_f8(None, _lib.DTYPE_F8E4M3, None, _lib.DTYPE_F32, None, 10, *args) == E
    assert L.haste_sgd_sr_step_f8(None, _lib.DTYPE_F8E5M2, None, _lib.DTYPE_F32, None, 0, *args) == 0
