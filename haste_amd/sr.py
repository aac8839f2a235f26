"""Stochastic rounding and the fused SGD step (host side).

Same signatures, assertions and semantics as the reference's Triton host
functions (shared_ffi/sr_triton.py:51-59 and :172-213), implemented on the HIP
kernels of libhaste_ffi.so.  Random bits are Triton's tl.randint(seed, i)
(Philox4x32-10, word 0, counter = element index from 0 per tensor), so the
results are bit-identical under the FMA contract stated in include/haste_ffi.h.
"""
from __future__ import annotations

import torch

from . import _lib
from ._C import dtype_code, require_device, stream_of

__all__ = ["stochastic_rounding", "sgd_update", "sgd_update_multi"]

# output / weight dtypes of the reference's dispatch (sr_triton.py:43-46, and
# the store conversion of _sgd_m_wd_sr's w_ptr, :111,167-168)
_SR_OUT = {torch.bfloat16: _lib.DTYPE_BF16, torch.float16: _lib.DTYPE_F16,
           torch.float8_e4m3fn: _lib.DTYPE_F8E4M3, torch.float8_e5m2: _lib.DTYPE_F8E5M2}
_F8_W = {torch.float8_e4m3fn: _lib.DTYPE_F8E4M3, torch.float8_e5m2: _lib.DTYPE_F8E5M2}


def stochastic_rounding(x: torch.Tensor, output: torch.Tensor, seed: int) -> None:
    """output[i] = SR(x[i], tl.randint(seed, i)) (sr_triton.py:27-59): float8_e4m3fn
    outputs take the 20-bit rounding of stochastic_rounding_to_fp8, bf16, fp16 and
    float8_e5m2 outputs the bf16 rounding stored in their dtype."""
    assert x.is_contiguous()
    assert output.is_contiguous()
    assert x.shape == output.shape
    assert x.dtype == torch.float32
    assert output.dtype != torch.float32
    if output.dtype not in _SR_OUT:
        raise NotImplementedError(
            f"stochastic_rounding: output dtype {output.dtype} is not supported (bfloat16, "
            "float16, float8_e4m3fn and float8_e5m2 are)")
    require_device(x, "x")
    require_device(output, "output")
    if output.dtype == torch.bfloat16:
        _lib.call("haste_sr_round_bf16", x.data_ptr(), output.data_ptr(), x.numel(), int(seed),
                  0, stream_of(x))
    else:
        _lib.call("haste_sr_round", x.data_ptr(), output.data_ptr(), _SR_OUT[output.dtype],
                  x.numel(), int(seed), 0, stream_of(x))


def sgd_update(weights: torch.Tensor, gradient: torch.Tensor, momentum_buf: torch.Tensor,
               learning_rate: float, weight_decay: float, momentum: float, use_momentum: bool,
               stochastic_rounding: bool, seed: int) -> None:
    """Fused SGD + optional momentum + weight decay + SR, in place on ``weights``
    (sr_triton.py:172-213).  ``momentum_buf`` may be None when momentum is off."""
    assert weights.is_contiguous(), "weights must be contiguous"
    assert gradient.is_contiguous(), "gradient must be contiguous"
    use_mom_flag = 1 if (use_momentum and momentum != 0.0) else 0
    if momentum_buf is not None:
        assert momentum_buf.is_contiguous(), "momentum_buf must be contiguous"
        assert weights.shape == gradient.shape == momentum_buf.shape
    else:
        assert weights.shape == gradient.shape
        assert not use_mom_flag, "momentum_buf is required when momentum is used"
    if weights.dtype not in (torch.bfloat16, torch.float16) and weights.dtype not in _F8_W:
        raise NotImplementedError(f"sgd_update: weights must be bfloat16, float16, "
                                  f"float8_e4m3fn or float8_e5m2 (got {weights.dtype})")
    require_device(weights, "weights")
    require_device(gradient, "gradient")
    if use_mom_flag:
        assert momentum_buf.dtype == torch.float32
    if weights.dtype in _F8_W:
        # fp8 weights: the bf16 result is stored as fp8 (rounded to nearest,
        # saturating), as the reference's store into an fp8 w_ptr converts it
        _lib.call("haste_sgd_sr_step_f8", weights.data_ptr(), _F8_W[weights.dtype],
                  gradient.data_ptr(), dtype_code(gradient.dtype),
                  momentum_buf.data_ptr() if use_mom_flag else None, weights.numel(),
                  float(learning_rate), float(weight_decay), float(momentum), use_mom_flag,
                  1 if stochastic_rounding else 0, int(seed), 0, stream_of(weights))
        return
    # fp16 weights: the bf16 result is stored as fp16, as the reference's store does
    fn = "haste_sgd_sr_step" if weights.dtype == torch.bfloat16 else "haste_sgd_sr_step_f16"
    _lib.call(fn, weights.data_ptr(), gradient.data_ptr(),
              dtype_code(gradient.dtype),
              momentum_buf.data_ptr() if use_mom_flag else None, weights.numel(),
              float(learning_rate), float(weight_decay), float(momentum), use_mom_flag,
              1 if stochastic_rounding else 0, int(seed), 0, stream_of(weights))


def sgd_update_multi(weights, gradients, momentum_bufs, learning_rate: float, weight_decay: float,
                     momentum: float, use_momentum: bool, stochastic_rounding: bool,
                     seed: int) -> None:
    """``sgd_update`` over several tensors in one launch per 8 tensors; every
    tensor uses ``seed`` with offsets from 0 (as a loop of sgd_update calls,
    optim_sr.py:64-112).  Gradients must share one dtype."""
    n = len(weights)
    assert len(gradients) == n and (momentum_bufs is None or len(momentum_bufs) == n)
    if n == 0:
        return
    if any(w.dtype != torch.bfloat16 for w in weights):
        # fp16 and fp8 weights go one tensor at a time (same seed, offsets from
        # 0); the bf16 ones share the launch below
        keep = []
        for i, w in enumerate(weights):
            m = None if momentum_bufs is None else momentum_bufs[i]
            if w.dtype != torch.bfloat16:
                sgd_update(w, gradients[i], m, learning_rate, weight_decay, momentum,
                           use_momentum, stochastic_rounding, seed)
            else:
                keep.append(i)
        if not keep:
            return
        weights = [weights[i] for i in keep]
        gradients = [gradients[i] for i in keep]
        momentum_bufs = None if momentum_bufs is None else [momentum_bufs[i] for i in keep]
        n = len(weights)
    use_mom_flag = 1 if (use_momentum and momentum != 0.0) else 0
    gdt = gradients[0].dtype
    arr = (_lib.SgdTensor * n)()
    for i, (w, g) in enumerate(zip(weights, gradients)):
        m = None if momentum_bufs is None else momentum_bufs[i]
        assert w.is_contiguous() and g.is_contiguous() and w.shape == g.shape
        assert g.dtype == gdt, "sgd_update_multi: gradients must share one dtype"
        if w.dtype != torch.bfloat16:
            raise NotImplementedError(f"sgd_update: weights must be bfloat16 (got {w.dtype})")
        require_device(w, "weights")
        require_device(g, "gradient")
        if use_mom_flag:
            assert m is not None and m.is_contiguous() and m.shape == w.shape
            assert m.dtype == torch.float32
        arr[i] = _lib.SgdTensor(w.data_ptr(), g.data_ptr(), m.data_ptr() if use_mom_flag else None,
                                w.numel(), 0)
    _lib.call("haste_sgd_sr_step_multi", arr, n, dtype_code(gdt), float(learning_rate),
              float(weight_decay), float(momentum), use_mom_flag, 1 if stochastic_rounding else 0,
              int(seed), stream_of(weights[0]))
