"""Autograd Function for the grouped FFI layer (reference: shared_ffi/bindings.py:8-54).

Numerics contract (drop-in mode, as the reference):
  logits  = RNE(fp32 gathered contraction + fp32 bias), features dtype
  dX      = bf16 stochastic rounding of the fp32 feature gradient with the fixed
            seed 123 and offsets over [B, D] row-major (bindings.py:44-48);
            fp16 inputs are rounded to nearest instead (bindings.py:49-50)
  dW      = RNE of the fp32 weight gradient, weights dtype
  dbias   = column sum of grad_output (fp32 accumulation), bias dtype
When a parameter's ``grad_dtype`` is torch.float32 (torch >= 2.10), its
gradient is returned in fp32 straight from the kernel's accumulator (no
rounding); SRSgd / sgd_update read fp32 gradients directly.

Differences in mechanics (not in values): the feature gradient is computed
deterministically and written straight into [B, D] (no fp32 [D, B]
intermediate and transposes), the bias gradient comes out of the
weight-gradient kernel (no second read of grad_output), and gradients that
autograd does not need are skipped.  gsize is kept on ctx instead of a saved
tensor, so backward does no device->host sync.
"""
from __future__ import annotations

from typing import Any, Optional

import torch

from . import _C, _lib

SR_SEED_GRAD_X = 123  # bindings.py:48


def _grad_dtype(p: torch.Tensor) -> torch.dtype:
    """dtype autograd will store for p.grad: p.grad_dtype if set (torch >= 2.10), else p.dtype."""
    gd = getattr(p, "grad_dtype", None)
    return gd if gd is not None else p.dtype


class GroupFFIMulFunction(torch.autograd.Function):
    @staticmethod
    @torch.amp.custom_fwd(device_type="cuda")
    def forward(ctx: Any, features: torch.Tensor, weights: torch.Tensor,
                group_locations: torch.Tensor, bias: Optional[torch.Tensor],
                gsize: int = 32) -> torch.Tensor:
        _C.require_device(features, "features")
        if features.dim() != 2:
            raise RuntimeError(f"features must be 2-D [B, D] (got {list(features.shape)})")
        B, D = features.shape
        O, F = weights.shape
        xT, ldx = _C.padded_transpose(features)          # bindings.py:19, rows padded to 8
        out = _C.ffi_forward_cuda(group_locations, xT, weights, bias, B, D, F, O, gsize)
        ctx.save_for_backward(xT, weights, group_locations)
        ctx.gsize = int(gsize)
        ctx.use_bias = bias is not None
        ctx.w_grad_dtype = _grad_dtype(weights)
        ctx.bias_dtype = _grad_dtype(bias) if bias is not None else None
        return out

    @staticmethod
    @torch.amp.custom_bwd(device_type="cuda")
    def backward(ctx, grad_output):
        xT, weights, group_locations = ctx.saved_tensors
        gsize = ctx.gsize
        D, B = xT.shape
        O, F = weights.shape
        dtype = weights.dtype
        dev = weights.device
        if grad_output.dtype != dtype:
            grad_output = grad_output.to(dtype)
        dY, lddy = _C.rows_aligned(grad_output)
        locs = group_locations.contiguous()
        W = weights.contiguous()
        stream = _C.stream_of(W)
        code = _C.dtype_code(dtype)

        need_x, need_w = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        need_b = ctx.use_bias and ctx.needs_input_grad[3]

        grad_x = None
        if need_x:
            ws = _C.bwd_features_workspace(B, D, F, O, gsize, dtype, dev)
            if dtype == torch.bfloat16:
                grad_x = torch.empty(B, D, dtype=dtype, device=dev)
                _lib.call("haste_ffi_bwd_features_sr", locs.data_ptr(), W.data_ptr(),
                          dY.data_ptr(), lddy, grad_x.data_ptr(), SR_SEED_GRAD_X, ws.data_ptr(),
                          ws.numel(), B, D, F, O, gsize, code, 0, stream)
            else:
                dxt = torch.empty(D, B, dtype=torch.float32, device=dev)
                _lib.call("haste_ffi_bwd_features", locs.data_ptr(), W.data_ptr(), dY.data_ptr(),
                          lddy, dxt.data_ptr(), ws.data_ptr(), ws.numel(), B, D, F, O, gsize,
                          code, 0, stream)
                grad_x = dxt.t().to(dtype).contiguous()

        grad_w = grad_b = None
        if need_w or need_b:
            ldx = xT.stride(0)
            grad_w = torch.empty(O, F, dtype=ctx.w_grad_dtype, device=dev) if need_w else None
            grad_b = torch.empty(O, dtype=ctx.bias_dtype, device=dev) if need_b else None
            if need_w:
                dw_ptr, dw_code = grad_w.data_ptr(), _C.dtype_code(ctx.w_grad_dtype)
            else:  # bias only: the kernel still needs a dW target
                scratch = torch.empty(O, F, dtype=dtype, device=dev)
                dw_ptr, dw_code = scratch.data_ptr(), code
            _lib.call("haste_ffi_bwd_weights", locs.data_ptr(), xT.data_ptr(), ldx, dY.data_ptr(),
                      lddy, dw_ptr, dw_code, None if grad_b is None else grad_b.data_ptr(),
                      0 if grad_b is None else _C.dtype_code(ctx.bias_dtype), B, D, F, O, gsize,
                      code, stream)
        return grad_x, grad_w, None, grad_b, None
