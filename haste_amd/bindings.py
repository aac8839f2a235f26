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

import collections
import weakref
from typing import Any, Optional

import torch

from . import _C, _lib

SR_SEED_GRAD_X = 123  # bindings.py:48


def _grad_dtype(p: torch.Tensor) -> torch.dtype:
    """dtype autograd will store for p.grad: p.grad_dtype if set (torch >= 2.10), else p.dtype."""
    gd = getattr(p, "grad_dtype", None)
    return gd if gd is not None else p.dtype


# Feature-gradient workspaces reused across backward calls, one per layer: the
# index plan in a workspace depends on group_locations only, so a call with the
# same index tensor (same object, unchanged version counter: a rewire bumps it)
# skips rebuilding it.  Keyed by the index tensor's address (a layer) and by
# shape, dtype, device and stream (a workspace's partial sums are written and
# read in stream order); the _WS_CACHE_SIZE most recently used are kept, so a
# model with up to that many FFI layers never rebuilds a plan it had.
class _Workspace:
    __slots__ = ("ws", "dims", "stream", "locs", "locs_version", "locs_ptr", "wt_ptr",
                 "wt_version", "bias", "__weakref__")

    def __init__(self, ws, dims, stream):
        self.ws, self.dims, self.stream = ws, dims, stream
        self.locs = None          # weakref to the index tensor of the plan
        self.locs_version = -1
        self.locs_ptr = 0
        self.wt_ptr = 0           # (data_ptr, version) of the weights whose W^T an
        self.wt_version = -1      # optimizer step wrote into the workspace, if any
        self.bias = None          # weakref to the layer's bias (its last backward), or None

    def plan_valid(self, locs) -> bool:
        return (self.locs is not None and self.locs() is locs
                and self.locs_version == locs._version and self.locs_ptr == locs.data_ptr())

    def wt_valid(self, W) -> bool:
        return self.wt_ptr == W.data_ptr() and self.wt_version == W._version


_WS_CACHE: "collections.OrderedDict[tuple, _Workspace]" = collections.OrderedDict()
_WS_CACHE_SIZE = 4
# weights data_ptr -> the workspace whose plan was last used with them, so that
# SRSgd can refresh its transposed weights while it updates them (the next
# backward then skips the gather)
_WT_TARGETS: "weakref.WeakValueDictionary[int, _Workspace]" = weakref.WeakValueDictionary()


def _bwdf_workspace(locs: torch.Tensor, B: int, D: int, F: int, O: int, gsize: int,
                    dtype: torch.dtype, stream: int) -> _Workspace:
    key = (locs.data_ptr(), locs.device, B, D, F, O, gsize, dtype, stream)
    ent = _WS_CACHE.get(key)
    if ent is None:
        ent = _Workspace(_C.bwd_features_workspace(B, D, F, O, gsize, dtype, locs.device),
                         (B, D, F, O, gsize), stream)
        _WS_CACHE[key] = ent
        while len(_WS_CACHE) > _WS_CACHE_SIZE:
            _WS_CACHE.popitem(last=False)
    _WS_CACHE.move_to_end(key)
    return ent


def mark_wt_refreshed(ent: _Workspace, weights: torch.Tensor) -> None:
    """The workspace now holds the transposed weights of ``weights`` as they are."""
    ent.wt_ptr, ent.wt_version = weights.data_ptr(), weights._version


def clear_wt_refreshed(weights: Optional[torch.Tensor] = None) -> None:
    """Forget the refreshed transposed-weight copy of ``weights`` (of every
    layer when None): the next backward gathers W^T from the weights again."""
    for ent in _WS_CACHE.values():
        if weights is None or ent.wt_ptr == weights.data_ptr():
            ent.wt_ptr, ent.wt_version = 0, -1


def wt_target(weights: torch.Tensor):
    """The workspace (if any) whose plan the last backward of ``weights`` used and
    whose index tensor is unchanged since: an optimizer that updates these
    weights may refresh its transposed weights (haste_sgd_sr_step_wt) and then
    call ``mark_wt_refreshed``.  The reuse is keyed on the weights' version
    counter: changes made through ``.data`` do not move it, so code that edits
    the weights that way between an optimizer step and the next backward must
    call ``clear_wt_refreshed`` (or build SRSgd with refresh_transposed=False)."""
    ent = _WT_TARGETS.get(weights.data_ptr())
    if ent is None or ent.locs is None:
        return None
    locs = ent.locs()
    if locs is None or not ent.plan_valid(locs):
        return None
    return ent


def _ffi_grads(xT: torch.Tensor, weights: torch.Tensor, group_locations: torch.Tensor,
               gsize: int, grad_output: torch.Tensor, need_x: bool, need_w: bool, need_b: bool,
               w_grad_dtype: torch.dtype, bias_dtype: Optional[torch.dtype], bias_ref=None):
    """(grad_x, grad_w, grad_b) of the grouped FFI layer for grad_output [B, O]
    (read in place at any row stride when its columns are contiguous)."""
    D, B = xT.shape
    O, F = weights.shape
    dtype = weights.dtype
    dev = weights.device
    if grad_output.dtype != dtype:
        grad_output = grad_output.to(dtype)
    # an fp32 layer computes with fp16 copies of W, X and grad_output, as the
    # reference's fp32 kernels round them when they load them
    f32 = dtype == torch.float32
    dY, lddy = _C.grad_rows(_C.f16_compute(grad_output))
    locs = group_locations.contiguous()
    W = _C.f16_compute(weights).contiguous()
    stream = _C.stream_of(W)
    code = _C.dtype_code(W.dtype)

    grad_x = None
    # bf16 layer with weight or bias gradients too: dX is finished by the
    # weight-gradient launch (haste_ffi_bwd_weights_dx) instead of a reduce kernel
    dx_in_w = need_x and dtype == torch.bfloat16 and (need_w or need_b)
    if need_x:
        ent = _bwdf_workspace(locs, B, D, F, O, gsize, W.dtype, stream)
        ws = ent.ws
        # 1: the plan is current; 2: the transposed weights too (written by the
        # SRSgd step that last updated these weights, haste_sgd_sr_step_wt, and
        # the weights' version counter has not moved since)
        ready = 0
        if ent.plan_valid(locs):
            ready = 2 if ent.wt_valid(W) else 1
        if dx_in_w:
            grad_x = torch.empty(B, D, dtype=dtype, device=dev)
            _lib.call("haste_ffi_bwd_features_partials", locs.data_ptr(), W.data_ptr(),
                      dY.data_ptr(), lddy, ws.data_ptr(), ws.numel(), B, D, F, O, gsize, code,
                      ready, stream)
        elif dtype == torch.bfloat16:
            grad_x = torch.empty(B, D, dtype=dtype, device=dev)
            _lib.call("haste_ffi_bwd_features_sr", locs.data_ptr(), W.data_ptr(),
                      dY.data_ptr(), lddy, grad_x.data_ptr(), SR_SEED_GRAD_X, ws.data_ptr(),
                      ws.numel(), B, D, F, O, gsize, code, ready, stream)
        else:
            dxt = torch.empty(D, B, dtype=torch.float32, device=dev)
            _lib.call("haste_ffi_bwd_features", locs.data_ptr(), W.data_ptr(), dY.data_ptr(),
                      lddy, dxt.data_ptr(), ws.data_ptr(), ws.numel(), B, D, F, O, gsize,
                      code, ready, stream)
            grad_x = dxt.t().to(dtype).contiguous()
        ent.locs, ent.locs_version, ent.locs_ptr = weakref.ref(locs), locs._version, locs.data_ptr()
        if W is weights and dtype == torch.bfloat16:
            _WT_TARGETS[W.data_ptr()] = ent
            ent.bias = bias_ref

    grad_w = grad_b = None
    if f32 and need_b:
        # the reference's torch.sum(grad_output, dim=0) in fp32 (bindings.py:40),
        # not the kernel's sum of the fp16 copy
        grad_b = grad_output.sum(0).to(bias_dtype)
        need_b = False
    if need_w or need_b:
        xT, ldx = _C.rows_aligned(_C.f16_compute(xT))
        grad_w = torch.empty(O, F, dtype=w_grad_dtype, device=dev) if need_w else None
        if need_b:
            grad_b = torch.empty(O, dtype=bias_dtype, device=dev)
        if need_w:
            dw_ptr, dw_code = grad_w.data_ptr(), _C.dtype_code(w_grad_dtype)
        else:  # bias only: the kernel still needs a dW target
            scratch = torch.empty(O, F, dtype=W.dtype, device=dev)
            dw_ptr, dw_code = scratch.data_ptr(), code
        if dx_in_w:
            _lib.call("haste_ffi_bwd_weights_dx", locs.data_ptr(), xT.data_ptr(), ldx,
                      dY.data_ptr(), lddy, dw_ptr, dw_code, grad_b.data_ptr() if need_b else None,
                      _C.dtype_code(bias_dtype) if need_b else 0, grad_x.data_ptr(),
                      SR_SEED_GRAD_X, ws.data_ptr(), ws.numel(), B, D, F, O, gsize, code,
                      stream)
        else:
            _lib.call("haste_ffi_bwd_weights", locs.data_ptr(), xT.data_ptr(), ldx,
                      dY.data_ptr(), lddy, dw_ptr, dw_code, grad_b.data_ptr() if need_b else None,
                      _C.dtype_code(bias_dtype) if need_b else 0, B, D, F, O, gsize, code,
                      stream)
    return grad_x, grad_w, grad_b


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
        # bindings.py:19, rows padded to 8; an fp32 layer keeps the fp16 copy its
        # kernels compute with (the reference's fp32 kernels round X as they load it)
        xT, ldx = _C.padded_transpose(_C.f16_compute(features))
        if features.dtype == torch.float32:
            out = _C.ffi_forward_f32(group_locations, xT, ldx, weights, bias, B, D, F, O, gsize)
        else:
            out = _C.ffi_forward_cuda(group_locations, xT, weights, bias, B, D, F, O, gsize)
        ctx.save_for_backward(xT, weights, group_locations)
        ctx.gsize = int(gsize)
        ctx.use_bias = bias is not None
        ctx.w_grad_dtype = _grad_dtype(weights)
        ctx.bias_dtype = _grad_dtype(bias) if bias is not None else None
        # the layer's bias, so that SRSgd can step it in its weights' launch
        ctx.bias_ref = weakref.ref(bias) if bias is not None else None
        return out

    @staticmethod
    @torch.amp.custom_bwd(device_type="cuda")
    def backward(ctx, grad_output):
        xT, weights, group_locations = ctx.saved_tensors
        grad_x, grad_w, grad_b = _ffi_grads(
            xT, weights, group_locations, ctx.gsize, grad_output, ctx.needs_input_grad[0],
            ctx.needs_input_grad[1], ctx.use_bias and ctx.needs_input_grad[3], ctx.w_grad_dtype,
            ctx.bias_dtype, ctx.bias_ref)
        return grad_x, grad_w, None, grad_b, None


class HeadTailFFIFunction(torch.autograd.Function):
    """torch.cat((head(x_head), ffi(x_tail)), dim=1) of the head/tail split model
    (src/model.py:227-232,245-248: a dense nn.Linear head and an FFI tail), built
    in one [B, H + O] buffer: the FFI kernel writes the tail logits in place (the
    view starts at the column that puts the tail's rows on 128-byte lines), so
    the forward never copies the B x O tail, and the backward reads the tail's
    columns of grad_output in place.  Values are those of the torch.cat
    formulation: the same head op (F.linear) and FFI kernels."""

    @staticmethod
    @torch.amp.custom_fwd(device_type="cuda")
    def forward(ctx: Any, x_head: torch.Tensor, head_weight: torch.Tensor,
                head_bias: Optional[torch.Tensor], x_tail: torch.Tensor, weights: torch.Tensor,
                group_locations: torch.Tensor, bias: Optional[torch.Tensor],
                gsize: int = 32) -> torch.Tensor:
        _C.require_device(x_tail, "x_tail")
        if x_tail.dim() != 2 or x_head.dim() != 2 or x_head.shape[0] != x_tail.shape[0]:
            raise RuntimeError("x_head and x_tail must be 2-D with the same batch size")
        B, D = x_tail.shape
        O, F = weights.shape
        H = head_weight.shape[0]
        dt = x_tail.dtype
        head = torch.nn.functional.linear(x_head, head_weight, head_bias).to(dt)
        s0 = (64 - H % 64) % 64                    # tail rows start on 128-byte lines
        ld = _C.round64(s0 + H + O)
        buf = torch.empty(B, ld, dtype=dt, device=x_tail.device)
        out = buf[:, s0: s0 + H + O]
        out[:, :H].copy_(head)
        xT, ldx = _C.padded_transpose(_C.f16_compute(x_tail))
        locs = _C._check_locations(group_locations, O, F, gsize)
        if weights.dtype != dt or (bias is not None and bias.dtype != dt):
            raise RuntimeError("weights and bias dtype must match x_tail's")
        W = _C.f16_compute(weights).contiguous()
        b = None if bias is None else bias.contiguous()
        _C.forward_into(locs, xT, ldx, W, b, buf[:, s0 + H:], ld, B, D, F, O, gsize, dt,
                        _C.stream_of(x_tail))
        ctx.save_for_backward(x_head, head_weight, xT, weights, group_locations)
        ctx.H, ctx.gsize = H, int(gsize)
        ctx.head_has_bias = head_bias is not None
        ctx.use_bias = bias is not None
        ctx.w_grad_dtype = _grad_dtype(weights)
        ctx.bias_dtype = _grad_dtype(bias) if bias is not None else None
        ctx.bias_ref = weakref.ref(bias) if bias is not None else None
        return out

    @staticmethod
    @torch.amp.custom_bwd(device_type="cuda")
    def backward(ctx, grad_output):
        x_head, head_weight, xT, weights, group_locations = ctx.saved_tensors
        H = ctx.H
        gh = grad_output[:, :H]
        n = ctx.needs_input_grad
        gx_h = gh.to(head_weight.dtype) @ head_weight if n[0] else None
        gw_h = gh.t().to(x_head.dtype) @ x_head if n[1] else None
        gb_h = gh.sum(0) if (ctx.head_has_bias and n[2]) else None
        gx_t, gw_t, gb_t = _ffi_grads(xT, weights, group_locations, ctx.gsize,
                                      grad_output[:, H:], n[3], n[4], ctx.use_bias and n[6],
                                      ctx.w_grad_dtype, ctx.bias_dtype, ctx.bias_ref)
        return gx_h, gw_h, gb_h, gx_t, gw_t, None, gb_t, None
