"""Reference-compatible kernel entry points over the HIP C ABI.

Mirrors the pybind module ``shared_ffi._C`` of the reference
(shared_ffi/ffi_wrapper.cpp:28-45): same function names, argument order,
defaults, output dtypes/shapes and error messages, implemented on
libhaste_ffi.so.  Outputs are allocated with torch's caching allocator on the
input's device; kernels run on torch's current stream (the reference used the
legacy default stream).

Also holds the layout helpers shared by bindings.py / step.py: the HIP kernels
need 16-byte aligned rows (row pitch a multiple of 8 elements) for X^T and the
logits; the grad of the logits may have any row pitch.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch

from . import _lib

_DTYPE_CODE = {torch.bfloat16: _lib.DTYPE_BF16, torch.float16: _lib.DTYPE_F16,
               torch.float32: _lib.DTYPE_F32}


def round8(n: int) -> int:
    return (int(n) + 7) // 8 * 8


def round64(n: int) -> int:
    """Row length in 2-byte elements rounded to 128 bytes (one cache line)."""
    return (int(n) + 63) // 64 * 64


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPE_CODE[dtype]
    except KeyError:
        raise RuntimeError(f"unsupported dtype {dtype}") from None


def stream_of(t: torch.Tensor) -> int:
    """The raw handle of torch's current stream on t's device (what
    torch.cuda.current_stream(t.device).cuda_stream returns, without building a
    Stream object: this runs several times per layer and step)."""
    return torch._C._cuda_getCurrentRawStream(t.device.index)


def require_device(t: torch.Tensor, name: str) -> None:
    if not isinstance(t, torch.Tensor) or not t.is_cuda:
        raise RuntimeError(f"{name} must be a tensor on a HIP device (MI355X); got "
                           f"{'a ' + str(t.device) + ' tensor' if isinstance(t, torch.Tensor) else type(t)}")


def _aligned16(t: torch.Tensor) -> bool:
    return t.data_ptr() % 16 == 0


def rows_aligned(t: torch.Tensor) -> Tuple[torch.Tensor, int]:
    """Return (t2, ld): a 2-D view whose rows start 16-byte aligned (unit
    column stride, row stride ld % 8 == 0), copying into a padded buffer only
    when ``t`` does not already satisfy that."""
    assert t.dim() == 2
    if t.stride(1) == 1 and t.stride(0) % 8 == 0 and t.stride(0) >= t.shape[1] and _aligned16(t):
        return t, t.stride(0)
    ld = round8(t.shape[1])
    buf = torch.empty(t.shape[0], ld, dtype=t.dtype, device=t.device)
    buf[:, : t.shape[1]].copy_(t)
    return buf[:, : t.shape[1]], ld


def grad_rows(t: torch.Tensor) -> Tuple[torch.Tensor, int]:
    """(t2, ld) for the grad of the logits [B, O] handed to a backward: used in
    place when its columns are contiguous (any row stride and alignment; rows
    that do not start on 16-byte boundaries take the kernels' two-chunk loads,
    which cost about what a realigning copy would, without the copy's buffer),
    copied into aligned rows otherwise or when O < 16."""
    assert t.dim() == 2
    if (t.stride(1) == 1 or t.shape[1] == 1) and t.stride(0) >= t.shape[1] and \
            t.data_ptr() % 2 == 0 and (t.shape[1] >= 16 or
                                        (t.stride(0) % 8 == 0 and t.data_ptr() % 16 == 0)):
        return t, t.stride(0)
    return rows_aligned(t)


def padded_transpose(features: torch.Tensor) -> Tuple[torch.Tensor, int]:
    """features [B, D] -> (xT [D, B] view of a [D, round8(B)] buffer, ld), by the
    HIP transpose kernel (padding columns are zero)."""
    B, D = features.shape
    ld = round8(B)
    buf = torch.empty(D, ld, dtype=features.dtype, device=features.device)
    x, ldx = (features, features.stride(0)) if features.stride(1) == 1 else (
        features.contiguous(), D)
    _lib.call("haste_transpose_features", x.data_ptr(), ldx, buf.data_ptr(), ld, B, D,
              stream_of(features))
    return buf[:, :B], ld


def f16_compute(t: torch.Tensor) -> torch.Tensor:
    """An fp32 operand as the reference's fp32 kernels use it: rounded to fp16 to
    nearest (__float2half_rn as they load it, e.g. ffi_forward_kernels.cu:350-356,
    ffi_backward_features.cu:288-303, ffi_backward_weights.cu:352-368); 16-bit
    tensors pass through."""
    return t.to(torch.float16) if t.dtype == torch.float32 else t


def _check_locations(locations: torch.Tensor, L: int, FANIN: int, gsize: int) -> torch.Tensor:
    require_device(locations, "locations")
    Gc = (L + gsize - 1) // gsize
    if locations.dtype != torch.int32:
        raise RuntimeError(f"locations must be int32 (got {locations.dtype})")
    if tuple(locations.shape) != (Gc, FANIN):
        raise RuntimeError(f"locations must be [{Gc}, {FANIN}] for L={L}, gsize={gsize} "
                           f"(got {list(locations.shape)})")
    return locations.contiguous()


def _check_sizes(features: torch.Tensor, weights: torch.Tensor, B: int, H: int, FANIN: int,
                 L: int) -> None:
    if tuple(features.shape) != (H, B):
        raise RuntimeError(f"features must be [H={H}, B={B}] (got {list(features.shape)})")
    if tuple(weights.shape) != (L, FANIN):
        raise RuntimeError(f"weights must be [L={L}, FANIN={FANIN}] (got {list(weights.shape)})")


# ----------------------------------------------------------------------------
# shared_ffi._C.ffi_forward_cuda  (ffi_forward_kernels.cu:492-719)
# ----------------------------------------------------------------------------
def ffi_forward_cuda(locations: torch.Tensor, features: torch.Tensor, weights: torch.Tensor,
                     bias: Optional[torch.Tensor] = None, B: int = None, H: int = None,
                     FANIN: int = None, L: int = None, gsize: int = 32) -> torch.Tensor:
    """Grouped FFI forward.  ``features`` is X^T [H, B]; returns logits [B, L]
    as a view of a [B, ceil64(L)] buffer (the reference's view is of a
    [B, ceil8(L)] buffer; the values and the view's shape are the same)."""
    require_device(features, "features")
    require_device(weights, "weights")
    _check_sizes(features, weights, B, H, FANIN, L)
    if weights.dtype != features.dtype:
        raise RuntimeError("weights dtype must match features dtype")
    locations = _check_locations(locations, L, FANIN, gsize)
    if bias is not None:
        if not (bias.dim() == 1 and bias.size(0) == L):
            raise RuntimeError("bias must be [L]")
        if bias.dtype != features.dtype:
            raise RuntimeError("bias dtype must match features dtype")
        bias = bias.contiguous()
    xT, ldx = rows_aligned(f16_compute(features))
    W = f16_compute(weights).contiguous()
    # rows padded to 128-byte lines (the reference pads to 8 labels): a group's
    # logit row segment is then one line, written whole
    L_pad = round64(L)
    out = torch.empty(B, L_pad, dtype=features.dtype, device=features.device)
    forward_into(locations, xT, ldx, W, bias, out, L_pad, B, H, FANIN, L, gsize,
                 features.dtype, stream_of(features))
    return out if L_pad == L else out.narrow(1, 0, L)


def ffi_forward_f32(locations: torch.Tensor, xT16: torch.Tensor, ldx: int,
                    weights: torch.Tensor, bias: Optional[torch.Tensor], B: int, H: int,
                    FANIN: int, L: int, gsize: int) -> torch.Tensor:
    """ffi_forward_cuda of an fp32 layer whose transposed features are already the
    fp16 copy ``xT16`` ([H, B] rows at stride ldx % 8 == 0, 16-byte aligned):
    fp32 logits [B, L] (a view of a [B, ceil64(L)] buffer)."""
    require_device(weights, "weights")
    if tuple(weights.shape) != (L, FANIN):
        raise RuntimeError(f"weights must be [L={L}, FANIN={FANIN}] (got {list(weights.shape)})")
    if weights.dtype != torch.float32 or xT16.dtype != torch.float16:
        raise RuntimeError("ffi_forward_f32: fp32 weights and fp16 transposed features")
    locations = _check_locations(locations, L, FANIN, gsize)
    if bias is not None:
        if not (bias.dim() == 1 and bias.size(0) == L):
            raise RuntimeError("bias must be [L]")
        if bias.dtype != torch.float32:
            raise RuntimeError("bias dtype must match features dtype")
        bias = bias.contiguous()
    L_pad = round64(L)
    out = torch.empty(B, L_pad, dtype=torch.float32, device=weights.device)
    forward_into(locations, xT16, ldx, f16_compute(weights).contiguous(), bias, out, L_pad, B, H,
                 FANIN, L, gsize, torch.float32, stream_of(weights))
    return out if L_pad == L else out.narrow(1, 0, L)


def forward_into(locations: torch.Tensor, xT: torch.Tensor, ldx: int, W: torch.Tensor,
                 bias: Optional[torch.Tensor], out: torch.Tensor, ldo: int, B: int, D: int,
                 F: int, O: int, G: int, dtype: torch.dtype, stream: int) -> None:
    """The forward kernel on prepared operands: ``dtype`` bf16/fp16 (xT, W, bias and
    out in it) or fp32 (xT and W already rounded to fp16 by f16_compute; bias
    and out fp32, out[:, :O] of a [B, ldo] buffer)."""
    b = None if bias is None else bias.data_ptr()
    if dtype == torch.float32:
        _lib.call("haste_ffi_forward_f16_f32out", locations.data_ptr(), xT.data_ptr(), ldx,
                  W.data_ptr(), b, out.data_ptr(), ldo, B, D, F, O, G, stream)
    else:
        _lib.call("haste_ffi_forward", locations.data_ptr(), xT.data_ptr(), ldx, W.data_ptr(), b,
                  out.data_ptr(), ldo, B, D, F, O, G, dtype_code(dtype), stream)


def bwd_features_workspace(B: int, H: int, FANIN: int, L: int, gsize: int, dtype: torch.dtype,
                           device) -> torch.Tensor:
    n = _lib.lib().haste_ffi_bwd_features_workspace_size(B, H, FANIN, L, gsize, dtype_code(dtype))
    if n < 0:
        raise RuntimeError(_lib.last_error())
    return torch.empty(max(int(n), 16), dtype=torch.uint8, device=device)


# ----------------------------------------------------------------------------
# shared_ffi._C.ffi_backward_features_cuda  (ffi_backward_features.cu:417-633)
# ----------------------------------------------------------------------------
def ffi_backward_features_cuda(features: torch.Tensor, weights: torch.Tensor,
                               locations: torch.Tensor, grad_outputs: torch.Tensor, B: int, H: int,
                               FANIN: int, L: int, gsize: int) -> torch.Tensor:
    """Returns fp32 dX^T [H, B] (deterministic; the reference used atomics)."""
    require_device(weights, "weights")
    require_device(grad_outputs, "grad_outputs")
    _check_sizes(features, weights, B, H, FANIN, L)
    locations = _check_locations(locations, L, FANIN, gsize)
    if tuple(grad_outputs.shape) != (B, L):
        raise RuntimeError(f"grad_outputs must be [B={B}, L={L}] (got {list(grad_outputs.shape)})")
    if grad_outputs.dtype != weights.dtype:
        raise RuntimeError("grad_outputs dtype must match weights dtype")
    dY, lddy = grad_rows(f16_compute(grad_outputs))
    W = f16_compute(weights).contiguous()
    ws = bwd_features_workspace(B, H, FANIN, L, gsize, W.dtype, weights.device)
    out = torch.empty(H, B, dtype=torch.float32, device=weights.device)
    _lib.call("haste_ffi_bwd_features", locations.data_ptr(), W.data_ptr(), dY.data_ptr(), lddy,
              out.data_ptr(), ws.data_ptr(), ws.numel(), B, H, FANIN, L, gsize,
              dtype_code(W.dtype), 0, stream_of(weights))
    return out


# ----------------------------------------------------------------------------
# shared_ffi._C.ffi_backward_weights_cuda  (ffi_backward_weights.cu:486-684)
# ----------------------------------------------------------------------------
def ffi_backward_weights_cuda(features: torch.Tensor, weights: torch.Tensor,
                              locations: torch.Tensor, grad_outputs: torch.Tensor, B: int, H: int,
                              FANIN: int, L: int, gsize: int) -> torch.Tensor:
    """Returns dW [L, FANIN] in the features dtype (RNE of the fp32 sum; for fp32
    features the fp32 sum of the fp16-rounded operands, as the reference)."""
    require_device(features, "features")
    require_device(grad_outputs, "grad_outputs")
    _check_sizes(features, weights, B, H, FANIN, L)
    locations = _check_locations(locations, L, FANIN, gsize)
    if tuple(grad_outputs.shape) != (B, L):
        raise RuntimeError(f"grad_outputs must be [B={B}, L={L}] (got {list(grad_outputs.shape)})")
    xT, ldx = rows_aligned(f16_compute(features))
    dY, lddy = grad_rows(f16_compute(grad_outputs).to(xT.dtype))
    dW = torch.empty(L, FANIN, dtype=features.dtype, device=features.device)
    _lib.call("haste_ffi_bwd_weights", locations.data_ptr(), xT.data_ptr(), ldx, dY.data_ptr(),
              lddy, dW.data_ptr(), dtype_code(features.dtype), None, 0, B, H, FANIN, L, gsize,
              dtype_code(xT.dtype), stream_of(features))
    return dW
