"""One training step of a grouped FFI layer on preallocated buffers.

``FFITrainStep`` runs forward -> backward (features, weights, bias) -> fused
SR-SGD update of weights and bias, calling libhaste_ffi.so directly with
buffers allocated once, so a step launches only HIP kernels (no allocator
traffic, no host sync) and can be captured in a HIP graph.  It computes the
same quantities as GroupFFIMulFunction + SRSgd with two deliberate choices:
the weight and bias gradients are kept in fp32 (``grad_dtype``, the SGD kernel
reads them directly), and the grad of the logits ``dY`` is an input.
"""
from __future__ import annotations

import torch

from . import _C, _lib
from .bindings import SR_SEED_GRAD_X


class FFITrainStep:
    def __init__(self, weights: torch.Tensor, bias, group_locations: torch.Tensor, batch: int,
                 in_features: int, group_size: int, lr: float, weight_decay: float,
                 seed: int = 42, grad_dtype: torch.dtype = torch.float32):
        _C.require_device(weights, "weights")
        if weights.dtype != torch.bfloat16:
            raise NotImplementedError("FFITrainStep: bf16 weights only")
        self.W = weights
        self.bias = bias
        self.idx = group_locations
        self.B, self.D, self.G = int(batch), int(in_features), int(group_size)
        self.O, self.F = weights.shape
        self.lr, self.wd, self.seed = float(lr), float(weight_decay), int(seed)
        dev = weights.device
        # rows of X^T, logits and dY start on 128-byte lines, so a group's row
        # segment (G labels) never straddles two cache lines
        self.ldx = _C.round64(self.B)
        self.ldo = _C.round64(self.O)
        self.xT_buf = torch.zeros(self.D, self.ldx, dtype=torch.bfloat16, device=dev)
        self.logits_buf = torch.empty(self.B, self.ldo, dtype=torch.bfloat16, device=dev)
        self.dX = torch.empty(self.B, self.D, dtype=torch.bfloat16, device=dev)
        self.grad_dtype = grad_dtype
        self.dW = torch.empty(self.O, self.F, dtype=grad_dtype, device=dev)
        self.dbias = torch.empty(self.O, dtype=grad_dtype, device=dev) if bias is not None else None
        self.ws = _C.bwd_features_workspace(self.B, self.D, self.F, self.O, self.G,
                                            torch.bfloat16, dev)
        self._plan_version = None  # idx._version the workspace plan was made for
        self.code = _lib.DTYPE_BF16
        self.gcode = _C.dtype_code(grad_dtype)
        ts = [(self.W, self.dW)] + ([(bias, self.dbias)] if bias is not None else [])
        self._sgd_tensors = (_lib.SgdTensor * len(ts))(
            *[_lib.SgdTensor(w.data_ptr(), g.data_ptr(), None, w.numel(), 0) for w, g in ts])
        self._sgd_args = [self._sgd_tensors, len(ts), self.gcode, self.lr, self.wd, 0.0, 0, 1,
                          self.seed, _C.stream_of(self.W)]

    @property
    def logits(self) -> torch.Tensor:
        return self.logits_buf[:, : self.O]

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        """x [B, D] bf16 -> logits [B, O] (view of a [B, ldo] buffer)."""
        if tuple(x.shape) != (self.B, self.D) or x.dtype != torch.bfloat16:
            raise ValueError(f"FFITrainStep.forward: x must be bf16 [{self.B}, {self.D}] "
                             f"(got {x.dtype} {list(x.shape)})")
        _C.require_device(x, "x")
        if x.stride(1) != 1:
            x = x.contiguous()
        _lib.call("haste_transpose_features", x.data_ptr(), x.stride(0), self.xT_buf.data_ptr(),
                  self.ldx, self.B, self.D, _C.stream_of(self.W))
        _lib.call("haste_ffi_forward", self.idx.data_ptr(), self.xT_buf.data_ptr(), self.ldx,
                  self.W.data_ptr(), None if self.bias is None else self.bias.data_ptr(),
                  self.logits_buf.data_ptr(), self.ldo, self.B, self.D, self.F, self.O, self.G,
                  self.code, _C.stream_of(self.W))
        return self.logits

    def _check_dY(self, dY: torch.Tensor, lddy: int) -> None:
        _C.require_device(dY, "dY")
        if (dY.dtype != torch.bfloat16 or lddy % 8 or lddy < self.O
                or dY.numel() < (self.B - 1) * lddy + self.O):
            raise ValueError(f"FFITrainStep: dY must be a bf16 buffer of {self.B} rows of "
                             f"stride lddy >= {self.O}, lddy % 8 == 0 (got {dY.dtype}, "
                             f"{dY.numel()} elements, lddy={lddy})")

    def backward_features(self, dY: torch.Tensor, lddy: int) -> None:
        """dX [B, D] bf16 = SR(feature gradient, seed 123) (bindings.py:44-48)."""
        self._check_dY(dY, lddy)
        # the index plan depends on idx only: rebuilt when idx changes (rewire)
        ready = int(self._plan_version == self.idx._version)
        _lib.call("haste_ffi_bwd_features_sr", self.idx.data_ptr(), self.W.data_ptr(),
                  dY.data_ptr(), lddy, self.dX.data_ptr(), SR_SEED_GRAD_X, self.ws.data_ptr(),
                  self.ws.numel(), self.B, self.D, self.F, self.O, self.G, self.code, ready,
                  _C.stream_of(self.W))
        self._plan_version = self.idx._version

    def backward_weights(self, dY: torch.Tensor, lddy: int) -> None:
        """dW [O, F] and dbias [O] in grad_dtype."""
        self._check_dY(dY, lddy)
        _lib.call("haste_ffi_bwd_weights", self.idx.data_ptr(), self.xT_buf.data_ptr(), self.ldx,
                  dY.data_ptr(), lddy, self.dW.data_ptr(), self.gcode,
                  None if self.dbias is None else self.dbias.data_ptr(), self.gcode, self.B,
                  self.D, self.F, self.O, self.G, self.code, _C.stream_of(self.W))

    def backward(self, dY: torch.Tensor, lddy: int) -> None:
        """dY: [B, lddy] bf16 buffer (lddy % 8 == 0) holding grad of the logits."""
        self.backward_features(dY, lddy)
        self.backward_weights(dY, lddy)

    def sgd(self) -> None:
        """SR-SGD (momentum 0) on weights and bias with the current seed, then seed += 1
        (optim_sr.py:59-62: one seed per step, offsets from 0 per tensor); one launch."""
        self._sgd_args[-2] = self.seed
        self._sgd_args[-1] = _C.stream_of(self.W)
        _lib.call("haste_sgd_sr_step_multi", *self._sgd_args)
        self.seed += 1

    def step(self, x: torch.Tensor, dY: torch.Tensor, lddy: int) -> None:
        self.forward(x)
        self.backward(dY, lddy)
        self.sgd()
