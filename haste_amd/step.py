"""One training step of a grouped FFI layer on preallocated buffers.

``FFITrainStep`` runs forward -> backward to features -> backward to weights
and bias fused with the SR-SGD update of weights and bias, calling
libhaste_ffi.so directly with buffers allocated once, so a step launches only
HIP kernels (no allocator traffic, no host sync).  With ``device_seed=True`` the
SR-SGD seed lives in device memory and the fused update advances it there, so
``step`` (and ``step_bce``) can be captured once in a HIP graph
(torch.cuda.graph) and replayed step after step with the seed += 1 schedule;
otherwise the seed is a launch argument, and a captured step would replay the
seed it was captured with.  It computes the same quantities as GroupFFIMulFunction + SRSgd with
two deliberate choices: the weight and bias gradients are fp32 (``grad_dtype``)
and, in ``step``, never leave the chip (the SGD update is applied in the
epilogue of the weight-gradient kernel; the result is bit-identical to
``backward_weights`` followed by ``sgd``), and the grad of the logits ``dY`` is
an input.

The step keeps the transposed weights of the bwd-features workspace valid
across steps by the version counter of ``weights``: pass the tensor through
which the weights are changed (the Parameter itself, not ``.data``, whose
version counter is separate) so that a change made outside the step is seen.
"""
from __future__ import annotations

import torch

from . import _C, _lib
from .bindings import SR_SEED_GRAD_X


class FFITrainStep:
    def __init__(self, weights: torch.Tensor, bias, group_locations: torch.Tensor, batch: int,
                 in_features: int, group_size: int, lr: float, weight_decay: float,
                 seed: int = 42, grad_dtype: torch.dtype = torch.float32,
                 device_seed: bool = False):
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
        self._dW = None      # allocated by the first unfused backward_weights call
        self._dbias = None
        self.ws = _C.bwd_features_workspace(self.B, self.D, self.F, self.O, self.G,
                                            torch.bfloat16, dev)
        self._plan_version = None  # idx._version the workspace plan was made for
        # W._version for which the workspace holds W^T of the current weights
        # (written by backward_features, or by backward_weights_sgd for the weights
        # it updates); None when stale
        self._wt_version = None
        self._dx_pending = False  # backward_features(defer_dx=True) left dX to the weight update
        self.bce_ws = None   # forward_bce's label bits + loss partials (allocated on first use)
        self.dY_buf = None
        self.loss_buf = None
        self.code = _lib.DTYPE_BF16
        self.gcode = _C.dtype_code(grad_dtype)
        self._sgd_args = None
        # device_seed: the fused update's seed, read and advanced on the device
        self._seed_dev = (torch.tensor([self.seed], dtype=torch.int64, device=dev)
                          if device_seed else None)

    def state_dict(self) -> dict:
        """The step's own state (the parameters W, bias and idx belong to the caller):
        the SR seed the next update will use (device_seed: read from the device,
        a sync)."""
        return {"seed": self.current_seed()}

    def load_state_dict(self, state: dict) -> None:
        self.seed = int(state["seed"])
        if self._seed_dev is not None:
            self._seed_dev.fill_(self.seed)

    def current_seed(self) -> int:
        """The seed the next SGD update uses (device_seed: a device sync)."""
        return int(self._seed_dev.item()) if self._seed_dev is not None else int(self.seed)

    @property
    def dW(self) -> torch.Tensor:
        """[O, F] weight gradient of the last ``backward_weights`` call."""
        self._grad_buffers()
        return self._dW

    @property
    def dbias(self):
        self._grad_buffers()
        return self._dbias

    def _grad_buffers(self) -> None:
        if self._dW is not None:
            return
        dev = self.W.device
        self._dW = torch.empty(self.O, self.F, dtype=self.grad_dtype, device=dev)
        if self.bias is not None:
            self._dbias = torch.empty(self.O, dtype=self.grad_dtype, device=dev)
        ts = [(self.W, self._dW)] + ([(self.bias, self._dbias)] if self.bias is not None else [])
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

    def forward_bce(self, x: torch.Tensor, labels: torch.Tensor,
                    write_logits: bool = False) -> torch.Tensor:
        """Forward fused with the sparse BCE loss (src/runner.py:469-478): ``labels``
        is the COO [nnz, 2] int32 (row, label) list of positives.  Writes
        dY = sigma(logits) - Y into ``dY_buf`` ([B, ldo]; the logits into
        ``logits_buf`` too when ``write_logits``) and returns the summed loss as a
        0-d fp32 tensor (computed on the device, no host sync)."""
        if tuple(x.shape) != (self.B, self.D) or x.dtype != torch.bfloat16:
            raise ValueError(f"FFITrainStep.forward_bce: x must be bf16 [{self.B}, {self.D}] "
                             f"(got {x.dtype} {list(x.shape)})")
        _C.require_device(x, "x")
        _C.require_device(labels, "labels")
        if labels.dtype != torch.int32 or labels.dim() != 2 or labels.shape[1] != 2:
            raise ValueError("FFITrainStep.forward_bce: labels must be int32 [nnz, 2] (row, label)")
        labels = labels.contiguous()
        if x.stride(1) != 1:
            x = x.contiguous()
        if self.bce_ws is None:
            n = _lib.lib().haste_ffi_forward_bce_workspace_size(self.B, self.O, self.G)
            if n < 0:
                raise ValueError("FFITrainStep.forward_bce: unsupported shape")
            self.bce_ws = torch.zeros(n, dtype=torch.uint8, device=self.W.device)
            self.dY_buf = torch.zeros(self.B, self.ldo, dtype=torch.bfloat16, device=self.W.device)
            self.loss_buf = torch.zeros((), dtype=torch.float32, device=self.W.device)
        st = _C.stream_of(self.W)
        _lib.call("haste_transpose_features", x.data_ptr(), x.stride(0), self.xT_buf.data_ptr(),
                  self.ldx, self.B, self.D, st)
        _lib.call("haste_ffi_forward_bce", self.idx.data_ptr(), self.xT_buf.data_ptr(), self.ldx,
                  self.W.data_ptr(), None if self.bias is None else self.bias.data_ptr(),
                  labels.data_ptr(), labels.shape[0], self.dY_buf.data_ptr(), self.ldo,
                  self.logits_buf.data_ptr() if write_logits else None, self.loss_buf.data_ptr(),
                  self.bce_ws.data_ptr(), self.bce_ws.numel(), self.B, self.D, self.F, self.O,
                  self.G, self.code, st)
        return self.loss_buf

    def step_bce(self, x: torch.Tensor, labels: torch.Tensor) -> torch.Tensor:
        """A training step with the loss fused into the forward: forward + BCE
        gradient -> backward to features (dX) -> fused weight/bias gradient +
        SR-SGD.  Returns the loss (0-d fp32 device tensor) of the step's forward."""
        loss = self.forward_bce(x, labels)
        self.backward_features(self.dY_buf, self.ldo, defer_dx=True)
        self.backward_weights_sgd(self.dY_buf, self.ldo)
        return loss

    def _check_dY(self, dY: torch.Tensor, lddy: int) -> None:
        _C.require_device(dY, "dY")
        if (dY.dtype != torch.bfloat16 or lddy < self.O or (lddy % 8 and self.O < 8)
                or dY.numel() < (self.B - 1) * lddy + self.O):
            raise ValueError(f"FFITrainStep: dY must be a bf16 buffer of {self.B} rows of "
                             f"stride lddy >= {self.O} (a multiple of 8 when O < 8; got "
                             f"{dY.dtype}, {dY.numel()} elements, lddy={lddy})")

    def backward_features(self, dY: torch.Tensor, lddy: int, defer_dx: bool = False) -> None:
        """dX [B, D] bf16 = SR(feature gradient, seed 123) (bindings.py:44-48).
        ``defer_dx``: leave the per-slice partial sums in the workspace; the next
        ``backward_weights_sgd`` writes dX from them in its own launch (the final
        pass then fills the tail of the weight update instead of being a kernel of
        its own).  dX is not valid in between."""
        self._check_dY(dY, lddy)
        # the index plan depends on idx only: rebuilt when idx changes (rewire);
        # W^T is reused when the last fused weight update wrote it for these weights
        ready = 0
        if self._plan_version == self.idx._version:
            ready = 2 if self._wt_version == self.W._version else 1
        if defer_dx:
            _lib.call("haste_ffi_bwd_features_partials", self.idx.data_ptr(), self.W.data_ptr(),
                      dY.data_ptr(), lddy, self.ws.data_ptr(), self.ws.numel(), self.B, self.D,
                      self.F, self.O, self.G, self.code, ready, _C.stream_of(self.W))
        else:
            _lib.call("haste_ffi_bwd_features_sr", self.idx.data_ptr(), self.W.data_ptr(),
                      dY.data_ptr(), lddy, self.dX.data_ptr(), SR_SEED_GRAD_X, self.ws.data_ptr(),
                      self.ws.numel(), self.B, self.D, self.F, self.O, self.G, self.code, ready,
                      _C.stream_of(self.W))
        self._dx_pending = defer_dx
        self._plan_version = self.idx._version
        self._wt_version = self.W._version

    def backward_weights(self, dY: torch.Tensor, lddy: int) -> None:
        """dW [O, F] and dbias [O] in grad_dtype."""
        self._check_dY(dY, lddy)
        if self._dx_pending:
            raise RuntimeError("FFITrainStep.backward_weights: dX of backward_features("
                               "defer_dx=True) is finished by backward_weights_sgd only")
        self._grad_buffers()
        _lib.call("haste_ffi_bwd_weights", self.idx.data_ptr(), self.xT_buf.data_ptr(), self.ldx,
                  dY.data_ptr(), lddy, self.dW.data_ptr(), self.gcode,
                  None if self.dbias is None else self.dbias.data_ptr(), self.gcode, self.B,
                  self.D, self.F, self.O, self.G, self.code, _C.stream_of(self.W))

    def backward(self, dY: torch.Tensor, lddy: int) -> None:
        """dY: [B, lddy] bf16 buffer holding grad of the logits (the last row may end at O)."""
        self.backward_features(dY, lddy)
        self.backward_weights(dY, lddy)

    def sgd(self) -> None:
        """SR-SGD (momentum 0) on weights and bias with the current seed, then seed += 1
        (optim_sr.py:59-62: one seed per step, offsets from 0 per tensor); one launch.
        Applies the gradients of the last ``backward_weights`` call."""
        self._grad_buffers()
        if self._seed_dev is not None:
            self.seed = self.current_seed()
        self._sgd_args[-2] = self.seed
        self._sgd_args[-1] = _C.stream_of(self.W)
        _lib.call("haste_sgd_sr_step_multi", *self._sgd_args)
        torch.autograd.graph.increment_version(self.W)
        self._wt_version = None  # W changed, W^T not refreshed
        self.seed += 1
        if self._seed_dev is not None:
            self._seed_dev.add_(1)

    def backward_weights_sgd(self, dY: torch.Tensor, lddy: int) -> None:
        """Weight and bias gradients (fp32, kept on chip) applied at once by SR-SGD
        (momentum 0) with the current seed, then seed += 1: bit-identical to
        ``backward_weights`` + ``sgd`` with fp32 gradients, in one kernel.  After
        ``backward_features(defer_dx=True)`` the same launch also writes dX."""
        self._check_dY(dY, lddy)
        if self.grad_dtype != torch.float32:
            raise ValueError("FFITrainStep.backward_weights_sgd: the fused update uses fp32 "
                             "gradients (grad_dtype=torch.float32)")
        # refresh W^T in the bwd-features workspace when its plan matches idx
        plan_ok = self._plan_version == self.idx._version
        bias = None if self.bias is None else self.bias.data_ptr()
        if self._seed_dev is not None and not self._dx_pending:
            raise ValueError("FFITrainStep(device_seed=True).backward_weights_sgd follows "
                             "backward_features(defer_dx=True) (as step and step_bce do)")
        if self._dx_pending and self._seed_dev is not None:
            if not plan_ok:
                raise RuntimeError("FFITrainStep.backward_weights_sgd: idx changed after "
                                   "backward_features(defer_dx=True)")
            _lib.call("haste_ffi_bwd_weights_sgd_dx_dev_seed", self.idx.data_ptr(),
                      self.xT_buf.data_ptr(), self.ldx, dY.data_ptr(), lddy, self.W.data_ptr(),
                      bias, None, None, self.lr, self.wd, 0.0, 0, 1, self._seed_dev.data_ptr(),
                      self.dX.data_ptr(), SR_SEED_GRAD_X, self.ws.data_ptr(), self.ws.numel(),
                      self.B, self.D, self.F, self.O, self.G, self.code, _C.stream_of(self.W))
            self._dx_pending = False
        elif self._dx_pending:
            if not plan_ok:
                raise RuntimeError("FFITrainStep.backward_weights_sgd: idx changed after "
                                   "backward_features(defer_dx=True)")
            _lib.call("haste_ffi_bwd_weights_sgd_dx", self.idx.data_ptr(), self.xT_buf.data_ptr(),
                      self.ldx, dY.data_ptr(), lddy, self.W.data_ptr(), bias, None, None, self.lr,
                      self.wd, 0.0, 0, 1, self.seed, self.dX.data_ptr(), SR_SEED_GRAD_X,
                      self.ws.data_ptr(), self.ws.numel(), self.B, self.D, self.F, self.O, self.G,
                      self.code, _C.stream_of(self.W))
            self._dx_pending = False
        else:
            _lib.call("haste_ffi_bwd_weights_sgd", self.idx.data_ptr(), self.xT_buf.data_ptr(),
                      self.ldx, dY.data_ptr(), lddy, self.W.data_ptr(), bias, None, None, None,
                      _lib.DTYPE_F32, None, _lib.DTYPE_F32, self.lr, self.wd, 0.0, 0, 1,
                      self.seed, self.ws.data_ptr() if plan_ok else None,
                      self.ws.numel() if plan_ok else 0, self.B, self.D, self.F, self.O, self.G,
                      self.code, _C.stream_of(self.W))
        # the kernel wrote W in place: move torch's version counter, as an in-place
        # torch op would, and record that the workspace holds W^T of this version
        torch.autograd.graph.increment_version(self.W)
        self._wt_version = self.W._version if plan_ok else None
        if self._seed_dev is None:
            self.seed += 1

    def step(self, x: torch.Tensor, dY: torch.Tensor, lddy: int) -> None:
        """forward -> backward to features (partials) -> fused weight/bias gradient +
        SR-SGD, whose launch also finishes dX."""
        self.forward(x)
        self.backward_features(dY, lddy, defer_dx=True)
        self.backward_weights_sgd(dY, lddy)
