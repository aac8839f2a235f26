"""Grouped fixed-fan-in layer with on-device rewiring (reference:
shared_ffi/rewire.py:36-239, ``GroupFixedFanIn``).

Constructor arguments, parameter/buffer names and dtypes (``weights`` [O, F],
``bias`` [O], persistent buffer ``group_locations`` int32 [ceil(O/G), F]) and
initialisation follow the reference (rewire.py:64-127).  ``rewire()`` runs as
one HIP kernel (libhaste_ffi.so ``haste_rewire``) with no host sync; its
contract is deterministic (see include/haste_ffi.h): the reference's
torch.randint / uniform_ draws and topk tie order are replaced by Philox
streams keyed by a seed drawn from torch's default CPU generator, and ties in
fraction mode go to the lower slot.  ``regrow_mode="unused"`` (new) draws only
indices not already present in the group.  ``fp32_grads=True`` (new) keeps
the weight and bias gradients in fp32 (``grad_dtype``), which the SR-SGD
kernel consumes directly.
"""
from __future__ import annotations

import math

import torch

from . import _C, _lib, ops

GROWTH_MODES = ["random"]
PRUNE_MODES = ["threshold", "fraction"]
INIT_MODES = ["random", "zero"]
REGROW_MODES = ["random", "unused"]
GROUP_SIZES = [16, 32, 64, 128]

__all__ = ["GroupFixedFanIn", "GroupFixedFanInReal", "inflate_group_locations"]
SCORE_MODES = ["mean", "max"]


class GroupFixedFanIn(torch.nn.Module):
    """Fixed fan-in sparse linear layer whose labels share index sets in groups
    of ``group_size`` (see the reference docstring, rewire.py:37-58)."""

    __constants__ = ["in_features", "out_features", "fan_in"]
    in_features: int
    out_features: int
    fan_in: int

    def __init__(self, in_features: int, out_features: int, fan_in: int, bias: bool = True,
                 device=None, dtype=None, *, group_size=32, prune_mode="threshold",
                 rewire_threshold=None, rewire_fraction=None, growth_mode="random",
                 init_mode="random", regrow_mode="random", fp32_grads=False, **kwargs):
        super().__init__(**kwargs)
        factory_kwargs = {"device": device, "dtype": dtype}
        self.in_features = in_features
        self.out_features = out_features
        self.fan_in = fan_in

        assert prune_mode in PRUNE_MODES, f"Invalid prune_mode={prune_mode}; supported: {PRUNE_MODES}"
        assert growth_mode in GROWTH_MODES, f"Invalid growth_mode={growth_mode}; supported: {GROWTH_MODES}"
        assert init_mode in INIT_MODES, f"Invalid init_mode={init_mode}; supported: {INIT_MODES}"
        assert regrow_mode in REGROW_MODES, f"Invalid regrow_mode={regrow_mode}; supported: {REGROW_MODES}"
        if prune_mode == "threshold" and rewire_threshold is None:
            raise ValueError("rewire_threshold must be specified for prune_mode 'threshold'")
        elif prune_mode == "fraction" and rewire_fraction is None:
            raise ValueError("rewire_fraction must be specified for prune_mode 'fraction'")
        self.prune_mode = prune_mode
        self.growth_mode = growth_mode
        self.init_mode = init_mode
        self.regrow_mode = regrow_mode
        if prune_mode == "fraction":
            self.rewire_fraction = rewire_fraction
            assert 0 <= rewire_fraction < 1, \
                f"Invalid reware_fraction={rewire_fraction}; supported range [0,1)"
        else:
            self.rewire_threshold = rewire_threshold

        self.weights = torch.nn.parameter.Parameter(torch.empty((out_features, fan_in), **factory_kwargs))
        bound = 1 / math.sqrt(self.fan_in)
        torch.nn.init.uniform_(self.weights, -bound, bound)
        if bias:
            self.bias = torch.nn.parameter.Parameter(torch.empty(out_features, **factory_kwargs))
            torch.nn.init.zeros_(self.bias)
        else:
            self.register_parameter("bias", None)

        assert group_size in GROUP_SIZES, \
            f"Current kernels only support group size from {GROUP_SIZES}. Selected group size={group_size}"
        if fp32_grads:
            # keep fp32 gradients for low-precision parameters (torch >= 2.10)
            self.weights.grad_dtype = torch.float32
            if self.bias is not None:
                self.bias.grad_dtype = torch.float32
        self.group_size = group_size
        self.num_groups = (out_features + self.group_size - 1) // self.group_size
        group_locations = torch.randint(high=self.in_features, size=(self.num_groups, fan_in),
                                        dtype=torch.int32)
        self.register_buffer("group_locations", group_locations, persistent=True)
        self._pruned_total = None  # device int32 counter of pruned slots (no host sync)

    def forward(self, features):
        return ops.group_ffi_mul(features, self.weights, self.group_locations, self.bias,
                                 gsize=self.group_size)

    def extra_repr(self) -> str:
        return "in_features={}, out_features={}, fan_in={}, bias={}".format(
            self.in_features, self.out_features, self.fan_in, self.bias is not None)

    @property
    def pruned_total(self) -> int:
        """Total number of slots pruned by rewire() so far (syncs the device)."""
        return 0 if self._pruned_total is None else int(self._pruned_total.item())

    @torch.no_grad()
    def rewire(self, seed: int = None):
        """Prune + regrow every group in one kernel launch (reference rewire.py:143-239).

        ``seed`` keys the Philox streams of the regrowth draws; by default it is
        drawn from torch's default CPU generator."""
        W = self.weights
        if self.out_features == 0:
            return
        _C.require_device(W, "weights")
        wcode = _C.dtype_code(W.dtype)   # bf16, fp16 or fp32: rewired in their own dtype
        if not W.is_contiguous() or not self.group_locations.is_contiguous():
            raise RuntimeError("rewire: weights and group_locations must be contiguous")
        F = self.fan_in
        if self.prune_mode == "threshold":
            mode, thr, k = _lib.PRUNE_THRESHOLD, float(self.rewire_threshold), 0
        else:
            k = int(F * self.rewire_fraction)
            if k == 0:
                return
            mode, thr = _lib.PRUNE_FRACTION, 0.0
        if seed is None:
            seed = int(torch.randint(0, 2**62, (1,), dtype=torch.int64).item())
        if self._pruned_total is None or self._pruned_total.device != W.device:
            self._pruned_total = torch.zeros(1, dtype=torch.int32, device=W.device)
        _lib.call("haste_rewire", W.data_ptr(), wcode, self.group_locations.data_ptr(), None,
                  self._pruned_total.data_ptr(), self.out_features, F, self.group_size,
                  self.in_features, mode, thr, k,
                  _lib.REGROW_UNUSED if self.regrow_mode == "unused" else _lib.REGROW_RANDOM,
                  _lib.INIT_RANDOM if self.init_mode == "random" else _lib.INIT_ZERO,
                  float(1.0 / math.sqrt(F)), int(seed), _C.stream_of(W))
        # the kernel wrote through raw pointers: tell torch (and index-plan caches
        # keyed on the version counter) that both tensors changed
        torch.autograd.graph.increment_version(self.weights)
        torch.autograd.graph.increment_version(self.group_locations)



class GroupFixedFanInReal(GroupFixedFanIn):
    """The application's grouped layer (src/group_fanin_real.py, ``GroupFixedFanInReal``):
    the same parameters and forward, and its rewire variant (:150-286):
      * scores per (group, slot): the mean (``score_mode="mean"``) or max
        (``"max"``) over the group's rows of |w|, or of the saliency |w * grad|
        when ``use_grad`` is set (the product in the tensors' dtype, as the
        reference; fp32 gradients are used as they are);
      * ``prune_mode="fraction"`` prunes the ``int(num_groups * fan_in * fraction)``
        smallest scores of the whole layer (the reference's global topk; ties go
        to the lower slot), ``"threshold"`` every score below the threshold;
      * regrowth and initialisation as GroupFixedFanIn (Philox streams keyed by one
        seed per call; ``regrow_mode="unused"`` is also available).
    Runs as two kernels and one device-side k-th-value selection, no host sync."""

    def __init__(self, in_features: int, out_features: int, fan_in: int, bias: bool = True,
                 device=None, dtype=None, *, group_size=32, prune_mode="threshold",
                 rewire_threshold=None, rewire_fraction=None, growth_mode="random",
                 init_mode="random", score_mode="mean", regrow_mode="random",
                 fp32_grads=False, **kwargs):
        assert score_mode in SCORE_MODES, f"Invalid score_mode={score_mode}; supported: {SCORE_MODES}"
        super().__init__(in_features, out_features, fan_in, bias, device, dtype,
                         group_size=group_size, prune_mode=prune_mode,
                         rewire_threshold=rewire_threshold, rewire_fraction=rewire_fraction,
                         growth_mode=growth_mode, init_mode=init_mode, regrow_mode=regrow_mode,
                         fp32_grads=fp32_grads, **kwargs)
        self.score_mode = score_mode
        self.use_grad = False

    @torch.no_grad()
    def rewire(self, seed: int = None):
        W = self.weights
        if self.out_features == 0:
            return
        _C.require_device(W, "weights")
        wcode = _C.dtype_code(W.dtype)   # bf16, fp16 or fp32: rewired in their own dtype
        if not W.is_contiguous() or not self.group_locations.is_contiguous():
            raise RuntimeError("rewire: weights and group_locations must be contiguous")
        O, F, G = self.out_features, self.fan_in, self.group_size
        Gc = self.num_groups
        grad = W.grad if self.use_grad else None
        if self.use_grad and grad is None:
            raise RuntimeError("rewire: use_grad is set but weights.grad is None")
        if grad is not None:
            grad = grad.contiguous()
        gptr = None if grad is None else grad.data_ptr()
        # saliency |W * grad| in torch's promoted dtype of the two (the kernel's rule)
        gcode = _lib.DTYPE_BF16 if grad is None else _C.dtype_code(grad.dtype)
        smode = _lib.SCORE_MAX if self.score_mode == "max" else _lib.SCORE_MEAN
        st = _C.stream_of(W)
        scores = key_thr = None
        if self.prune_mode == "threshold":
            mode, thr, k = _lib.PRUNE_THRESHOLD, float(self.rewire_threshold), 0
        else:
            k = int(Gc * F * self.rewire_fraction)
            if k == 0:
                return
            mode, thr = _lib.PRUNE_GLOBAL_FRACTION, 0.0
            scores = torch.empty(Gc, F, dtype=torch.float32, device=W.device)
            _lib.call("haste_rewire_scores", W.data_ptr(), wcode, gptr, gcode, smode,
                      scores.data_ptr(), O, F, G, st)
            # unique keys (scores are >= 0, so their bits order them): the k-th
            # smallest is the last pruned slot; ties go to the lower slot
            keys = (scores.view(-1).view(torch.int32).to(torch.int64) << 32) | torch.arange(
                Gc * F, dtype=torch.int64, device=W.device)
            key_thr = torch.kthvalue(keys, k).values.contiguous()
        if seed is None:
            seed = int(torch.randint(0, 2**62, (1,), dtype=torch.int64).item())
        if self._pruned_total is None or self._pruned_total.device != W.device:
            self._pruned_total = torch.zeros(1, dtype=torch.int32, device=W.device)
        _lib.call("haste_rewire_ex", W.data_ptr(), wcode, self.group_locations.data_ptr(), gptr,
                  gcode,
                  smode, None if scores is None else scores.data_ptr(),
                  None if key_thr is None else key_thr.data_ptr(), None,
                  self._pruned_total.data_ptr(), O, F, G, self.in_features, mode, thr, k,
                  _lib.REGROW_UNUSED if self.regrow_mode == "unused" else _lib.REGROW_RANDOM,
                  _lib.INIT_RANDOM if self.init_mode == "random" else _lib.INIT_ZERO,
                  float(1.0 / math.sqrt(F)), int(seed), st)
        torch.autograd.graph.increment_version(self.weights)
        torch.autograd.graph.increment_version(self.group_locations)


@torch.no_grad()
def inflate_group_locations(group_locations: torch.Tensor, out_features: int,
                            group_size: int) -> torch.Tensor:
    """[ceil(L/G), F] group indices -> [L, F] per-label indices (each group row
    repeated group_size times, truncated to L), the checkpoint conversion of
    src/runner.py:323-334 from a grouped layer to a per-label fixed fan-in one."""
    return group_locations.repeat_interleave(int(group_size), dim=0)[: int(out_features)]
