"""SGD with momentum, weight decay and stochastic rounding (reference:
shared_ffi/optim_sr.py:7-114, class ``SRSgd``; the north star calls it SGD_SR).

Semantics kept from the reference:
  * per param group, ``seed`` is read and then incremented by 1 on every
    step (optim_sr.py:59-62); every tensor of the group uses that seed with
    offsets restarting at 0 (so weights and bias share random streams);
  * fp32 params take the plain torch path (optim_sr.py:73-84);
  * low-precision params are updated in place by one fused kernel (one
    launch per gradient dtype covers all of the group's tensors)
    (g' = fma(wd, w, g); m' = fma(mu, m, g'); w' = fma(-lr, m' or g', w);
    SR to bf16 with tl.randint(seed, i), or RNE when SR is off);
  * non-contiguous params are updated through a contiguous copy.
The weights of a grouped FFI layer whose last backward used an index plan
(``bindings.wt_target``) are updated by haste_sgd_sr_step_wt instead: the same
update, bit for bit, which also writes the transposed weights that layer's
next backward reads, so the backward skips gathering them
(``refresh_transposed=False`` turns this off).  When the layer's bias is a
parameter of the same group with a gradient, haste_sgd_sr_step_wt_bias steps
it in the same launch (again bit for bit).  Every updated parameter's
version counter is moved, as an in-place torch op would move it.
  * every parameter that requires a gradient gets its fp32 ``momentum_buf``
    at construction, zero, whether or not momentum is used (optim_sr.py:35-44),
    so a checkpoint carries the same state keys as the reference's.

Checkpoints: ``state_dict()`` holds each group's current ``seed`` and the fp32
momentum buffers.  ``load_state_dict`` keeps the buffers in fp32 (torch's
default casts floating-point state to the parameter's dtype, which would round
them to bf16), so a restored optimizer continues bit-identically.
"""
from __future__ import annotations

from itertools import chain

import torch
from torch.optim import Optimizer
from torch.optim import optimizer as _torch_optimizer

from . import _C, _lib
from . import bindings as _bindings
from .sr import sgd_update_multi

__all__ = ["SRSgd", "SGD_SR"]


class SRSgd(Optimizer):
    def __init__(self, params, lr: float = 1e-3, weight_decay: float = 0.0,
                 momentum: float = 0.0, use_momentum: bool = True,
                 stochastic_rounding: bool = True, seed: int = 123,
                 refresh_transposed: bool = True):
        defaults = dict(lr=lr, weight_decay=weight_decay, momentum=momentum,
                        use_momentum=use_momentum, stochastic_rounding=stochastic_rounding,
                        seed=seed)
        super().__init__(params, defaults)
        self.refresh_transposed = bool(refresh_transposed)
        for group in self.param_groups:
            for p in group["params"]:
                if p.requires_grad:
                    self._momentum_buf(p)

    def load_state_dict(self, state_dict) -> None:
        # torch casts floating-point state to the parameter's dtype; the momentum
        # buffers are fp32 whatever the parameter's dtype, so they are put back
        saved = {k: v.get("momentum_buf") for k, v in state_dict["state"].items()}
        saved_ids = [i for g in state_dict["param_groups"] for i in g["params"]]
        super().load_state_dict(state_dict)
        params = [p for g in self.param_groups for p in g["params"]]
        for pid, p in zip(saved_ids, params):
            m = saved.get(pid)
            if isinstance(m, torch.Tensor):
                self.state[p]["momentum_buf"] = m.to(dtype=torch.float32, device=p.device).clone()

    def zero_grad(self, set_to_none: bool = True) -> None:
        """torch.optim.Optimizer.zero_grad, same semantics, without the
        profiler scope and compiler guard torch wraps it in (about 20 us of
        host time per call, on the path of every training step)."""
        for group in self.param_groups:
            for p in group["params"]:
                if p.grad is None:
                    continue
                if set_to_none:
                    p.grad = None
                else:
                    if p.grad.grad_fn is not None:
                        p.grad.detach_()
                    else:
                        p.grad.requires_grad_(False)
                    p.grad.zero_()

    @staticmethod
    def _uses_momentum(group) -> bool:
        return bool(group["use_momentum"]) and group["momentum"] != 0.0

    def _momentum_buf(self, p: torch.Tensor) -> torch.Tensor:
        state = self.state[p]
        buf = state.get("momentum_buf")
        if buf is None:
            buf = torch.zeros_like(p.data, dtype=torch.float32, device=p.device)
            state["momentum_buf"] = buf
        return buf

    def step(self, closure=None):
        """One step, torch.optim.Optimizer.step semantics: the step pre-hooks
        (global, then this optimizer's) run first and may replace the arguments,
        the post-hooks (this optimizer's, then global) after.  torch wraps the
        step of every Optimizer subclass in a profiler scope that does the same
        around the call; this one is marked as wrapped already (``hooked``),
        which saves about 15 us of host time per step, and runs the hooks
        itself.  The step shows in a torch profile through its kernels and
        library calls, without an ``Optimizer.step#SRSgd.step`` scope."""
        pre = _torch_optimizer._global_optimizer_pre_hooks
        post = _torch_optimizer._global_optimizer_post_hooks
        if not (pre or post or self._optimizer_step_pre_hooks or self._optimizer_step_post_hooks):
            return self._sr_step(closure)
        args, kwargs = (self, closure), {}
        for hook in chain(pre.values(), self._optimizer_step_pre_hooks.values()):
            result = hook(self, args, kwargs)
            if result is not None:
                if isinstance(result, tuple) and len(result) == 2:
                    args, kwargs = result
                else:
                    raise RuntimeError(f"{hook} must return None or a tuple of (new_args, "
                                       f"new_kwargs), but got {result}.")
        out = args[0]._sr_step(*args[1:], **kwargs)
        for hook in chain(self._optimizer_step_post_hooks.values(), post.values()):
            hook(self, args, kwargs)
        return out

    step.hooked = True  # Optimizer.__init__ then leaves it unwrapped

    @torch.no_grad()
    def _sr_step(self, closure=None):
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()

        for group in self.param_groups:
            lr = group["lr"]
            wd = group["weight_decay"]
            mu = group["momentum"]
            use_mom = group["use_momentum"]
            sr = group["stochastic_rounding"]
            seed = group["seed"]
            group["seed"] += 1
            mom_on = self._uses_momentum(group)

            # FFI layers whose last backward used an index plan: their weights
            # (and their bias, when it is a parameter of this group with a
            # gradient) are stepped by haste_sgd_sr_step_wt[_bias]
            targets, fused_bias = {}, {}
            if self.refresh_transposed:
                ids = {id(q) for q in group["params"]}
                for p in group["params"]:
                    if p.grad is None or p.dtype != torch.bfloat16 or p.dim() != 2:
                        continue
                    ent = _bindings.wt_target(p) if p.data.is_contiguous() else None
                    if ent is None or ent.dims[2:4] != (p.shape[1], p.shape[0]):
                        continue
                    targets[id(p)] = ent
                    b = ent.bias() if ent.bias is not None else None
                    if (b is not None and id(b) in ids and b.grad is not None
                            and b.dtype == torch.bfloat16 and b.dim() == 1
                            and b.shape[0] == p.shape[0] and b.data.is_contiguous()
                            and all(b is not c for c in fused_bias.values())):
                        fused_bias[id(p)] = b  # (a bias shared by two layers: stepped once)
            stepped = {id(b) for b in fused_bias.values()}

            # bf16 tensors are updated by one fused launch per gradient dtype
            batches = {}
            for p in group["params"]:
                if p.grad is None or id(p) in stepped:
                    continue
                grad = p.grad

                if p.dtype == torch.float32:
                    if wd != 0.0:
                        grad = grad.add(p, alpha=wd)
                    if mom_on:
                        buf = self._momentum_buf(p)
                        buf.mul_(mu).add_(grad)
                        update = buf
                    else:
                        update = grad
                    p.add_(update, alpha=-lr)
                    continue

                w = p.data
                g_contig = grad if grad.is_contiguous() else grad.contiguous()
                ent = targets.get(id(p))
                if ent is not None:
                    # an FFI layer's weights: the same update, which also writes the
                    # transposed weights its next backward reads (no gather there)
                    B, D, F, O, G = ent.dims
                    m = self._momentum_buf(p) if mom_on else None
                    mp = None if m is None else m.data_ptr()
                    b = fused_bias.get(id(p))
                    if b is None:
                        _lib.call("haste_sgd_sr_step_wt", w.data_ptr(), g_contig.data_ptr(),
                                  _C.dtype_code(g_contig.dtype), mp, float(lr), float(wd),
                                  float(mu), int(mom_on), int(bool(sr)), int(seed),
                                  ent.ws.data_ptr(), ent.ws.numel(), B, D, F, O, G,
                                  _lib.DTYPE_BF16, _C.stream_of(w))
                    else:
                        gb = b.grad if b.grad.is_contiguous() else b.grad.contiguous()
                        mb = self._momentum_buf(b) if mom_on else None
                        _lib.call("haste_sgd_sr_step_wt_bias", w.data_ptr(), g_contig.data_ptr(),
                                  _C.dtype_code(g_contig.dtype), mp, b.data.data_ptr(),
                                  gb.data_ptr(), _C.dtype_code(gb.dtype),
                                  None if mb is None else mb.data_ptr(), float(lr), float(wd),
                                  float(mu), int(mom_on), int(bool(sr)), int(seed),
                                  ent.ws.data_ptr(), ent.ws.numel(), B, D, F, O, G,
                                  _lib.DTYPE_BF16, _C.stream_of(w))
                        torch.autograd.graph.increment_version(b)
                    torch.autograd.graph.increment_version(p)
                    _bindings.mark_wt_refreshed(ent, p)
                    continue
                w_contig = w if w.is_contiguous() else w.contiguous()
                b = batches.setdefault(grad.dtype, ([], [], [], []))
                b[0].append(w_contig)
                b[1].append(g_contig)
                b[2].append(self._momentum_buf(p) if mom_on else None)
                b[3].append(p)
            for ws, gs, ms, ps in batches.values():
                sgd_update_multi(ws, gs, ms if mom_on else None, learning_rate=lr,
                                 weight_decay=wd, momentum=mu, use_momentum=use_mom,
                                 stochastic_rounding=sr, seed=seed)
                for w_contig, p in zip(ws, ps):
                    if w_contig.data_ptr() != p.data.data_ptr():
                        p.data.copy_(w_contig)
                    # the kernel wrote through a raw pointer: move the version counter
                    # as an in-place torch op would
                    torch.autograd.graph.increment_version(p)
        return loss


SGD_SR = SRSgd
