"""Public op ``group_ffi_mul`` (reference: shared_ffi/ops.py:7-24)."""
from typing import Optional

import torch

from . import bindings as _bindings

__all__ = ["group_ffi_mul", "head_tail_logits"]


def group_ffi_mul(features: torch.Tensor,
                  weights: torch.Tensor,
                  group_locations: torch.Tensor,
                  bias: Optional[torch.Tensor],
                  gsize: int = 32):
    """Grouped fixed-fan-in product: out[..., l] = sum_j features[..., idx[l//gsize, j]] *
    weights[l, j] (+ bias[l]).  Inputs with more than two dimensions are
    flattened to [N, D] and the result reshaped back (shared_ffi/ops.py:18-22)."""
    if features.ndim > 2:
        original_shape = features.shape[:-1]
        reshaped = features.reshape(-1, features.shape[-1])
        result = _bindings.GroupFFIMulFunction.apply(reshaped, weights, group_locations, bias, gsize)
        return result.view(original_shape + (weights.shape[0],))
    return _bindings.GroupFFIMulFunction.apply(features, weights, group_locations, bias, gsize)


def head_tail_logits(x_head: torch.Tensor, head: torch.nn.Linear, x_tail: torch.Tensor,
                     weights: torch.Tensor, group_locations: torch.Tensor,
                     bias: Optional[torch.Tensor], gsize: int = 32) -> torch.Tensor:
    """torch.cat((head(x_head), group_ffi_mul(x_tail, weights, ...)), dim=1) of the
    head/tail split model (src/model.py:245-248), with the FFI tail written into
    the concatenated [B, H + O] output in place instead of copied (and its
    gradient read in place), so the B x O tail makes no extra HBM round trip."""
    return _bindings.HeadTailFFIFunction.apply(x_head, head.weight, head.bias, x_tail, weights,
                                               group_locations, bias, gsize)
