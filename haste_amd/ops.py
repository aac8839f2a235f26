"""Public op ``group_ffi_mul`` (reference: shared_ffi/ops.py:7-24)."""
from typing import Optional

import torch

from . import bindings as _bindings

__all__ = ["group_ffi_mul"]


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
