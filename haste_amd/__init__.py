"""haste_amd -- MI355X-native drop-in for HASTE's ``shared_ffi`` package.

Same module layout and entry points as the reference's shared_ffi
(shared_ffi/__init__.py:3-33): ``ffi_forward``, ``backward_features``,
``backward_weights`` here, and the submodules ``ops`` (group_ffi_mul),
``bindings`` (GroupFFIMulFunction), ``optim_sr`` (SRSgd / SGD_SR),
``rewire`` (GroupFixedFanIn), ``sr_triton`` (stochastic_rounding, sgd_update).
All compute runs in hand-written gfx950 HIP kernels (libhaste_ffi.so, C ABI in
include/haste_ffi.h); there is no CPU path.
"""
from . import _C

__all__ = ["ffi_forward", "backward_features", "backward_weights"]


def ffi_forward(locations, features, weights, bias=None, gsize=32):
    """Forward kernel call with sizes derived as the reference derives them
    (shared_ffi/__init__.py:3-13): features is X^T [H, B]."""
    B = features.size(1)
    H = features.size(0)
    FANIN = weights.size(1)
    L = weights.size(0)
    return _C.ffi_forward_cuda(locations, features, weights, bias, int(B), int(H), int(FANIN),
                               int(L), int(gsize))


def backward_features(features, weights, locations, grad_outputs, gsize=32):
    """fp32 dX^T [H, B] (shared_ffi/__init__.py:15-23)."""
    B = features.size(1)
    H = features.size(0)
    FANIN = weights.size(1)
    L = weights.size(0)
    return _C.ffi_backward_features_cuda(features, weights, locations, grad_outputs, int(B),
                                         int(H), int(FANIN), int(L), int(gsize))


def backward_weights(features, weights, locations, grad_outputs, gsize=32):
    """dW [L, FANIN] in the features dtype (shared_ffi/__init__.py:25-33)."""
    B = features.size(1)
    H = features.size(0)
    FANIN = weights.size(1)
    L = weights.size(0)
    return _C.ffi_backward_weights_cuda(features, weights, locations, grad_outputs, int(B),
                                        int(H), int(FANIN), int(L), int(gsize))
