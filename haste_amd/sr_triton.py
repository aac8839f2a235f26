"""Import-compatibility alias of the reference module ``shared_ffi.sr_triton``.

The reference implements these in Triton (shared_ffi/sr_triton.py); here they
are HIP kernels, re-exported from ``haste_amd.sr`` so that
``from shared_ffi.sr_triton import stochastic_rounding, sgd_update`` keeps working.
No Triton is used.
"""
from .sr import sgd_update, stochastic_rounding  # noqa: F401

__all__ = ["stochastic_rounding", "sgd_update"]
