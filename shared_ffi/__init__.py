"""``shared_ffi`` import name for haste_amd, so code written against HASTE's
package (``from shared_ffi.rewire import GroupFixedFanIn``, src/model.py:7;
``from shared_ffi.optim_sr import SRSgd``, src/runner.py:21; ``from shared_ffi
import ops``, src/group_fanin_real.py:3; ``import shared_ffi`` then
``shared_ffi.ffi_forward``, shared_ffi/bindings.py:4,22) runs unchanged on the
MI355X build.  Every name is haste_amd's own object: the submodules are
registered under ``shared_ffi.<name>`` as well, so both spellings share one
module (one workspace cache, one library handle).
"""
import sys as _sys

import haste_amd as _haste
from haste_amd import _C, bindings, ops, optim_sr, rewire, sr_triton  # noqa: F401
from haste_amd import backward_features, backward_weights, ffi_forward  # noqa: F401

__all__ = ["ffi_forward", "backward_features", "backward_weights"]

for _name in ("_C", "bindings", "ops", "optim_sr", "rewire", "sr_triton"):
    _sys.modules[f"{__name__}.{_name}"] = getattr(_haste, _name)
del _name
