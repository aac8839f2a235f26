"""The reference's import lines work against this build through the
``shared_ffi`` package, and resolve to haste_amd's objects (CPU: imports only)."""
import importlib


def test_reference_import_lines():
    import haste_amd
    import shared_ffi
    from shared_ffi import ops                                  # src/group_fanin_real.py:3
    from shared_ffi.optim_sr import SRSgd                       # src/runner.py:21
    from shared_ffi.rewire import GroupFixedFanIn               # src/model.py:7
    from shared_ffi.sr_triton import sgd_update, stochastic_rounding  # optim_sr.py:4, bindings.py:5
    from shared_ffi.bindings import GroupFFIMulFunction

    assert ops is haste_amd.ops
    assert SRSgd is haste_amd.optim_sr.SRSgd
    assert GroupFixedFanIn is haste_amd.rewire.GroupFixedFanIn
    assert sgd_update is haste_amd.sr_triton.sgd_update
    assert stochastic_rounding is haste_amd.sr_triton.stochastic_rounding
    assert GroupFFIMulFunction is haste_amd.bindings.GroupFFIMulFunction
    assert shared_ffi.ffi_forward is haste_amd.ffi_forward
    assert shared_ffi.backward_features is haste_amd.backward_features
    assert shared_ffi.backward_weights is haste_amd.backward_weights
    assert shared_ffi._C.ffi_forward_cuda is haste_amd._C.ffi_forward_cuda
    assert importlib.import_module("shared_ffi.ops") is haste_amd.ops
