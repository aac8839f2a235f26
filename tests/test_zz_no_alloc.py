"""GPU parity of haste_ffi_forward_bce_noalloc (the forward + sparse BCE with
the library's own per-GPU scratch instead of a caller workspace) against
haste_ffi_forward_bce, through the C ABI: bit-identical dY, logits and loss,
on two calls in a row, the second with a smaller input (the scratch keeps the
first call's contents; the second call must not see them)."""
import numpy as np
import pytest
import torch

from haste_amd import _C, _lib

pytestmark = pytest.mark.gpu


def make(B, D, O, G, F, seed, dev):
    g = torch.Generator(device=dev).manual_seed(seed)
    Gc = (O + G - 1) // G
    x = torch.randn(B, D, generator=g, device=dev).to(torch.bfloat16)
    W = ((torch.rand(O, F, generator=g, device=dev) * 2 - 1) / F ** 0.5).to(torch.bfloat16)
    bias = (torch.randn(O, generator=g, device=dev) * 0.1).to(torch.bfloat16)
    idx = torch.randint(0, D, (Gc, F), generator=g, device=dev, dtype=torch.int32)
    rows = torch.randint(0, B, (6 * B,), generator=g, device=dev, dtype=torch.int32)
    labs = torch.randint(0, O, (6 * B,), generator=g, device=dev, dtype=torch.int32)
    labels = torch.stack([rows, labs], 1).contiguous()
    return x, W, bias, idx, labels


def run(noalloc, x, W, bias, idx, labels, B, D, O, G, F, dev):
    xT, ldx = _C.padded_transpose(x)
    ldo = (O + 63) // 64 * 64
    dY = torch.full((B, ldo), 3.0, dtype=torch.bfloat16, device=dev)
    logits = torch.full((B, ldo), 3.0, dtype=torch.bfloat16, device=dev)
    loss = torch.full((), 5.0, dtype=torch.float32, device=dev)
    st = _C.stream_of(x)
    common = (idx.data_ptr(), xT.data_ptr(), ldx, W.data_ptr(), bias.data_ptr(),
              labels.data_ptr(), labels.shape[0], dY.data_ptr(), ldo, logits.data_ptr(),
              loss.data_ptr())
    if noalloc:
        _lib.call("haste_ffi_forward_bce_noalloc", *common, B, D, F, O, G, _lib.DTYPE_BF16, st)
    else:
        n = _lib.lib().haste_ffi_forward_bce_workspace_size(B, O, G)
        ws = torch.zeros(n, dtype=torch.uint8, device=dev)
        _lib.call("haste_ffi_forward_bce", *common, ws.data_ptr(), n, B, D, F, O, G,
                  _lib.DTYPE_BF16, st)
        torch.cuda.synchronize()
        ldyw = ((O + G - 1) // G * G + 31) // 32
        assert not ws[: B * ldyw * 4].any()  # the label bitmap is left zero
    torch.cuda.synchronize()
    return dY[:, :O].clone(), logits[:, :O].clone(), loss.clone()


@pytest.mark.parametrize("shapes", [
    [(512, 768, 131073, 64, 128), (96, 300, 5003, 32, 64)],   # config 1, then smaller
    [(256, 512, 20000, 16, 32), (64, 768, 4096, 32, 32)],     # then config 0
])
def test_noalloc_matches_workspace_entry_point(dev, shapes):
    for i, (B, D, O, G, F) in enumerate(shapes):
        data = make(B, D, O, G, F, seed=40 + i, dev=dev)
        a = run(True, *data, B, D, O, G, F, dev)
        b = run(False, *data, B, D, O, G, F, dev)
        for u, v in zip(a, b):
            assert torch.equal(u.view(torch.int16) if u.dtype == torch.bfloat16 else u.view(torch.int32),
                               v.view(torch.int16) if v.dtype == torch.bfloat16 else v.view(torch.int32)), (i, B, O)
        assert np.isfinite(a[2].item())
