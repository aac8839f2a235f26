"""GPU tests of the forward fused with the sparse BCE loss (haste_ffi_forward_bce,
FFITrainStep.forward_bce / step_bce) against the oracle's bce_loss_grad."""
import numpy as np
import pytest
import torch

import oracle
from haste_amd.step import FFITrainStep

pytestmark = pytest.mark.gpu
TOL16 = dict(rtol=1e-2, atol=1e-3)


def bits(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def _setup(dev, B, D, O, G, F, nnz, seed=0, extra_labels=None):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(B, D, generator=g).to(torch.bfloat16)
    W = (torch.randn(O, F, generator=g) * 0.3).to(torch.bfloat16)
    bias = (torch.randn(O, generator=g) * 0.5).to(torch.bfloat16)
    idx = torch.randint(0, D, ((O + G - 1) // G, F), generator=g, dtype=torch.int32)
    rows = torch.randint(0, B, (nnz,), generator=g)
    cols = torch.randint(0, O, (nnz,), generator=g)
    labels = torch.stack([rows, cols], 1).to(torch.int32)
    if extra_labels is not None:
        labels = torch.cat([labels, torch.tensor(extra_labels, dtype=torch.int32).view(-1, 2)])
    st = FFITrainStep(W.to(dev), bias.to(dev), idx.to(dev), B, D, G, lr=0.05, weight_decay=1e-4)
    return st, x.to(dev), labels


# (B, D, O, G, F): ragged B and O, a last group of one label, every G, F up to 256
CASES = [(64, 768, 4096, 32, 32), (100, 300, 1001, 64, 128), (37, 200, 513, 16, 64),
         (130, 256, 2049, 128, 128), (64, 512, 999, 32, 256), (512, 768, 8193, 64, 128)]


@pytest.mark.parametrize("B,D,O,G,F", CASES)
def test_forward_bce_matches_oracle(dev, B, D, O, G, F):
    # duplicates, a pair per corner, and pairs outside [0, B) x [0, O) (ignored)
    extra = [0, 0, 0, 0, B - 1, O - 1, -1, 3, B, 0, 0, O, 2, -5]
    st, x, labels = _setup(dev, B, D, O, G, F, nnz=5 * B, extra_labels=extra)
    logits = st.forward(x).clone()
    loss = st.forward_bce(x, labels.to(dev), write_logits=True)
    torch.cuda.synchronize()
    # the fused forward writes the same logits as the plain one, bit for bit
    assert np.array_equal(bits(st.logits), bits(logits))
    ref_loss, ref_dY, _ = oracle.ffi.bce_loss_grad(logits.cpu(), labels)
    dY = st.dY_buf[:, :O].float().cpu()
    torch.testing.assert_close(dY, ref_dY.float(), **TOL16)
    # hardware exp / log / reciprocal: at most one bf16 step away from the oracle
    ulp = torch.maximum(ref_dY.float().abs(), torch.tensor(2.0 ** -24)) * 2.0 ** -7
    assert bool(((dY - ref_dY.float()).abs() <= ulp).all())
    assert abs(loss.item() - ref_loss) <= 1e-5 * abs(ref_loss)
    # padding columns of the last group are zero; the label bitmap is clear again
    if st.ldo > O:
        assert st.dY_buf[:, O:st.ldo].abs().sum().item() == 0
    nb = B * ((((O + G - 1) // G) * G + 31) // 32) * 4
    assert int(st.bce_ws[:nb].count_nonzero().item()) == 0


def test_forward_bce_deterministic_and_no_labels(dev):
    B, D, O, G, F = 128, 768, 5000, 64, 128
    st, x, labels = _setup(dev, B, D, O, G, F, nnz=640, seed=4)
    l1 = st.forward_bce(x, labels.to(dev)).clone()
    d1 = st.dY_buf.clone()
    l2 = st.forward_bce(x, labels.to(dev)).clone()
    torch.cuda.synchronize()
    assert l1.item() == l2.item()
    assert torch.equal(d1, st.dY_buf)
    # no positives: dY = sigma(x) and loss = sum softplus(x)
    empty = torch.zeros(0, 2, dtype=torch.int32, device=dev)
    loss = st.forward_bce(x, empty, write_logits=True)
    ref_loss, ref_dY, _ = oracle.ffi.bce_loss_grad(st.logits.cpu(), torch.zeros(0, 2, dtype=torch.int32))
    torch.testing.assert_close(st.dY_buf[:, :O].float().cpu(), ref_dY.float(), **TOL16)
    assert abs(loss.item() - ref_loss) <= 1e-5 * abs(ref_loss)


def test_step_bce_equals_step_on_its_gradient(dev):
    """step_bce = forward_bce, then the backward + fused update on its dY: the
    weights, bias and dX equal those of step() given that dY."""
    B, D, O, G, F = 256, 768, 6000, 64, 128
    st1, x, labels = _setup(dev, B, D, O, G, F, nnz=1280, seed=7)
    st2, _, _ = _setup(dev, B, D, O, G, F, nnz=1280, seed=7)
    loss = st1.step_bce(x, labels.to(dev))
    dY = st1.dY_buf.clone()
    st2.step(x, dY, st2.ldo)
    torch.cuda.synchronize()
    assert np.isfinite(loss.item())
    assert np.array_equal(bits(st1.W), bits(st2.W))
    assert np.array_equal(bits(st1.bias), bits(st2.bias))
    assert np.array_equal(bits(st1.dX), bits(st2.dX))
