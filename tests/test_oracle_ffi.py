"""Pins the PyTorch-CPU gather+bmm restatement (oracle/ffi.py) of the FFI layer."""
import itertools

import numpy as np
import pytest
import torch

import oracle


def _case(B, D, O, G, F, seed=0, dup=False):
    g = torch.Generator().manual_seed(seed)
    Gc = (O + G - 1) // G
    x = torch.randn(B, D, generator=g, dtype=torch.float64)
    W = torch.randn(O, F, generator=g, dtype=torch.float64)
    bias = torch.randn(O, generator=g, dtype=torch.float64)
    idx = torch.randint(0, D, (Gc, F), generator=g, dtype=torch.int32)
    if dup:
        idx[0, :] = 1
        idx[-1, 1::2] = idx[-1, 0::2]
    dY = torch.randn(B, O, generator=g, dtype=torch.float64)
    return x, W, bias, idx, dY


def _brute(x, W, bias, idx, dY, G):
    """Pure-Python per-element loops straight from the definitions."""
    B, D = x.shape
    O, F = W.shape
    xl, Wl, il, dl = x.tolist(), W.tolist(), idx.tolist(), dY.tolist()
    out = [[sum(xl[b][il[l // G][j]] * Wl[l][j] for j in range(F)) + float(bias[l])
            for l in range(O)] for b in range(B)]
    dX = [[0.0] * D for _ in range(B)]
    dW = [[0.0] * F for _ in range(O)]
    for b, l, j in itertools.product(range(B), range(O), range(F)):
        d = il[l // G][j]
        dX[b][d] += Wl[l][j] * dl[b][l]
        dW[l][j] += dl[b][l] * xl[b][d]
    db = [sum(dl[b][l] for b in range(B)) for l in range(O)]
    t = lambda a: torch.tensor(a, dtype=torch.float64)  # noqa: E731
    return t(out), t(dX), t(dW), t(db)


@pytest.mark.parametrize("B,D,O,G,F,dup", [(3, 7, 10, 4, 3, False), (5, 9, 17, 8, 4, True),
                                          (2, 5, 16, 16, 2, True), (4, 6, 1, 2, 6, False)])
def test_against_brute_force(B, D, O, G, F, dup):
    x, W, bias, idx, dY, = _case(B, D, O, G, F, dup=dup)
    out, dX, dW, db = _brute(x, W, bias, idx, dY, G)
    xT = x.t().contiguous()
    torch.testing.assert_close(oracle.ffi_forward(idx, xT, W, bias, G).double(), out, rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(oracle.ffi_backward_features(idx, W, dY, G, D).t().double(), dX,
                               rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(oracle.ffi_backward_weights(idx, xT, dY, G).double(), dW, rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(oracle.bias_grad(dY).double(), db, rtol=1e-5, atol=1e-5)


def test_dense_special_case():
    """G = 1, F = D, idx[l] = arange(D): the layer is a dense linear layer."""
    B, D, O = 6, 12, 9
    x, W, bias, _, dY = _case(B, D, O, 1, D, seed=3)
    idx = torch.arange(D, dtype=torch.int32).repeat(O, 1)
    xT = x.t().contiguous()
    ref = torch.nn.functional.linear(x, W, bias)
    torch.testing.assert_close(oracle.ffi_forward(idx, xT, W, bias, 1).double(), ref, rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(oracle.ffi_backward_features(idx, W, dY, 1, D).t().double(), dY @ W,
                               rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(oracle.ffi_backward_weights(idx, xT, dY, 1).double(), dY.t() @ x,
                               rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("G,F", [(16, 32), (64, 128), (32, 8)])
def test_adjoint_identities(G, F):
    """<fwd(x), dY> = <x, bwd_features(dY)> and <fwd_W(W), dY> = <W, bwd_weights(dY)>."""
    B, D, O = 9, 40, 3 * G + 5
    x, W, _, idx, dY = _case(B, D, O, G, F, seed=7, dup=True)
    xT = x.t().contiguous()
    lhs = (oracle.ffi_forward(idx, xT, W, None, G).double() * dY).sum()
    rhs_x = (x * oracle.ffi_backward_features(idx, W, dY, G, D).t().double()).sum()
    rhs_w = (W * oracle.ffi_backward_weights(idx, xT, dY, G).double()).sum()
    assert abs(lhs - rhs_x) <= 1e-4 * abs(lhs) + 1e-4
    assert abs(lhs - rhs_w) <= 1e-4 * abs(lhs) + 1e-4


def test_padding_rows_are_zero():
    Wp = oracle.pad_groups(torch.ones(5, 3), 4)
    assert Wp.shape == (2, 4, 3)
    assert Wp[1, 1:].abs().sum() == 0 and Wp[1, 0].sum() == 3


def test_duplicate_indices_sum():
    """Two slots with the same index contribute twice (the reference sums them)."""
    B, D, O, G, F = 2, 4, 2, 2, 2
    x = torch.tensor([[1.0, 2.0, 3.0, 4.0], [0.5, 0.25, 0.0, -1.0]])
    W = torch.tensor([[1.0, 10.0], [2.0, 20.0]])
    idx = torch.tensor([[3, 3]], dtype=torch.int32)
    out = oracle.ffi_forward(idx, x.t().contiguous(), W, None, G)
    assert np.allclose(out.numpy(), [[44.0, 88.0], [-11.0, -22.0]])
    dY = torch.tensor([[1.0, 0.0], [0.0, 1.0]])
    dXT = oracle.ffi_backward_features(idx, W, dY, G, D)
    assert np.allclose(dXT[3].numpy(), [11.0, 22.0]) and dXT[:3].abs().sum() == 0


# ---- sparse BCE (fused into the forward by haste_ffi_forward_bce) ----
def _bce_case(B=5, O=37, nnz=12, seed=3):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(B, O, generator=g) * 4).to(torch.bfloat16)
    rows = torch.randint(0, B, (nnz,), generator=g)
    cols = torch.randint(0, O, (nnz,), generator=g)
    labels = torch.stack([rows, cols], 1).to(torch.int32)
    return x, labels


def test_bce_matches_library_bce_with_logits():
    """The loss is torch's binary_cross_entropy_with_logits (sum) on the same
    binary targets, and dY its autograd gradient, rounded to bf16."""
    x, labels = _bce_case()
    loss, dY, y = oracle.ffi.bce_loss_grad(x, labels)
    xd = x.double().requires_grad_(True)
    ref = torch.nn.functional.binary_cross_entropy_with_logits(xd, y.double(), reduction="sum")
    ref.backward()
    assert abs(loss - ref.item()) <= 1e-12 * abs(ref.item())
    assert torch.equal(dY, xd.grad.to(torch.bfloat16))


def test_bce_closed_forms():
    """x = 0 everywhere: loss = B*O*ln 2 and dY = 1/2 - y; a repeated positive
    counts once; pairs out of range are ignored; large |x| gives exact 0/1 terms."""
    B, O = 3, 10
    x = torch.zeros(B, O, dtype=torch.bfloat16)
    labels = torch.tensor([[0, 1], [0, 1], [2, 9], [3, 0], [-1, 2], [1, 10]], dtype=torch.int32)
    loss, dY, y = oracle.ffi.bce_loss_grad(x, labels)
    assert abs(loss - B * O * np.log(2.0)) < 1e-9
    expect = torch.full((B, O), 0.5)
    expect[0, 1] = -0.5
    expect[2, 9] = -0.5
    assert torch.equal(dY.float(), expect)
    assert y.sum().item() == 2
    big = torch.tensor([[100.0, -100.0]], dtype=torch.bfloat16)
    loss, dY, _ = oracle.ffi.bce_loss_grad(big, torch.tensor([[0, 0]], dtype=torch.int32))
    assert 0.0 <= loss < 1e-40  # two terms of log1p(exp(-100))
    assert dY.float().tolist() == [[0.0, 0.0]]


def test_bce_gradient_is_loss_derivative():
    """Central finite differences of the fp64 loss in x match sigma(x) - y."""
    x, labels = _bce_case(B=2, O=6, nnz=4, seed=5)
    loss, dY, y = oracle.ffi.bce_loss_grad(x, labels)
    xd = x.double()
    h = 1e-6
    for b in range(2):
        for l in range(6):
            xp, xm = xd.clone(), xd.clone()
            xp[b, l] += h
            xm[b, l] -= h
            f = lambda t: (t.clamp(min=0) - y.double() * t + torch.log1p(torch.exp(-t.abs()))).sum()
            num = (f(xp) - f(xm)).item() / (2 * h)
            assert abs(num - (torch.sigmoid(xd[b, l]) - y[b, l]).item()) < 1e-6
