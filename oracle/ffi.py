"""PyTorch-CPU gather + bmm restatement of HASTE's grouped fixed-fan-in layer.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).  All math in fp32 on the
CPU; inputs may be bf16/fp16/fp32 tensors and are upcast exactly.

Shapes follow the reference's kernel interface (shared_ffi/__init__.py:3-33):
  idx  int32 [Gc, F]   group_locations, Gc = ceil(O / G)
  xT   [D, B]          features transposed (bindings.py:19)
  W    [O, F]          weights
  dY   [B, O]          grad of the logits
Labels l of group g = l // G share the F input indices idx[g, :].

Parity pins (tests/test_oracle_ffi.py): pure-Python per-element loops on tiny
shapes, the dense special case (G = 1, F = D, idx = arange -> x @ W.T), the
adjoint identities <fwd(x), dY> = <x, bwd_features(dY)> and
<fwd_W(W), dY> = <W, bwd_weights(dY)> in fp64, and duplicate-index cases.
"""
from __future__ import annotations

from typing import Optional

import torch


def pad_groups(W: torch.Tensor, G: int) -> torch.Tensor:
    """W [O, F] -> [Gc, G, F] with zero rows for labels >= O (the reference
    zero-fills those rows, ffi_forward_kernels.cu:187-195)."""
    O, F = W.shape
    Gc = (O + G - 1) // G
    Wp = torch.zeros(Gc * G, F, dtype=torch.float32)
    Wp[:O] = W.float()
    return Wp.view(Gc, G, F)


def _gather(xT: torch.Tensor, idx: torch.Tensor) -> torch.Tensor:
    """Xg[g, j, b] = xT[idx[g, j], b]  ->  [Gc, F, B] fp32."""
    return xT.float()[idx.long()]


def ffi_forward(idx: torch.Tensor, xT: torch.Tensor, W: torch.Tensor,
                bias: Optional[torch.Tensor], G: int) -> torch.Tensor:
    """logits[b, l] = sum_j xT[idx[l//G, j], b] * W[l, j] + bias[l], fp32 [B, O].

    Restates group_shared_fanin_v1 (ffi_forward_kernels.cu:125-286): per group a
    gathered [B x F] x [F x G] contraction with fp32 accumulation, bias added in
    fp32 in the epilogue (dump_and_store_tile, :85-93)."""
    O, F = W.shape
    D, B = xT.shape
    Xg = _gather(xT, idx)                        # [Gc, F, B]
    Wp = pad_groups(W, G)                        # [Gc, G, F]
    out = torch.bmm(Wp, Xg)                      # [Gc, G, B]
    out = out.permute(2, 0, 1).reshape(B, -1)[:, :O]
    if bias is not None:
        out = out + bias.float()[None, :]
    return out.contiguous()


def ffi_backward_features(idx: torch.Tensor, W: torch.Tensor, dY: torch.Tensor,
                          G: int, D: int) -> torch.Tensor:
    """dXT[d, b] = sum_{g, j: idx[g, j] = d} sum_{l in g} W[l, j] * dY[b, l], fp32 [D, B].

    Restates group_shared_fanin_bf_v1 (ffi_backward_features.cu:50-217): per
    group P = W_g^T dY_g^T, rows scattered by idx (duplicates summed, :202-212)."""
    O, F = W.shape
    B = dY.shape[0]
    Gc = idx.shape[0]
    Wp = pad_groups(W, G)                                    # [Gc, G, F]
    dYp = torch.zeros(B, Gc * G, dtype=torch.float32)
    dYp[:, :O] = dY.float()
    dYg = dYp.view(B, Gc, G).permute(1, 2, 0)                # [Gc, G, B]
    P = torch.bmm(Wp.transpose(1, 2), dYg)                   # [Gc, F, B]
    out = torch.zeros(D, B, dtype=torch.float32)
    out.index_add_(0, idx.long().reshape(-1), P.reshape(Gc * F, B))
    return out


def ffi_backward_weights(idx: torch.Tensor, xT: torch.Tensor, dY: torch.Tensor,
                         G: int) -> torch.Tensor:
    """dW[l, j] = sum_b dY[b, l] * xT[idx[l//G, j], b], fp32 [O, F].

    Restates group_shared_fanin_bw_v1 (ffi_backward_weights.cu:110-268)."""
    O = dY.shape[1]
    B = dY.shape[0]
    Gc = idx.shape[0]
    Xg = _gather(xT, idx)                                    # [Gc, F, B]
    dYp = torch.zeros(B, Gc * G, dtype=torch.float32)
    dYp[:, :O] = dY.float()
    dYg = dYp.view(B, Gc, G).permute(1, 2, 0)                # [Gc, G, B]
    dW = torch.bmm(dYg, Xg.transpose(1, 2))                  # [Gc, G, F]
    return dW.reshape(Gc * G, -1)[:O].contiguous()


def bias_grad(dY: torch.Tensor) -> torch.Tensor:
    """torch.sum(grad_output, dim=0) (bindings.py:40), fp32."""
    return dY.float().sum(0)


def bce_loss_grad(logits: torch.Tensor, labels: torch.Tensor):
    """Sparse BCE of the application's training loop (src/runner.py:469-478) on
    logits x [B, O] (bf16 values, upcast exactly) with positives given as COO
    int32 [nnz, 2] (row, label) pairs (src/data.py:26-46; y = 1 there, a repeated
    pair counts once, pairs outside [0, B) x [0, O) are ignored):
      loss = sum max(x, 0) - sum_pos x + sum log(1 + exp(-|x|))   (fp64 here)
      dY   = sigmoid(x) - y, rounded to bf16 (RNE)
    Returns (loss as a Python float, dY bf16 [B, O], y fp32 [B, O])."""
    x = logits.double()
    B, O = x.shape
    y = torch.zeros(B, O, dtype=torch.float64)
    lab = labels.long()
    ok = (lab[:, 0] >= 0) & (lab[:, 0] < B) & (lab[:, 1] >= 0) & (lab[:, 1] < O)
    lab = lab[ok]
    y[lab[:, 0], lab[:, 1]] = 1.0
    loss = (x.clamp(min=0.0) - y * x + torch.log1p(torch.exp(-x.abs()))).sum().item()
    dY = (torch.sigmoid(x) - y).to(torch.bfloat16)
    return loss, dY, y.float()
