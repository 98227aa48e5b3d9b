"""``pytorch_egnn_baseline`` with the reference's signature, on the fused HIP layer.

Same arguments and return value as models/EGNN/pytorch_baseline.py:6-50:
``w1_msg``/``w2_msg`` are the node weights W_n1/W_n2 (F, H), ``w_e`` (F_E, H),
``w_d`` (H), ``w_hl`` (H, O), ``w1_mov`` (O, M), ``w2_mov`` (M); the loss is
<out_msg, grad_out_msg> + <out_mov, grad_out_mov> with sum aggregation over
``row_indices`` and the function returns ``(h.grad, coord.grad)`` after
enabling gradients on ``h``, ``coord`` and ``w1_msg`` (:12-15).  Instead of
materialising the per-edge tensors it runs the fused forward and backward.
Only beta = 1 (SiLU) is supported.
"""
from __future__ import annotations

import torch

from ...fused import egnn_fused


def swish_torch(x, beta=1.0):
    """x * sigmoid(beta x) (pytorch_baseline.py:3-4)."""
    return x * torch.sigmoid(beta * x)


def pytorch_egnn_baseline(h, coord, edge_feat, row_indices, col_indices, w1_msg, w2_msg, w1_mov, w2_mov, w_e, w_d,
                          w_hl, grad_out_msg, grad_out_mov, msg_beta=1.0, mov_beta=1.0):
    if msg_beta != 1.0 or mov_beta != 1.0:
        raise NotImplementedError("the fused layer computes SiLU (beta = 1)")
    h.requires_grad_(True)
    coord.requires_grad_(True)
    w1_msg.requires_grad_(True)
    N = h.shape[0]
    rows = row_indices.to(torch.int64)
    if rows.numel() > 1 and bool((rows[1:] < rows[:-1]).any()):
        raise ValueError("row_indices must be sorted (dst-sorted CSR order, datasets_loaders.py)")
    counts = torch.bincount(rows, minlength=N)
    row_ptrs = torch.zeros(N + 1, dtype=torch.int32, device=h.device)
    row_ptrs[1:] = torch.cumsum(counts, 0).to(torch.int32)
    F = h.shape[1]
    FE = 0 if edge_feat is None else edge_feat.shape[1]
    packed = torch.cat([w1_msg, w2_msg, w_d.reshape(1, -1)] + ([w_e] if FE else []), dim=0)
    out_msg, out_mov = egnn_fused(h, coord[:, :3], edge_feat if FE else None, row_ptrs,
                                  col_indices.to(torch.int32), None, packed, w_hl, w1_mov, w2_mov.reshape(-1),
                                  mean_agg=False, equivariant=True)
    loss = (out_msg.float() * grad_out_msg.float()).sum() + (out_mov * grad_out_mov[:, :3].float()).sum()
    loss.backward()
    return h.grad, coord.grad
