"""Torch-eager CPU restatement of the EGNN layer and stack (concat form).

TEST INFRASTRUCTURE ONLY (see ``oracle/egnn_oracle.py`` for who may import it).

Two uses:
* an independent formulation that pins the numpy oracle: the edge model is a
  ``torch.nn.Linear`` on the concatenation ``[h_i, h_j, r2, e]``
  (``E_GCL.edge_model``, egnn_clean.py:49-58) instead of the split packed
  weights, and gradients come from torch autograd instead of a hand-written
  chain rule;
* the CPU baseline of ``bench.py``: the same torch-eager style as the
  reference's CPU-capable path (``pytorch_baseline.py:18-48``,
  ``egnn_clean.py:95-146``), run in fp32 on the host cores.

Semantics follow egnn_clean.py: E_GCL with edge_mlp Lin(2H+1+FE -> H)-SiLU-
Lin(H -> H)-SiLU (:22-26), coord_mlp Lin(H -> H)-SiLU-Lin(H -> 1, no bias)
(:33-42), node_mlp Lin(2H -> H)-SiLU-Lin(H -> H) (:28-31), sum aggregation of
messages (:62), mean (default) or sum aggregation of coordinates (:72-82),
residual h update (:68-69); EGNN = embedding_in, n_layers x E_GCL,
embedding_out (:133-146).  The edge index is (row, col) with row the
aggregation target, and coord_diff = x[row] - x[col] (:86).
"""
from __future__ import annotations

import torch
from torch import nn

__all__ = ["fused_concat", "node_update_ref", "EGCLRef", "EGNNRef", "MPNNGCLRef", "MPNNRef", "egcl_params_packed", "segment_sum",
           "segment_mean"]


def segment_sum(data, seg, n):
    """unsorted_segment_sum (egnn_clean.py:149-154)."""
    out = data.new_zeros((n, data.shape[1]))
    out.index_add_(0, seg, data)
    return out


def segment_mean(data, seg, n):
    """unsorted_segment_mean (egnn_clean.py:157-164): divide by max(count, 1)."""
    out = segment_sum(data, seg, n)
    cnt = torch.bincount(seg, minlength=n).to(data.dtype).clamp(min=1)
    return out / cnt[:, None]


def fused_concat(h, coord, edge_feat, row, col, w1_packed, w2, w1_mov=None, w2_mov=None, b1=None, b2=None,
                 bx1=None, *, mean_agg=False, equivariant=True):
    """The fused layer in concat form: returns (out_msg, out_mov or None).

    ``w1_packed`` (2F+g+FE, H) is used as one Linear on cat([h_i, h_j, r2, e])
    exactly as egnn_clean.py:51-56 builds its input.
    """
    parts = [h[row], h[col]]
    if equivariant:
        diff = coord[row, :3] - coord[col, :3]
        parts.append((diff * diff).sum(dim=1, keepdim=True))
    if edge_feat is not None and edge_feat.shape[1] > 0:
        parts.append(edge_feat)
    x = torch.cat(parts, dim=1)
    m1 = nn.functional.silu(nn.functional.linear(x, w1_packed.t(), b1))
    m = nn.functional.silu(nn.functional.linear(m1, w2.t(), b2))
    n = h.shape[0]
    out_msg = segment_sum(m, row, n)
    if not equivariant:
        return out_msg, None
    p = nn.functional.silu(nn.functional.linear(m, w1_mov.t(), bx1))
    phi = p @ w2_mov.reshape(-1, 1)
    trans = diff * phi
    out_mov = segment_mean(trans, row, n) if mean_agg else segment_sum(trans, row, n)
    return out_msg, out_mov


def node_update_ref(x1, x2, w1, b1, w2, b2, residual=True):
    """node_mlp(cat([x1, x2])) (+ x1): egnn_clean.py:60-70 with nn.Linear-layout weights."""
    x = x1 if x2 is None else torch.cat([x1, x2], dim=1)
    out = nn.functional.linear(nn.functional.silu(nn.functional.linear(x, w1, b1)), w2, b2)
    return x1 + out if residual else out


class EGCLRef(nn.Module):
    """E_GCL (egnn_clean.py:5-103) with the default options (no attention,
    no normalisation, no tanh)."""

    def __init__(self, input_nf, output_nf, hidden_nf, edges_in_d=0, coords_agg="mean", residual=True):
        super().__init__()
        self.residual = residual
        self.coords_agg = coords_agg
        self.edge_mlp = nn.Sequential(nn.Linear(2 * input_nf + 1 + edges_in_d, hidden_nf), nn.SiLU(),
                                      nn.Linear(hidden_nf, hidden_nf), nn.SiLU())
        self.node_mlp = nn.Sequential(nn.Linear(hidden_nf + input_nf, hidden_nf), nn.SiLU(),
                                      nn.Linear(hidden_nf, output_nf))
        last = nn.Linear(hidden_nf, 1, bias=False)
        nn.init.xavier_uniform_(last.weight, gain=0.001)
        self.coord_mlp = nn.Sequential(nn.Linear(hidden_nf, hidden_nf), nn.SiLU(), last)

    def forward(self, h, edge_index, coord, edge_attr=None):
        row, col = edge_index
        diff = coord[row] - coord[col]
        radial = (diff * diff).sum(dim=1, keepdim=True)
        parts = [h[row], h[col], radial] + ([edge_attr] if edge_attr is not None else [])
        m = self.edge_mlp(torch.cat(parts, dim=1))
        trans = diff * self.coord_mlp(m)
        agg_x = segment_mean(trans, row, coord.shape[0]) if self.coords_agg == "mean" else \
            segment_sum(trans, row, coord.shape[0])
        coord = coord + agg_x
        agg = segment_sum(m, row, h.shape[0])
        out = self.node_mlp(torch.cat([h, agg], dim=1))
        if self.residual:
            out = h + out
        return out, coord, edge_attr


class EGNNRef(nn.Module):
    """EGNN stack (egnn_clean.py:106-146)."""

    def __init__(self, in_node_nf, hidden_nf, out_node_nf, in_edge_nf=0, n_layers=4, coords_agg="mean"):
        super().__init__()
        self.embedding_in = nn.Linear(in_node_nf, hidden_nf)
        self.embedding_out = nn.Linear(hidden_nf, out_node_nf)
        self.layers = nn.ModuleList([EGCLRef(hidden_nf, hidden_nf, hidden_nf, edges_in_d=in_edge_nf,
                                             coords_agg=coords_agg) for _ in range(n_layers)])

    def forward(self, h, x, edges, edge_attr=None, act_round=None):
        """``act_round``: applied to h after the embedding and after every layer (the
        activations a bf16 stack stores between layers), e.g. :func:`round_bf16_st`."""
        rd = act_round or (lambda t: t)
        h = rd(self.embedding_in(h))
        for layer in self.layers:
            h, x, _ = layer(h, edges, x, edge_attr=edge_attr)
            h = rd(h)
        return self.embedding_out(h), x


class MPNNGCLRef(nn.Module):
    """E_GCL without the coordinate branch and without the radial input: the
    non-equivariant message-passing layer (edge_mlp on cat([h_i, h_j, e]))."""

    def __init__(self, input_nf, output_nf, hidden_nf, edges_in_d=0, residual=True):
        super().__init__()
        self.residual = residual
        self.edge_mlp = nn.Sequential(nn.Linear(2 * input_nf + edges_in_d, hidden_nf), nn.SiLU(),
                                      nn.Linear(hidden_nf, hidden_nf), nn.SiLU())
        self.node_mlp = nn.Sequential(nn.Linear(hidden_nf + input_nf, hidden_nf), nn.SiLU(),
                                      nn.Linear(hidden_nf, output_nf))

    def forward(self, h, edge_index, edge_attr=None):
        row, col = edge_index
        parts = [h[row], h[col]] + ([edge_attr] if edge_attr is not None else [])
        m = self.edge_mlp(torch.cat(parts, dim=1))
        agg = segment_sum(m, row, h.shape[0])
        out = self.node_mlp(torch.cat([h, agg], dim=1))
        if self.residual:
            out = h + out
        return out, edge_attr


class MPNNRef(nn.Module):
    """embedding_in, n_layers x MPNNGCLRef, embedding_out."""

    def __init__(self, in_node_nf, hidden_nf, out_node_nf, in_edge_nf=0, n_layers=2):
        super().__init__()
        self.embedding_in = nn.Linear(in_node_nf, hidden_nf)
        self.embedding_out = nn.Linear(hidden_nf, out_node_nf)
        self.layers = nn.ModuleList([MPNNGCLRef(hidden_nf, hidden_nf, hidden_nf, edges_in_d=in_edge_nf)
                                     for _ in range(n_layers)])

    def forward(self, h, edges, edge_attr=None, act_round=None):
        rd = act_round or (lambda t: t)
        h = rd(self.embedding_in(h))
        for layer in self.layers:
            h, _ = layer(h, edges, edge_attr=edge_attr)
            h = rd(h)
        return self.embedding_out(h)


def round_bf16_st(t):
    """Round to bfloat16 values in the forward, identity in the backward (straight through)."""
    return t + (t.to(torch.bfloat16).to(t.dtype) - t).detach()


def egcl_params_packed(layer) -> dict:
    """Map an E_GCL-style module's parameters onto the fused op's packed weights."""
    e0, e2 = layer.edge_mlp[0], layer.edge_mlp[2]
    c0, c2 = layer.coord_mlp[0], layer.coord_mlp[2]
    return dict(w1_msg=e0.weight.t(), b1=e0.bias, w2_msg=e2.weight.t(), b2=e2.bias, w1_mov=c0.weight.t(),
                bx1=c0.bias, w2_mov=c2.weight.reshape(-1))
