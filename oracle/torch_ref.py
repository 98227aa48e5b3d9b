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

__all__ = ["fused_concat", "node_update_ref", "first_layer", "EGCLRef", "EGNNRef", "MPNNGCLRef", "MPNNRef",
           "egcl_params_packed", "segment_sum", "segment_mean", "set_hoist", "bf16_rounding_realization",
           "bf16_roundoff", "BF16_UNIT_ROUNDOFF"]


def segment_sum(data, seg, n):
    """unsorted_segment_sum (egnn_clean.py:149-154).  bfloat16 data is summed in float32 and the sum
    rounded once (bf16 activations with fp32 accumulation)."""
    if data.dtype == torch.bfloat16:
        return segment_sum(data.float(), seg, n).to(torch.bfloat16)
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


class _GatherRows(torch.autograd.Function):
    """t[idx] whose backward sums the row gradients in float32 and rounds the sum once (torch's own
    index backward accumulates in the tensor's dtype, i.e. in bfloat16 for a bfloat16 tensor)."""

    @staticmethod
    def forward(ctx, t, idx):
        ctx.save_for_backward(idx)
        ctx.shape, ctx.dtype = t.shape, t.dtype
        return t[idx]

    @staticmethod
    def backward(ctx, g):
        (idx,) = ctx.saved_tensors
        acc = torch.float32 if ctx.dtype == torch.bfloat16 else g.dtype
        out = torch.zeros(ctx.shape, dtype=acc)
        out.index_add_(0, idx, g.to(acc))
        return out.to(ctx.dtype), None


def gather_rows(t, idx):
    """Rows ``t[idx]``; for bfloat16 ``t`` the gradient is accumulated in float32 (see _GatherRows)."""
    return _GatherRows.apply(t, idx) if t.dtype == torch.bfloat16 else t[idx]


def first_layer(lin, h, row, col, extra, hoist):
    """edge_mlp[0] on cat([h_i, h_j, *extra]) (egnn_clean.py:51-56).

    ``hoist``: the same linear map evaluated as P[row] + Q[col] + W_x [extra] with the per-node
    products P = h W_i^T + b, Q = h W_j^T formed (and, in bfloat16, rounded) once per node and the sum
    in float32 -- mathematically identical, rounded at other points.  Used to measure how much a
    quantity moves under bfloat16 rounding at the rounding points of a hoisted layer.
    """
    if not hoist:
        return lin(torch.cat([gather_rows(h, row), gather_rows(h, col)] + [t.to(h.dtype) for t in extra], dim=1))
    F = h.shape[1]
    W = lin.weight
    # contiguous weight slices: torch's CPU bfloat16 linear returns wrong input gradients for a
    # column slice of a row-major weight (a strided operand)
    P = nn.functional.linear(h, W[:, :F].contiguous(), lin.bias)
    Q = nn.functional.linear(h, W[:, F:2 * F].contiguous())
    acc = torch.float32 if h.dtype == torch.bfloat16 else h.dtype
    pre = gather_rows(P, row).to(acc) + gather_rows(Q, col).to(acc)
    k = 2 * F
    for t in extra:
        w = W[:, k:k + t.shape[1]].contiguous()
        pre = pre + nn.functional.linear(t.to(h.dtype), w).to(acc)
        k += t.shape[1]
    return pre.to(h.dtype)


class EGCLRef(nn.Module):
    """E_GCL (egnn_clean.py:5-103) with the default options (no attention,
    no normalisation, no tanh).

    Runs in float64 (the oracle), float32, or bfloat16 (parameters and h in bfloat16, coordinates
    in float32: the radial input is rounded where it enters the edge MLP, segment sums accumulate
    in float32).  ``hoist_first_layer``: evaluate edge_mlp[0] through :func:`first_layer`'s
    per-node products."""

    def __init__(self, input_nf, output_nf, hidden_nf, edges_in_d=0, coords_agg="mean", residual=True):
        super().__init__()
        self.hoist_first_layer = False
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
        extra = [radial] + ([edge_attr] if edge_attr is not None else [])
        m = self.edge_mlp[1:](first_layer(self.edge_mlp[0], h, row, col, extra, self.hoist_first_layer))
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
        self.hoist_first_layer = False
        self.residual = residual
        self.edge_mlp = nn.Sequential(nn.Linear(2 * input_nf + edges_in_d, hidden_nf), nn.SiLU(),
                                      nn.Linear(hidden_nf, hidden_nf), nn.SiLU())
        self.node_mlp = nn.Sequential(nn.Linear(hidden_nf + input_nf, hidden_nf), nn.SiLU(),
                                      nn.Linear(hidden_nf, output_nf))

    def forward(self, h, edge_index, edge_attr=None):
        row, col = edge_index
        extra = [edge_attr] if edge_attr is not None else []
        m = self.edge_mlp[1:](first_layer(self.edge_mlp[0], h, row, col, extra, self.hoist_first_layer))
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


BF16_UNIT_ROUNDOFF = 2.0 ** -9


def bf16_roundoff(t, gen):
    """``t`` times (1 + eps), eps uniform in [-u, u] per element, u = 2^-9 the unit roundoff of
    round-to-nearest bfloat16: the relative error a rounding to bfloat16 makes, drawn at random
    (the probabilistic model of rounding errors), evaluated in float64."""
    eps = (torch.rand(t.shape, generator=gen, dtype=torch.float64) * 2.0 - 1.0) * BF16_UNIT_ROUNDOFF
    return (t.double() * (1.0 + eps)).to(t.dtype)


class _Roundoff(torch.autograd.Function):
    """bf16_roundoff of a value in the forward and of its gradient in the backward."""

    @staticmethod
    def forward(ctx, t, gen):
        ctx.gen = gen
        return bf16_roundoff(t, gen)

    @staticmethod
    def backward(ctx, g):
        return bf16_roundoff(g, ctx.gen), None


def bf16_rounding_realization(model, gen):
    """Make a float32 model apply a random bfloat16 roundoff (bf16_roundoff) to every Linear and SiLU
    output and to their gradients (forward hooks; returns the handles and the act_round to pass
    between layers).  Repeated with different generators, it samples how far rounding to bfloat16 at
    those points moves each output and gradient: each quantity's conditioning at bfloat16."""
    handles = [mod.register_forward_hook(lambda m, i, o: _Roundoff.apply(o, gen))
               for mod in model.modules() if isinstance(mod, (nn.Linear, nn.SiLU))]
    return handles, (lambda t: _Roundoff.apply(t, gen))


def set_hoist(model, on: bool):
    """Switch every layer of a stack (or a single layer) to the hoisted first-layer evaluation."""
    for mod in model.modules():
        if hasattr(mod, "hoist_first_layer"):
            mod.hoist_first_layer = on
    return model


def round_bf16_st(t):
    """Round to bfloat16 values in the forward, identity in the backward (straight through)."""
    return t + (t.to(torch.bfloat16).to(t.dtype) - t).detach()


def egcl_params_packed(layer) -> dict:
    """Map an E_GCL-style module's parameters onto the fused op's packed weights."""
    e0, e2 = layer.edge_mlp[0], layer.edge_mlp[2]
    c0, c2 = layer.coord_mlp[0], layer.coord_mlp[2]
    return dict(w1_msg=e0.weight.t(), b1=e0.bias, w2_msg=e2.weight.t(), b2=e2.bias, w1_mov=c0.weight.t(),
                bx1=c0.bias, w2_mov=c2.weight.reshape(-1))
