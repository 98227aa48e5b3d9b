"""One message-passing layer (fused messages + node update) as one autograd node.

``E_GCL.forward`` (egnn_clean.py:93-103) is edge_model + coord_model + node_model:

    agg, agg_x = sum_j m_ij, mean_j (x_i - x_j) phi_x(m_ij)
    x'         = x + agg_x
    h'         = h + node_mlp([h, agg])

As separate autograd nodes, h feeds both the fused message op and the node
update, so autograd adds the two gradients of h with an extra elementwise
kernel.  Here the backward runs the node update's backward first and then the
fused backward with ``EGNN_FLAG_ACCUMULATE_GRAD_H``, which adds the message
path's gradient of h into the node update's buffer inside the dh product's
epilogue.  ``EGNN_FLAG_COORD_RESIDUAL`` does the same for the coordinates: the
forward writes ``x + agg_x`` and the backward's coordinate gradient includes
the residual path, so neither needs an elementwise add.  The MPNN layer (``equivariant = False``) is the same without the
coordinate path.
"""
from __future__ import annotations

import torch

from .fused import _dims, _fused_backward, _fused_forward, _node_proj_buffer, _prep_inputs, get_schedule
from .node_update import node_update_backward, node_update_forward

__all__ = ["GCLLayerFn"]


class GCLLayerFn(torch.autograd.Function):
    """``GCLLayerFn.apply(h, coord, edge_attr, row_ptrs, col, perm, e0w, e0b, e2w, e2b, c0w, c0b, c2w,
    n0w, n0b, n2w, n2b, mean_agg, residual, equivariant)`` -> ``(h', x')`` (EGNN) or ``h'`` (MPNN).

    Weights in torch.nn.Linear layout: edge_mlp[0] / [2] (e0, e2), coord_mlp[0] / [2] (c0, c2; EGNN
    only, None for MPNN), node_mlp[0] / [2] (n0, n2).  No gradient flows to edge_attr or the CSR.
    """

    @staticmethod
    def forward(ctx, h, coord, edge_attr, row_ptrs, col, perm, e0w, e0b, e2w, e2b, c0w, c0b, c2w, n0w, n0b, n2w,
                n2b, mean_agg, residual, equivariant):
        ctx.shapes = [None if t is None else tuple(t.shape) for t in (e0w, e2w, c0w, c2w, e0b, e2b, c0b)]
        hp, coord_p, ef, w1, w2, w1m, w2m, b1, b2, bx1 = _prep_inputs(
            h, coord, edge_attr, e0w, e2w, c0w, c2w, e0b, e2b, c0b, equivariant)
        # the layer's dimensions and the graph's schedule, once for the forward and the backward
        dims = _dims(hp, ef, col, w1, w2, w1m, equivariant, mean_agg, True)
        sched = get_schedule(row_ptrs, col, hp.shape[0])
        pq = _node_proj_buffer(hp, ef, col, w1, w2, w1m, equivariant, mean_agg, True, dims=dims)
        agg, x_new = _fused_forward(hp, coord_p, ef, row_ptrs, col, perm, w1, w2, w1m, w2m, b1, b2, bx1,
                                    mean_agg=mean_agg, equivariant=equivariant, node_proj=pq, linear_weights=True,
                                    coord_residual=True, dims=dims, sched=sched)
        out, (nt, res, has_b, wdt) = node_update_forward(hp, agg, n0w, n0b, n2w, n2b, residual)
        ctx.save_for_backward(hp, coord_p, ef, row_ptrs, col, perm, w1, w2, w1m, w2m, b1, b2, bx1, pq, *nt)
        ctx.node = (res, has_b, wdt)
        ctx.dims, ctx.sched = dims, sched
        ctx.mean_agg, ctx.equivariant = mean_agg, equivariant
        ctx.coord_dtype = None if coord is None else coord.dtype
        if not equivariant:
            return out
        return out, x_new.to(coord.dtype)

    @staticmethod
    def backward(ctx, g_out, g_coord=None):
        saved = ctx.saved_tensors
        hp, coord, ef, row_ptrs, col, perm, w1, w2, w1m, w2m, b1, b2, bx1, pq = saved[:14]
        nt = saved[14:]
        res, has_b, wdt = ctx.node
        eq = ctx.equivariant
        N = hp.shape[0]
        if g_out is None:
            g_out = torch.zeros((N, nt[3].shape[0]), dtype=hp.dtype, device=hp.device)
        grad_x, gn0w, gn0b, gn2w, gn2b = node_update_backward(nt, res, has_b, wdt, g_out)
        K1 = hp.shape[1]
        g_h, g_agg = grad_x[:, :K1], grad_x[:, K1:]
        if eq and g_coord is None:
            g_coord = torch.zeros((N, 3), dtype=torch.float32, device=hp.device)
        g = _fused_backward(hp, coord, ef, row_ptrs, col, perm, w1, w2, w1m, w2m, b1, b2, bx1, g_agg,
                            g_coord if eq else None, mean_agg=ctx.mean_agg, equivariant=eq, node_proj=pq,
                            linear_weights=True, grad_h_into=g_h, coord_residual=True, dims=ctx.dims,
                            sched=ctx.sched)
        gc = g["coord"].to(ctx.coord_dtype) if eq else None   # includes g_coord (EGNN_FLAG_COORD_RESIDUAL)
        wg = [g[k] for k in ("w1_msg", "w2_msg", "w1_mov", "w2_mov", "b1", "b2", "bx1")]
        e0w_g, e2w_g, c0w_g, c2w_g, e0b_g, e2b_g, c0b_g = [
            None if (t is None or shp is None) else t.reshape(shp) for t, shp in zip(wg, ctx.shapes)]
        return (g["h"], gc, None, None, None, None, e0w_g, e0b_g, e2w_g, e2b_g, c0w_g, c0b_g, c2w_g,
                gn0w, gn0b, gn2w, gn2b, None, None, None)
