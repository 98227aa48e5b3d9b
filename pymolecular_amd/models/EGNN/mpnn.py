"""Non-equivariant MPNN layer and stack on the fused HIP layer (``equivariant = 0``).

The reference names an MPNN path but ships no module for it: layer.py:65
calls an ``mpnn_forward`` that is not in its tree.  This module is the
E_GCL of egnn_clean.py:5-103 with the coordinate branch removed:

    m_ij  = SiLU(W_2 SiLU(W_1 [h_i, h_j, e_ij] + b_1) + b_2)    (edge_model, :49-58, no radial)
    h_i'  = h_i + node_mlp([h_i, sum_j m_ij])                    (node_model, :60-70)

The message sum is one fused HIP call with ``equivariant = False``; it never
materialises the E x (2H+F_E) concatenation or the E x H messages.
"""
from __future__ import annotations

import torch
from torch import nn

from ...fused import egnn_fused
from ...layer_fn import GCLLayerFn
from ...node_update import dense, node_update
from .egnn_clean import _csr_cache

__all__ = ["MPNN_GCL", "MPNN"]


class MPNN_GCL(nn.Module):
    """Message-passing layer: E_GCL without coordinates (edge_mlp input 2F + F_E)."""

    def __init__(self, input_nf, output_nf, hidden_nf, edges_in_d=0, act_fn=nn.SiLU(), residual=True):
        super().__init__()
        if not isinstance(act_fn, nn.SiLU):
            raise NotImplementedError("the fused MPNN layer implements act_fn=SiLU")
        self.residual = residual
        self.edges_in_d = edges_in_d
        self.edge_mlp = nn.Sequential(nn.Linear(2 * input_nf + edges_in_d, hidden_nf), act_fn,
                                      nn.Linear(hidden_nf, hidden_nf), act_fn)
        self.node_mlp = nn.Sequential(nn.Linear(hidden_nf + input_nf, hidden_nf), act_fn,
                                      nn.Linear(hidden_nf, output_nf))

    def fused_messages(self, h, edge_index, edge_attr=None, csr=None):
        """sum_j m_ij per destination row, from the fused op."""
        row, col = edge_index
        row_ptrs, col_s, perm = csr if csr is not None else _csr_cache.get(row, col, h.shape[0])
        e0, e2 = self.edge_mlp[0], self.edge_mlp[2]
        ef = edge_attr if (edge_attr is not None and self.edges_in_d > 0) else None
        agg, _ = egnn_fused(h, None, ef, row_ptrs, col_s, perm, e0.weight, e2.weight, None, None,
                            e0.bias, e2.bias, None, mean_agg=False, equivariant=False, linear_weights=True)
        return agg

    def forward(self, h, edge_index, edge_attr=None, node_attr=None, csr=None):
        if node_attr is None:   # the whole layer as one autograd node (layer_fn.GCLLayerFn)
            row, col = edge_index
            row_ptrs, col_s, perm = csr if csr is not None else _csr_cache.get(row, col, h.shape[0])
            e0, e2, n0, n2 = self.edge_mlp[0], self.edge_mlp[2], self.node_mlp[0], self.node_mlp[2]
            ef = edge_attr if (edge_attr is not None and self.edges_in_d > 0) else None
            h_out = GCLLayerFn.apply(h, None, ef, row_ptrs, col_s, perm, e0.weight, e0.bias, e2.weight, e2.bias,
                                     None, None, None, n0.weight, n0.bias, n2.weight, n2.bias, False, self.residual,
                                     False)
            return h_out, edge_attr
        agg = self.fused_messages(h, edge_index, edge_attr, csr)
        x2 = agg if node_attr is None else torch.cat([agg, node_attr.to(agg.dtype)], dim=1)
        return node_update(h, x2, self.node_mlp[0], self.node_mlp[2], residual=self.residual), edge_attr


class MPNN(nn.Module):
    """embedding_in, ``n_layers`` x MPNN_GCL, embedding_out (the EGNN stack of
    egnn_clean.py:106-146 without coordinates)."""

    def __init__(self, in_node_nf, hidden_nf, out_node_nf, in_edge_nf=0, device='cpu', act_fn=nn.SiLU(),
                 n_layers=2, residual=True):
        super().__init__()
        self.hidden_nf = hidden_nf
        self.n_layers = n_layers
        self.embedding_in = nn.Linear(in_node_nf, hidden_nf)
        self.embedding_out = nn.Linear(hidden_nf, out_node_nf)
        for i in range(n_layers):
            self.add_module("gcl_%d" % i, MPNN_GCL(hidden_nf, hidden_nf, hidden_nf, edges_in_d=in_edge_nf,
                                                   act_fn=act_fn, residual=residual))
        self.to(device)

    def forward(self, h, edges, edge_attr=None):
        h = dense(h, self.embedding_in)
        row, col = edges
        csr = _csr_cache.get(row, col, h.shape[0])
        for i in range(self.n_layers):
            h, _ = self._modules["gcl_%d" % i](h, edges, edge_attr=edge_attr, csr=csr)
        return dense(h, self.embedding_out)
