"""``EGNN_Triton_Layer`` (models/EGNN/layer.py:7-103) on the fused HIP layer.

Same constructor (f_node, f_edge, msg_hidden_dim, msg_out_feat,
mov_hidden_dim, node_hidden_dim), same parameters (packed ``w1_msg``
(2F+1+F_E, H), ``w2_msg`` (H, O), ``w1_mov`` (O, M), ``w2_mov`` (M, 1),
``node_mlp``) and the same ``forward(node_feat, coord, edge_index,
edge_feat)``.  The reference's edge-parallel ``mpnn_forward`` kernel does not
exist in its tree (layer.py:4); its call (:65-91) sends each edge's message
both ways (``out_msg1``/``out_mov1`` at the source, ``out_msg2``/``out_mov2``
at the destination), and the host divides the coordinate sum by the total
incident degree (:54-63, 93-95).  Here that is one fused call over the
symmetrised, dst-sorted edge list (both directions share the edge's
features through ``edge_ids``), followed by the same epilogue: x' = x + sum(delta phi) / max(deg, 1) and
h' = h + node_mlp([h, sum m]) (the fused node update).
"""
from __future__ import annotations

import torch
import torch.nn as nn

from ...fused import TensorCache, coo_to_csr, egnn_fused
from ...node_update import node_update


class EGNN_HIP_Layer(nn.Module):
    def __init__(self, f_node, f_edge, msg_hidden_dim, msg_out_feat, mov_hidden_dim, node_hidden_dim):
        super().__init__()
        self.F_NODE = f_node
        self.F_EDGE = f_edge
        self.HIDDEN_FEATURES = msg_hidden_dim
        self.OUT_FEATURES = msg_out_feat
        self.HID_FEAT_MOV_MLP = mov_hidden_dim
        msg_in_dim = (f_node * 2) + 1 + f_edge
        self.w1_msg = nn.Parameter(torch.randn(msg_in_dim, msg_hidden_dim) / msg_hidden_dim ** 0.5)
        self.w2_msg = nn.Parameter(torch.randn(msg_hidden_dim, msg_out_feat) / msg_out_feat ** 0.5)
        self.w1_mov = nn.Parameter(torch.randn(msg_out_feat, mov_hidden_dim) / mov_hidden_dim ** 0.5)
        self.w2_mov = nn.Parameter(torch.randn(mov_hidden_dim, 1) / 1.0)
        node_mlp_in = f_node + msg_out_feat
        self.node_mlp = nn.Sequential(nn.Linear(node_mlp_in, node_hidden_dim), nn.SiLU(),
                                      nn.Linear(node_hidden_dim, f_node))
        # CSR of the symmetrised edge list, per live edge_index tensor (not per address)
        self._csr = TensorCache(maxsize=4)

    def _both_ways(self, edge_index, num_nodes):
        return self._csr.get((edge_index,), int(num_nodes), lambda: self._build_both_ways(edge_index, num_nodes))

    @staticmethod
    def _build_both_ways(edge_index, num_nodes):
        src, dst = edge_index[0].to(torch.int64), edge_index[1].to(torch.int64)
        E = src.numel()
        rows = torch.cat([dst, src])          # destination of each directed message
        cols = torch.cat([src, dst])
        row_ptrs, col_s, perm = coo_to_csr(rows, cols, num_nodes)
        eids = (perm.to(torch.int64) % max(E, 1)).to(torch.int32)   # both directions read edge e's features
        deg = torch.diff(row_ptrs).to(torch.float32).clamp(min=1.0)
        return row_ptrs, col_s, eids, deg

    def forward(self, node_feat, coord, edge_index, edge_feat):
        N = node_feat.shape[0]
        row_ptrs, col_s, eids, deg = self._both_ways(edge_index, N)
        ef = edge_feat if self.F_EDGE > 0 else None
        total_msg, total_mov = egnn_fused(node_feat, coord[:, :3], ef, row_ptrs, col_s, eids, self.w1_msg,
                                          self.w2_msg, self.w1_mov, self.w2_mov.reshape(-1), mean_agg=False,
                                          equivariant=True)
        new_coord = coord.clone()
        new_coord[:, :3] = coord[:, :3] + total_mov / deg[:, None]
        # node_feat + node_mlp(cat([node_feat, total_msg])) (:97-101) as one fused node update
        return node_update(node_feat, total_msg.to(node_feat.dtype), self.node_mlp[0], self.node_mlp[2],
                           residual=True), new_coord


# the reference's name for the same module (layer.py:7)
EGNN_Triton_Layer = EGNN_HIP_Layer
