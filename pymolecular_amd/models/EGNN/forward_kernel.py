"""Host callable with the parameter list of the reference's forward kernel.

``egnn_forward_kernel_node_parallel`` keeps the argument order, names and
meaning of models/EGNN/forward_kernel.py:14-43 (pointers, strides,
``num_nodes``, and the constexpr sizes as keywords).  The Triton launch
syntax ``kernel[grid](...)`` is accepted too: the grid is ignored because the
HIP path schedules its own 32-edge tiles.  It writes ``out_msg`` (N, O) and
columns 0..2 of ``out_mov`` (stride ``stride_mov_n``), with no biases and sum
aggregation, exactly what the reference kernel computes
(forward_kernel.py:141-153).  Tiling keywords of the Triton autotuner
(BLOCK_SIZE_NEIGHBORS, TILE_H, num_warps, ...) are accepted and ignored.
"""
from __future__ import annotations

import torch

from ...fused import egnn_fused_forward

_IGNORED = {"BLOCK_SIZE_NEIGHBORS", "TILE_H", "num_warps", "num_stages", "MSG_BETA", "MOV_BETA", "MOV_ACT_TYPE",
            "MSG_ACT_TYPE"}


class _Launcher:
    def __getitem__(self, grid):
        return self

    def __call__(self, h_ptr, coord_ptr, edge_feat_ptr, row_ptrs_ptr, col_indices_ptr, edge_id_ptr, out_msg_ptr,
                 out_mov_ptr, w1_msg_ptr, w2_msg_ptr, w1_mov_ptr, w2_mov_ptr, stride_h_n, stride_coord_n,
                 stride_edge_e, stride_msg_n, stride_mov_n, num_nodes, *, F_NODE, F_EDGE, HIDDEN_FEATURES,
                 OUT_FEATURES, HID_FEAT_MOV_MLP, **tuning):
        unknown = set(tuning) - _IGNORED
        if unknown:
            raise TypeError(f"unexpected keyword arguments {sorted(unknown)}")
        for k in ("MSG_BETA", "MOV_BETA"):
            if tuning.get(k, 1.0) != 1.0:
                raise NotImplementedError(f"{k} != 1 (the fused layer computes SiLU, beta = 1)")
        N = int(num_nodes)
        h = h_ptr.reshape(N, -1)[:, :F_NODE]
        w1 = w1_msg_ptr.reshape(2 * F_NODE + 1 + F_EDGE, HIDDEN_FEATURES)
        ef = None if F_EDGE == 0 else edge_feat_ptr.reshape(edge_feat_ptr.shape[0], -1)[:, :F_EDGE]
        out_msg, out_mov = egnn_fused_forward(
            h, coord_ptr.reshape(N, -1)[:, :3], ef, row_ptrs_ptr, col_indices_ptr, edge_id_ptr, w1,
            w2_msg_ptr.reshape(HIDDEN_FEATURES, OUT_FEATURES), w1_mov_ptr.reshape(OUT_FEATURES, HID_FEAT_MOV_MLP),
            w2_mov_ptr.reshape(-1), mean_agg=False, equivariant=True)
        out_msg_ptr.reshape(N, -1)[:, :OUT_FEATURES].copy_(out_msg)
        out_mov_ptr.reshape(N, -1)[:, :3].copy_(out_mov)


egnn_forward_kernel_node_parallel = _Launcher()
