"""Host callable with the parameter list of the reference's backward kernel.

``egnn_backward_kernel_node_parallel`` keeps the argument order of
models/EGNN/backward_kernel.py:14-50 and accepts ``kernel[grid](...)``.  It
writes dL/dh into ``grad_h``, dL/dx into columns 0..2 of ``grad_coord`` and
the weight gradients into ``grad_w1_msg`` (packed), ``grad_w2_msg``,
``grad_w1_mov`` and ``grad_w2_mov``.  Where the reference adds its weight
gradients into the *weights* (backward_kernel.py:251-257), reads
``grad_out_mov`` with the coordinate stride (:118) and races its plain store
of the main-node gradients against other programs' atomics (:247 vs :237),
this writes each result once to its own buffer: with the zero-filled buffers
``launch_triton`` passes (test_mem.py:15-20) the values are what the
reference's math defines.
"""
from __future__ import annotations

from ...fused import egnn_fused_backward
from .forward_kernel import _IGNORED


class _Launcher:
    def __getitem__(self, grid):
        return self

    def __call__(self, h_ptr, coord_ptr, edge_feat_ptr, row_ptrs_ptr, col_indices_ptr, edge_id_ptr,
                 grad_out_msg_ptr, grad_out_mov_ptr, grad_h_ptr, grad_coord_ptr, grad_w1_msg_ptr, grad_w2_msg_ptr,
                 grad_w1_mov_ptr, grad_w2_mov_ptr, w1_msg_ptr, w2_msg_ptr, w1_mov_ptr, w2_mov_ptr, stride_h_n,
                 stride_coord_n, stride_edge_e, stride_msg_n, stride_mov_n, num_nodes, *, F_NODE, F_EDGE,
                 HIDDEN_FEATURES, OUT_FEATURES, HID_FEAT_MOV_MLP, **tuning):
        unknown = set(tuning) - _IGNORED
        if unknown:
            raise TypeError(f"unexpected keyword arguments {sorted(unknown)}")
        N = int(num_nodes)
        H, O, M = HIDDEN_FEATURES, OUT_FEATURES, HID_FEAT_MOV_MLP
        ef = None if F_EDGE == 0 else edge_feat_ptr.reshape(edge_feat_ptr.shape[0], -1)[:, :F_EDGE]
        g = egnn_fused_backward(
            h_ptr.reshape(N, -1)[:, :F_NODE], coord_ptr.reshape(N, -1)[:, :3], ef, row_ptrs_ptr, col_indices_ptr,
            edge_id_ptr, w1_msg_ptr.reshape(2 * F_NODE + 1 + F_EDGE, H), w2_msg_ptr.reshape(H, O),
            w1_mov_ptr.reshape(O, M), w2_mov_ptr.reshape(-1), None, None, None,
            grad_out_msg_ptr.reshape(N, -1)[:, :O], grad_out_mov_ptr.reshape(N, -1)[:, :3], mean_agg=False,
            equivariant=True)
        grad_h_ptr.reshape(N, -1)[:, :F_NODE].copy_(g["h"])
        grad_coord_ptr.reshape(N, -1)[:, :3].copy_(g["coord"])
        grad_w1_msg_ptr.copy_(g["w1_msg"].reshape(grad_w1_msg_ptr.shape))
        grad_w2_msg_ptr.copy_(g["w2_msg"].reshape(grad_w2_msg_ptr.shape))
        grad_w1_mov_ptr.copy_(g["w1_mov"].reshape(grad_w1_mov_ptr.shape))
        grad_w2_mov_ptr.copy_(g["w2_mov"].reshape(grad_w2_mov_ptr.shape))


egnn_backward_kernel_node_parallel = _Launcher()
