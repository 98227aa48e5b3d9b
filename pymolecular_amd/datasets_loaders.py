"""``generate_graph_data`` with the reference's signature and 16-tuple (datasets_loaders.py:3-39).

Same CSR contract (int32 ``row_ptrs`` (N+1) with constant degree, uniform
int32 ``col_indices``, identity ``edge_ids``), same tensors in the same order.
Differences, all deliberate: generation is seeded (numpy PCG64 on the CPU,
then moved to ``device``), so the bytes are reproducible; and
``packed_w1_msg`` holds [w1_msg | w2_msg_src | w_d | w_e] as the kernels'
pointer arithmetic expects (the reference leaves it all zeros,
datasets_loaders.py:30-31, so its backward ran with zero layer-1 weights).
"""
from __future__ import annotations

import numpy as np
import torch


def generate_graph_data(num_nodes, avg_degree, F_NODE, F_EDGE, HIDDEN, OUT_FEAT, HID_MOV, *, seed=0,
                        device="cuda"):
    r = np.random.Generator(np.random.PCG64(seed))
    num_edges = num_nodes * avg_degree
    row_ptrs = np.minimum(np.arange(0, num_nodes + 1, dtype=np.int64) * avg_degree, num_edges).astype(np.int32)
    col_indices = r.integers(0, num_nodes, size=num_edges).astype(np.int32)
    edge_ids = np.arange(num_edges, dtype=np.int32)
    h = r.standard_normal((num_nodes, F_NODE), dtype=np.float32)
    coord = r.standard_normal((num_nodes, 4), dtype=np.float32)
    coord[:, 3] = 0.0
    edge_feat = r.standard_normal((num_edges, F_EDGE), dtype=np.float32)
    w1_msg = r.standard_normal((F_NODE, HIDDEN), dtype=np.float32)
    w2_msg_src = r.standard_normal((F_NODE, HIDDEN), dtype=np.float32)
    w_d = r.standard_normal((HIDDEN,), dtype=np.float32)
    w_e = r.standard_normal((F_EDGE, HIDDEN), dtype=np.float32)
    w_hl = r.standard_normal((HIDDEN, OUT_FEAT), dtype=np.float32)
    w1_mov = r.standard_normal((OUT_FEAT, HID_MOV), dtype=np.float32)
    w2_mov = r.standard_normal((HID_MOV,), dtype=np.float32)
    packed_w1_msg = np.concatenate([w1_msg, w2_msg_src, w_d[None, :], w_e], axis=0).reshape(-1)
    grad_out_msg = r.standard_normal((num_nodes, OUT_FEAT), dtype=np.float32)
    grad_out_mov = r.standard_normal((num_nodes, 3), dtype=np.float32)
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device)  # noqa: E731
    return (T(h), T(coord), T(edge_feat), T(row_ptrs), T(col_indices), T(edge_ids),
            T(w1_msg), T(w2_msg_src), T(w_d), T(w_e), T(w_hl), T(w1_mov), T(w2_mov), T(packed_w1_msg),
            T(grad_out_msg), T(grad_out_mov))
