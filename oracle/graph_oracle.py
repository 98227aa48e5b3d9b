"""CPU oracle for graph construction inside segments (float64 numpy).

TEST INFRASTRUCTURE ONLY.  Only ``tests/`` may import this module, and only to
check results; the product path (``pymolecular_amd.graph_build``, the HIP kernels
``egnn_knn_graph`` / ``egnn_radius_graph``) never imports it.

What it restates
----------------
The graph builders of the two geometric workloads (there is no reference
function: the reference draws random CSR graphs, datasets_loaders.py:3-39):

* squared distance of nodes i, j of a segment: ``(dx*dx + dy*dy) + dz*dz`` in
  float64 with ``d = x_i - x_j`` (each operation rounded, no fused multiply-add);
* candidates of node i: the other nodes of its segment in (squared distance,
  index) order;
* kNN: the first ``min(k, n - 1)``; radius: the first ``max_nb`` whose squared
  distance is at most ``cutoff * cutoff``;
* CSR rows in node order, each row's sources ascending.

Written with ``np.lexsort`` on (index, squared distance) per node, independently
of the generator's stable ``argsort`` code.  Pinning (``tests/test_graph_build.py``):
pure-Python brute force with ``math`` on tiny segments with exact ties, and the
workload generator's host builders (``graphs.knn_rows`` / ``graphs.radius_rows``).
"""
from __future__ import annotations

import numpy as np

__all__ = ["segment_dist2", "knn_graph", "radius_graph"]


def segment_dist2(P: np.ndarray) -> np.ndarray:
    """(n, n) squared distances of the rows of P (n, 3), ((dx*dx + dy*dy) + dz*dz)."""
    P = np.asarray(P, np.float64)
    dx = P[:, None, 0] - P[None, :, 0]
    dy = P[:, None, 1] - P[None, :, 1]
    dz = P[:, None, 2] - P[None, :, 2]
    return (dx * dx + dy * dy) + dz * dz


def _build(pos: np.ndarray, seg_ptr: np.ndarray, pick) -> tuple[np.ndarray, np.ndarray]:
    pos = np.asarray(pos, np.float64)
    seg_ptr = np.asarray(seg_ptr, np.int64)
    N = pos.shape[0]
    counts = np.zeros(N, np.int64)
    cols = [None] * N
    for s in range(len(seg_ptr) - 1):
        b, e = int(seg_ptr[s]), int(seg_ptr[s + 1])
        D = segment_dist2(pos[b:e])
        idx = np.arange(e - b)
        for a in range(e - b):
            others = idx[idx != a]
            order = others[np.lexsort((others, D[a, others]))]   # distance, then index
            sel = np.sort(pick(order, D[a])) + b
            cols[b + a] = sel
            counts[b + a] = sel.size
    rowptr = np.zeros(N + 1, np.int64)
    np.cumsum(counts, out=rowptr[1:])
    col = np.concatenate([c for c in cols if c is not None]) if N else np.zeros(0, np.int64)
    return rowptr.astype(np.int32), col.astype(np.int32)


def knn_graph(pos, seg_ptr, k: int):
    """CSR (rowptr, col): each node's min(k, n - 1) nearest other nodes of its segment."""
    return _build(pos, seg_ptr, lambda order, d: order[:k])


def radius_graph(pos, seg_ptr, cutoff: float, max_nb: int):
    """CSR (rowptr, col): each node's nearest max_nb other nodes of its segment within the cutoff."""
    c2 = float(cutoff) * float(cutoff)
    return _build(pos, seg_ptr, lambda order, d: order[:max_nb][d[order[:max_nb]] <= c2])
