"""Graph construction on the device: kNN and radius graphs inside segments.

The host builders of the workload generator (``graphs.protein_chains``: kNN with
k = 30 inside each chain; ``graphs.catalyst_slabs``: the nearest ``max_nb`` atoms
within a cutoff inside each system) as HIP kernels (``egnn_knn_graph`` /
``egnn_radius_graph`` in include/egnn.h), with the same CSR, bit for bit: fp64
squared distances ((dx*dx + dy*dy) + dz*dz) without fused multiply-adds, ties
broken by the lower index, each row's sources in ascending order.  There is no
reference function for this step (the reference draws random CSR graphs,
datasets_loaders.py:3-39).  No CPU path: ROCm tensors only.
"""
from __future__ import annotations

import ctypes

import torch

from . import _capi
from ._capi import check

__all__ = ["knn_graph", "radius_graph"]


def _prep(pos: torch.Tensor, seg_ptr: torch.Tensor):
    if not pos.is_cuda:
        raise RuntimeError("pos must be a ROCm device tensor: graph construction has no CPU path")
    if pos.dim() != 2 or pos.shape[1] != 3:
        raise ValueError(f"pos must be (N, 3), got {tuple(pos.shape)}")
    pos = pos.to(torch.float64).contiguous()
    seg = seg_ptr.to(device=pos.device, dtype=torch.int32).contiguous()
    if seg.dim() != 1 or seg.numel() < 2:
        raise ValueError("seg_ptr must hold n_seg + 1 >= 2 offsets")
    max_seg = int(torch.diff(seg).max().item())
    return pos, seg, max_seg


def _build(fn, pos, seg, max_seg, m, extra):
    N = pos.shape[0]
    L = _capi.lib()
    dev = pos.device
    rowptr = torch.empty(N + 1, dtype=torch.int32, device=dev)
    col = torch.empty(max(N * m, 1), dtype=torch.int32, device=dev)
    nbytes = L.egnn_graph_tmp_bytes(N)
    tmp = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=dev)
    ne = ctypes.c_int64(0)
    st = torch.cuda.current_stream(dev).cuda_stream
    rc = getattr(L, fn)(pos.data_ptr(), N, seg.data_ptr(), seg.numel() - 1, max_seg, *extra, rowptr.data_ptr(),
                        col.data_ptr(), col.numel(), tmp.data_ptr(), nbytes, ctypes.byref(ne), st)
    check(fn, rc)
    return rowptr, col[:ne.value]


def knn_graph(pos: torch.Tensor, seg_ptr: torch.Tensor, k: int):
    """CSR ``(rowptr, col)`` of each node's ``min(k, n - 1)`` nearest other nodes of its segment."""
    pos, seg, max_seg = _prep(pos, seg_ptr)
    return _build("egnn_knn_graph", pos, seg, max_seg, k, (int(k),))


def radius_graph(pos: torch.Tensor, seg_ptr: torch.Tensor, cutoff: float, max_nb: int):
    """CSR ``(rowptr, col)`` of each node's nearest ``max_nb`` other nodes of its segment within ``cutoff``."""
    pos, seg, max_seg = _prep(pos, seg_ptr)
    return _build("egnn_radius_graph", pos, seg, max_seg, max_nb, (ctypes.c_double(float(cutoff)), int(max_nb)))
