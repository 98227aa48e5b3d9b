"""Peak-memory sweep of the reference's test_mem.py on the HIP layer.

``run_memory_benchmark()`` prints, for each node count of test_mem.py:42 at
average degree 32, the peak device memory of the eager per-edge torch
computation and of the fused HIP backward (``launch_triton``), or "OOM" when
an allocation fails (test_mem.py:37-92).

Run: ``python -m pymolecular_amd.benchmarks.test_mem``.
"""
from __future__ import annotations

import sys

import torch

from ..datasets_loaders import generate_graph_data
from ._common import DEFAULT_KWARGS, eager_backward
from .test_speedup import _row_indices, launch_triton

NODE_SIZES = [1000, 5000, 10000, 25000, 50000, 100000, 250000]   # test_mem.py:42


def _peak_mb(fn):
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    torch.cuda.reset_peak_memory_stats()
    try:
        fn()
        torch.cuda.synchronize()
    except torch.OutOfMemoryError:
        return "OOM"
    return f"{torch.cuda.max_memory_allocated() / (1024 ** 2):.2f}"


def run_memory_benchmark(node_sizes=None, avg_degree=32):
    print("\n--- RUNNING MEMORY & OOM BENCHMARK ---")
    print(f"{'Nodes':>10} | {'Edges':>12} | {'PyTorch Peak (MB)':>20} | {'HIP Peak (MB)':>20}")
    print("-" * 70)
    kwargs = dict(DEFAULT_KWARGS)
    rows = []
    for n in (node_sizes or NODE_SIZES):
        data = generate_graph_data(n, avg_degree, kwargs['F_NODE'], kwargs['F_EDGE'], kwargs['HIDDEN_FEATURES'],
                                   kwargs['OUT_FEATURES'], kwargs['HID_FEAT_MOV_MLP'])
        ri = _row_indices(data, n)
        pt = _peak_mb(lambda: eager_backward(data[0], data[1], data[2], ri, data[4], data[6], data[7], data[11],
                                             data[12], data[9], data[8], data[10], data[14], data[15]))
        hip = _peak_mb(lambda: launch_triton(data, kwargs))
        print(f"{n:>10} | {n * avg_degree:>12} | {pt:>20} | {hip:>20}")
        rows.append((n, n * avg_degree, pt, hip))
        del data, ri
    return rows


if __name__ == "__main__":
    run_memory_benchmark()
    sys.exit(0)
