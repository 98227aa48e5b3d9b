"""Timing of graph construction: the device builders against the host builders.

``python -m pymolecular_amd.benchmarks.graph_build`` prints one JSON line per
workload graph: the proteins kNN graph (64 chains x 512 residues, k = 30) and the
slabs radius graph (256 systems x 80 atoms, 6 A, at most 50 neighbours), built
from the same fp64 positions by ``graph_build.knn_graph`` / ``radius_graph``
(HIP events around the call, positions already on the device) and by the
generator's numpy builders (``graphs.knn_rows`` / ``radius_rows``, one host
thread), with a check that both give the same CSR.
"""
from __future__ import annotations

import json
import time

import numpy as np
import torch

from .. import graph_build, graphs


def _time_device(fn, reps=10):
    fn()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        out = fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps, out


def main():
    cases = [
        ("proteins-64x512 kNN-30", graphs.protein_positions(), "knn", (30,), graphs.knn_rows),
        ("slabs-256x80 radius-6A-50", graphs.slab_positions(), "radius", (6.0, 50), graphs.radius_rows),
    ]
    for name, X, mode, args, host in cases:
        n_seg, n = X.shape[:2]
        pos = torch.from_numpy(X.reshape(-1, 3)).cuda()
        seg = torch.arange(n_seg + 1, dtype=torch.int32, device="cuda") * n
        fn = (lambda: graph_build.knn_graph(pos, seg, *args)) if mode == "knn" else \
            (lambda: graph_build.radius_graph(pos, seg, *args))
        ms, (rp, col) = _time_device(fn)
        t0 = time.perf_counter()
        rows, cols = host(X, *args)
        host_ms = (time.perf_counter() - t0) * 1e3
        same = bool(np.array_equal(np.repeat(np.arange(n_seg * n), np.diff(rp.cpu().numpy())), rows)
                    and np.array_equal(col.cpu().numpy(), cols))
        print(json.dumps({"graph": name, "N": n_seg * n, "E": int(col.numel()), "device_ms": round(ms, 4),
                          "host_ms": round(host_ms, 1), "host_threads": 1, "speedup": round(host_ms / ms, 1),
                          "identical_csr": same}), flush=True)


if __name__ == "__main__":
    main()
