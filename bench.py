#!/usr/bin/env python
"""Throughput of the fused EGNN layer, forward + backward, on one MI355X.

Workload (default): 1024 fully connected molecules (9..29 atoms, seeds
1002/2002/3002; N = 19,363, E = 383,714), an EGNN stack of 4 E_GCL layers at
H = 128 (embedding_in 5 -> 128, embedding_out 128 -> 128), forward + backward
of the sum-of-outputs loss sum(h_out) + sum(x_out) w.r.t. all parameters, no
optimizer (the metric is the layer's fwd+bwd).  bf16 activations and weights
with fp32 accumulation by default (``--dtype fp32`` for the fp32 run).

value = E * layers / t_step (edges per second through the fused layer, whole
stack timed: fused kernels, per-node GEMMs, node MLPs and autograd glue).
Inputs are resident in HBM before the timed region.

roofline: the dominant kernel class of one step (measured with HIP events on
the stream the kernels run on, through the library's instrumentation hook),
its algorithmic work per launch, and the MI355X peak of its bound.
cpu_baseline: the torch-eager CPU restatement (oracle/torch_ref.py) of the
same stack in fp32 on a bounded prefix of the molecules, on this host's cores.
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "edges/sec fused EGNN layer fwd+bwd; % of MFMA / HBM roofline achieved"
PEAK = {"bf16_mfma_tflops": 2516.6, "fp32_mfma_tflops": 157.3, "hbm_gbs": 8000.0}


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--dtype", choices=["bf16", "fp32"], default="bf16")
    ap.add_argument("--cpu-graphs", type=int, default=512, help="molecules in the CPU-baseline sample")
    ap.add_argument("--cpu-repeats", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true")
    return ap.parse_args()


def per_edge_work(H, O, M, FE, g, s):
    """Algorithmic MFMA FLOPs and HBM bytes per edge of the fused kernels."""
    fwd_flops = 2 * (H * O + g * O * M) + 2 * (g + FE) * H
    bwd_flops = 4 * (H * O + g * O * M) + 2 * (g + FE) * H + 2 * g * H
    gather = 2 * H * s + 8 + g * 24 + FE * s          # P_i, Q_j, erow/col, x_i/x_j, e
    fwd_bytes = gather                                   # row sums stay on chip
    bwd_bytes = gather + O * s + g * 12 + (2 * H + 2 * O + 2 * g * M) * s + g * 20   # + gm_i, gx_i, stores
    model_fwd = 2 * ((2 * H + g + FE) * H + H * O + g * (O * M + M))
    return dict(fwd_flops=fwd_flops, bwd_flops=bwd_flops, fwd_bytes=fwd_bytes, bwd_bytes=bwd_bytes,
                model_fwdbwd=3 * model_fwd)


def cpu_baseline(g, n_graphs, H, layers, repeats, seed=3002):
    import torch
    from oracle.torch_ref import EGNNRef
    torch.set_num_threads(len(os.sched_getaffinity(0)))
    offs = g.info["graph_offsets"]
    n_nodes = int(offs[n_graphs])
    e_end = int(g.rowptr[n_nodes])
    rows = np.repeat(np.arange(n_nodes), np.diff(g.rowptr[:n_nodes + 1]))
    edges = (torch.from_numpy(rows.astype(np.int64)), torch.from_numpy(g.col[:e_end].astype(np.int64)))
    h0 = torch.from_numpy(g.node_feat[:n_nodes])
    x0 = torch.from_numpy(g.coord[:n_nodes])
    torch.manual_seed(seed)
    model = EGNNRef(h0.shape[1], H, H, 0, n_layers=layers)

    def step():
        model.zero_grad(set_to_none=True)
        out_h, out_x = model(h0, x0, edges)
        (out_h.sum() + out_x.sum()).backward()

    step()
    ts = []
    for _ in range(repeats):
        t0 = time.perf_counter()
        step()
        ts.append(time.perf_counter() - t0)
    t = statistics.median(ts)
    return dict(value=e_end * layers / t, unit="edges/s", cores=torch.get_num_threads(), kind="port",
                sample=f"first {n_graphs} of 1024 molecules (N={n_nodes}, E={e_end}), {layers} layers fwd+bwd, "
                       f"fp32 torch eager (oracle/torch_ref.py), median of {repeats} after 1 warm-up; "
                       f"{t * 1e3:.1f} ms per step")


def main():
    a = parse()
    if a.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for --gpus {a.gpus}); multi-GPU sharding is designed "
              "(DESIGN.md) but not part of this build", file=sys.stderr)
        sys.exit(2)
    import torch
    from pymolecular_amd import _capi, graphs
    from pymolecular_amd.models.EGNN import EGNN

    dev = torch.device("cuda:0")
    dt = torch.bfloat16 if a.dtype == "bf16" else torch.float32
    H, L = 128, 4
    g = graphs.make_workload(2)
    N, E = g.N, g.E
    rows = np.repeat(np.arange(N), np.diff(g.rowptr)).astype(np.int64)
    edges = [torch.from_numpy(rows).to(dev), torch.from_numpy(g.col.astype(np.int64)).to(dev)]
    h0 = torch.from_numpy(g.node_feat).to(dev, dt)
    x0 = torch.from_numpy(g.coord).to(dev)
    torch.manual_seed(3002)
    model = EGNN(in_node_nf=h0.shape[1], hidden_nf=H, out_node_nf=H, in_edge_nf=0, n_layers=L).to(dev, dt)

    def step():
        model.zero_grad(set_to_none=True)
        out_h, out_x = model(h0, x0, edges, None)
        (out_h.float().sum() + out_x.float().sum()).backward()

    for _ in range(a.warmup):
        step()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(a.steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / a.steps
    value = E * L / (ms / 1e3)

    # per-kernel device time (HIP events on the launch stream, via the library hook)
    _capi.profile_enable(True)
    nprof = max(3, min(a.steps, 10))
    for _ in range(nprof):
        step()
    torch.cuda.synchronize()
    prof = _capi.profile_read()
    _capi.profile_enable(False)
    s = 2 if dt == torch.bfloat16 else 4
    w = per_edge_work(H, H, H, 0, 1, s)
    kern = {k: dict(ms_per_launch=(t / n if n else 0.0), launches_per_step=n / nprof,
                    share=0.0) for k, (t, n) in prof.items()}
    tot = sum(t for t, _ in prof.values()) / nprof
    for k, (t, n) in prof.items():
        kern[k]["share"] = (t / nprof) / ms if ms else 0.0
    dom = max(prof, key=lambda k: prof[k][0])
    dur_s = kern[dom]["ms_per_launch"] / 1e3
    peak_mfma = PEAK["bf16_mfma_tflops"] if s == 2 else PEAK["fp32_mfma_tflops"]
    flops = {"bwd_edge": w["bwd_flops"], "fwd_edge": w["fwd_flops"]}.get(dom, 0) * E
    nbytes = {"bwd_edge": w["bwd_bytes"], "fwd_edge": w["fwd_bytes"]}.get(dom, 0) * E
    t_mfma = flops / (peak_mfma * 1e12)
    t_hbm = nbytes / (PEAK["hbm_gbs"] * 1e9)
    if t_hbm >= t_mfma:
        roof = dict(bound="hbm", achieved=nbytes / dur_s / 1e9, peak=PEAK["hbm_gbs"], unit="GB/s")
    else:
        roof = dict(bound="mfma", achieved=flops / dur_s / 1e12, peak=peak_mfma, unit="TFLOP/s")
    roof["frac"] = roof["achieved"] / roof["peak"]
    roof["traffic"] = None
    roof["kernel"] = dom
    roof["ms_per_launch"] = kern[dom]["ms_per_launch"]
    roof["mfma_frac"] = (flops / dur_s / 1e12) / peak_mfma if dur_s else 0.0
    roof["hbm_frac"] = (nbytes / dur_s / 1e9) / PEAK["hbm_gbs"] if dur_s else 0.0
    model_mfu = (w["model_fwdbwd"] * E * L) / (ms / 1e3) / (peak_mfma * 1e12)

    out = {
        "metric": METRIC, "value": value, "unit": "edges/s", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
        "ms_per_step": ms, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": a.dtype, "data": "synthetic (seeded numpy PCG64 molecules; random-init weights, seed 3002)",
        "config": {"workload": "molecules-1024: 4 x E_GCL, H=128, fully connected molecules, fwd+bwd of "
                               "sum-of-outputs loss", "N": N, "E": E, "layers": L, "H": H, "F_E": 0,
                   "dtype": a.dtype},
        "roofline": roof,
        "model_flops_mfma_frac": model_mfu,
        "kernels": {k: {kk: round(vv, 5) for kk, vv in v.items()} for k, v in kern.items()},
        "kernel_ms_per_step": tot,
    }
    if not a.no_cpu:
        out["cpu_baseline"] = cpu_baseline(g, a.cpu_graphs, H, L, a.cpu_repeats)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
