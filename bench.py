#!/usr/bin/env python
"""Throughput of the fused EGNN/MPNN layer, forward + backward, on one MI355X.

Default workload: the skewed-degree power-law MPNN, one graph of N = 2,000,000
nodes and E = 18,566,352 edges (in-degree ~ d^-2.1 on [2, 4096]), 2 MPNN
layers at H = 128 with 16-dim N(0, 1) edge features, bf16 activations and
weights with fp32 accumulation -- the largest of the five workloads, all of
which fit one GPU.  ``--workload k`` (``--dtype``) selects another one:
1 molecules-128 (1 E_GCL, fp32), 2 molecules-1024 (4 E_GCL, fp32 or bf16),
3 proteins kNN-30 (4 E_GCL, 16 RBFs), 4 slabs (6 E_GCL, H = 256, 32 RBFs);
``--all`` prints one line for each workload and dtype.

A step is forward + backward of the sum-of-outputs loss of the whole stack
(embeddings, fused layers, node updates) with respect to all parameters,
inputs resident in HBM before the timed region.  value = E * layers / t_step:
edges per second through the fused layer.

roofline: the dominant edge kernel of the step (the fused backward), its
time per layer from HIP events recorded on the stream it runs on during the
timed steps (the library's instrumentation hook; one launch per layer, or
one per edge chunk of the one-wave-per-tile backward) -- plus, on the paths
whose backward kernel stores per-edge factors (H = 256, and fp32), the
weight-gradient products over those factors that finish its work (class
edge_wgrad) -- and its algorithmic work per layer from the per-edge model of
the reference formulation:
    FLOP_fwd(e) = 2 [(2F + g + F_E) H + H O + g (O M + M)],  FLOP_bwd = 2 FLOP_fwd
    B_fwd = E (8 + F s + c + F_E s) + N (4 + F s + 2c + O s)
    B_bwd = E (8 + F s + c + F_E s + 4F + c) + N (4 + F s + 3c + O s + 4F)
(g = 1 for EGNN, 0 for MPNN; c = 16 g; s = bytes per activation), bounded by
whichever of HBM (8 TB/s) and MFMA (bf16 2516.6, fp32 157.3 TFLOP/s) takes
longer for that work.  ``executed`` gives the same kernel's work as this
build executes it (projections hoisted to the nodes, scratch traffic).
``traffic`` is the measured HBM bytes per launch from the rocprofv3
FETCH_SIZE / WRITE_SIZE summary under profiles/ when one exists.
cpu_baseline: the torch-eager CPU restatement (oracle/torch_ref.py) of the
same stack in fp32 on a deterministic row subset of the same workload (at
least 10 % of its edges), on this host's cores.
"""
from __future__ import annotations

import argparse
import json
import os
import re
import statistics
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "edges/sec fused EGNN layer fwd+bwd; % of MFMA / HBM roofline achieved"
PEAK = {"bf16_mfma_tflops": 2516.6, "fp32_mfma_tflops": 157.3, "hbm_gbs": 8000.0}
DESCR = {
    1: "molecules-128: 1 x E_GCL, H=128, fully connected molecules (9..29 atoms), F_E=0",
    2: "molecules-1024: 4 x E_GCL, H=128, fully connected molecules (9..29 atoms), F_E=0",
    3: "proteins-64x512: 4 x E_GCL, H=128, kNN-30 chains, F_E=16 RBF",
    4: "slabs-256x80: 6 x E_GCL, H=256, radius 6 A capped at 50, F_E=32 RBF",
    5: "powerlaw-2M: 2 x MPNN layer, H=128, power-law in-degree (alpha 2.1, 2..4096), F_E=16",
}
ALL = [(1, "fp32"), (2, "fp32"), (2, "bf16"), (3, "bf16"), (4, "bf16"), (5, "bf16")]


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", type=int, default=5, choices=[1, 2, 3, 4, 5])
    ap.add_argument("--dtype", choices=["bf16", "fp32"], default=None,
                    help="default: bf16, except fp32 for the one-layer molecules-128 workload")
    ap.add_argument("--all", action="store_true", help="one line per workload and dtype")
    ap.add_argument("--cpu-frac", type=float, default=0.10, help="least fraction of the edges in the CPU sample")
    ap.add_argument("--cpu-min-edges", type=int, default=200_000, help="least edges in the CPU sample")
    ap.add_argument("--cpu-repeats", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--probe", action="store_true",
                    help="also time the identity-MLP instrument of the MPNN edge kernels (gather / segment-sum "
                         "data movement alone) at the power-law workload and print its line")
    ap.add_argument("--probe-only", action="store_true", help="run only the identity-MLP instrument (no workload line)")
    ap.add_argument("--copy-probe", action="store_true",
                    help="end with three 256 MiB device copies (scale reference for HBM byte counters)")
    return ap.parse_args()


def path_model(cls, N, E, F, H, O, M, FE, g, s):
    """(FLOPs, bytes) of one launch of an edge kernel under the reference formulation's per-edge model.

    FLOPs: the concat-input MLPs per edge (pytorch_baseline.py:27-35), the backward twice the forward.
    Bytes: every gathered row counted once per edge, node rows once per node, the dh_j fp32 write
    once per edge (c = 16 g: a padded fp32 coordinate row)."""
    c = 16 * g
    flop_fwd = 2 * ((2 * F + g + FE) * H + H * O + g * (O * M + M))
    if cls == "fwd_edge":
        return flop_fwd * E, E * (8 + F * s + c + FE * s) + N * (4 + F * s + 2 * c + O * s)
    if cls == "bwd_edge":
        return 2 * flop_fwd * E, E * (8 + F * s + c + FE * s + 4 * F + c) + N * (4 + F * s + 3 * c + O * s + 4 * F)
    return 0, 0


def kernel_work(cls, path, N, E, F, H, O, M, FE, g, s):
    """Executed algorithmic (MFMA FLOPs, HBM bytes) of one launch of a kernel class, as this build runs it.

    FLOPs count the products the kernel must execute with the first layer's node projections hoisted
    out of the edge loop (identity transposes and segment-sum products are overhead, not work).  Bytes
    count every gathered row once per edge: P_i, Q_j (H each), col and row id (8), edge id and
    features, the geometry record; scratch stores (Gh, Gx, factors) included; node outputs once."""
    eb = 8 + (4 + FE * s if FE else 0) + 24 * g
    # the edge-parallel MPNN backward (H = 128) sums dL/dpre1 over each row itself: dP rows and, for the
    # rows split over tiles, fp32 carries (about two per 32-edge tile) out; the node reduction then
    # reads Gh once, by source
    dst = path == "coop" and g == 0 and H == 128
    if cls == "fwd_edge":
        flops = 2 * ((g + FE) * H + H * O + g * O * M)
        return flops * E, E * (2 * H * s + eb) + N * (O * s + 12 * g)
    if cls == "bwd_edge":
        per_edge = 2 * H * s + eb + O * s + 12 * g + H * s + 16 * g      # + grad rows of i, Gh and Gx stores
        if path == "coop":   # weight gradients accumulated in registers
            flops = 4 * (g + FE) * H + 6 * H * O + 6 * g * O * M
        elif path == "wide":  # factors m1, m, g_q, g_a2 stored for the split-K products (dw2_mov, dw_d in the kernel)
            flops = 2 * (g + FE) * H + 4 * H * O + 4 * g * O * M
            per_edge += (H + O + g * M + O) * s
        else:         # one wave per tile: factors m1, m, g_q, p, g_a2 and r^2 stored for the split-K products
            flops = 2 * (g + FE) * H + 4 * H * O + 4 * g * O * M
            per_edge += (H + O + 2 * g * M + O) * s + 4 * g
        if dst:
            return flops * E, E * (per_edge + H / 4) + N * H * s
        return flops * E, E * per_edge
    if cls == "node_reduce":
        if dst:
            return 0, E * (H * s + 4) + N * (H * s + 8)
        return 0, E * (2 * H * s + 4 + 32 * g) + N * (2 * H * s + 12 * g + 8)
    if cls == "node_gemm":
        return 2 * N * F * 2 * H, N * (F + 2 * H) * s
    if cls == "wgrad":   # whole layer: dh and [dW_n1 | dW_n2; db1] over the nodes
        return 2 * N * (F + 1) * 2 * H + 2 * N * 2 * H * F, N * (F + 2 * H) * s + N * (2 * H + F) * s
    if cls == "edge_wgrad":   # whole layer: the weight-gradient products over the factors the edge kernel stored
        flops = nbytes = 0
        if path == "wide":     # [dW_hl; db2], [dW1_mov; dbx1] over the edge factors; dW_e over Gh
            flops = 2 * E * ((H + 1) * O + g * (O + 1) * M + H * FE)
            nbytes = E * ((H + O) * s + g * (O + M) * s + (H * s + FE * s + 4 if FE else 0))
        elif path == "one":    # the same, plus the dw2_mov and dw_d matrix-vector products over p, Gh and r^2
            flops = 2 * E * ((H + 1) * O + g * ((O + 1) * M + M + H) + H * FE)
            nbytes = E * ((H + O) * s + g * ((O + M) * s + M * s + 4 + H * s + 4) + (H * s + FE * s + 4 if FE else 0))
        return flops, nbytes
    return 0, 0


def model_flops_per_edge(F, H, O, M, FE, g):
    """Model-FLOPs convention of the concat formulation, forward + backward = 3 x forward."""
    return 3 * 2 * ((2 * F + g + FE) * H + H * O + g * (O * M + M))


def read_traffic(name, dtype, cls):
    """HBM bytes per launch from a profiles/ summary line 'TRAFFIC <workload> <dtype> <class> <bytes>'."""
    d = os.path.join(ROOT, "profiles")
    if not os.path.isdir(d):
        return None
    pat = re.compile(rf"^TRAFFIC\s+{re.escape(name)}\s+{dtype}\s+{cls}\s+([0-9.eE+]+)\s*$")
    for fn in sorted(os.listdir(d)):
        if not fn.endswith((".md", ".txt")):
            continue
        with open(os.path.join(d, fn)) as f:
            for line in f:
                m = pat.match(line.strip())
                if m:
                    return float(m.group(1))
    return None


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _closed_prefix(rowptr, col, n_edges):
    """Smallest row prefix [0, r) with at least n_edges edges whose sources all lie in [0, r), or 0."""
    N = rowptr.shape[0] - 1
    deg = np.diff(rowptr)
    rowmax = np.full(N, -1, dtype=np.int64)
    nz = deg > 0
    rowmax[nz] = np.maximum.reduceat(col.astype(np.int64), rowptr[:-1][nz])
    mx = np.maximum.accumulate(rowmax)
    r_ok = np.nonzero(mx < np.arange(1, N + 1))[0] + 1     # prefixes closed under sources
    r_ok = r_ok[rowptr[r_ok] >= n_edges]
    return int(r_ok[0]) if r_ok.size else 0


def cpu_sample(g, n_edges):
    """A deterministic subgraph with at least n_edges edges: (rows, cols, node ids, edge range, description).

    Batched graphs: the smallest prefix of whole graphs.  One connected graph: the first r rows holding
    n_edges edges, each source j read as node j mod r, so the sample has the graph's ratio of nodes to
    edges (its node-side work per edge) and the same per-edge work."""
    r = _closed_prefix(g.rowptr, g.col, n_edges)
    if r and int(g.rowptr[r]) <= 2 * n_edges:
        e_end = int(g.rowptr[r])
        rows = np.repeat(np.arange(r), np.diff(g.rowptr[:r + 1]))
        return rows, g.col[:e_end].astype(np.int64), np.arange(r), e_end, f"first {r} nodes (whole graphs)"
    r = int(np.searchsorted(g.rowptr, n_edges, side="left"))
    e_end = int(g.rowptr[r])
    rows = np.repeat(np.arange(r), np.diff(g.rowptr[:r + 1]))
    cols = (g.col[:e_end].astype(np.int64) % r)
    return rows, cols, np.arange(r), e_end, f"first {r} destination rows, source j read as node j mod {r}"


def cpu_baseline(k, g, H, layers, eq, frac, min_edges, repeats, seed):
    import torch
    from oracle.torch_ref import EGNNRef, MPNNRef
    torch.set_num_threads(len(os.sched_getaffinity(0)))
    target = min(g.E, max(int(np.ceil(frac * g.E)), min_edges))
    rows, cols, nodes, e_end, how = cpu_sample(g, target)
    edges = (torch.from_numpy(rows.astype(np.int64)), torch.from_numpy(cols))
    h0 = torch.from_numpy(g.node_feat[nodes])
    ea = None if g.edge_attr is None else torch.from_numpy(g.edge_attr[:e_end])
    FE = 0 if ea is None else ea.shape[1]
    torch.manual_seed(seed)
    if eq:
        x0 = torch.from_numpy(g.coord[nodes])
        model = EGNNRef(h0.shape[1], H, H, FE, n_layers=layers)
        run = lambda: sum(t.sum() for t in model(h0, x0, edges, ea))  # noqa: E731
    else:
        model = MPNNRef(h0.shape[1], H, H, FE, n_layers=layers)
        run = lambda: model(h0, edges, ea).sum()  # noqa: E731

    def step():
        model.zero_grad(set_to_none=True)
        run().backward()

    step()
    ts = []
    for _ in range(repeats):
        t0 = time.perf_counter()
        step()
        ts.append(time.perf_counter() - t0)
    t = statistics.median(ts)
    return dict(value=e_end * layers / t, unit="edges/s", cores=torch.get_num_threads(), kind="port",
                cpu_model=cpu_model(),
                sample=f"{how}: N={nodes.size}, E={e_end} ({100.0 * e_end / g.E:.1f} % of the workload's edges), "
                       f"{layers} layers fwd+bwd, fp32 torch eager (oracle/torch_ref.py), median of {repeats} "
                       f"after 1 warm-up; {t * 1e3:.1f} ms per step; value = sample edges x layers / time")


def run_workload(k, dtype, a, g=None):
    import torch
    from pymolecular_amd import _capi, graphs
    from pymolecular_amd.models.EGNN import EGNN, MPNN

    W = graphs.WORKLOADS[k]
    dtype = dtype or W["dtypes"][-1]
    dev = torch.device("cuda:0")
    dt = torch.bfloat16 if dtype == "bf16" else torch.float32
    H, L, eq = W["H"], W["layers"], W["eq"]
    g = g if g is not None else graphs.make_workload(k)
    N, E = g.N, g.E
    F0 = g.node_feat.shape[1]
    FE = 0 if g.edge_attr is None else g.edge_attr.shape[1]
    edges = [torch.from_numpy(g.rows().astype(np.int64)).to(dev), torch.from_numpy(g.col.astype(np.int64)).to(dev)]
    h0 = torch.from_numpy(g.node_feat).to(dev, dt)
    ea = None if g.edge_attr is None else torch.from_numpy(g.edge_attr).to(dev, dt)
    torch.manual_seed(3000 + k)
    if eq:
        x0 = torch.from_numpy(g.coord).to(dev)
        model = EGNN(in_node_nf=F0, hidden_nf=H, out_node_nf=H, in_edge_nf=FE, n_layers=L).to(dev, dt)
        loss = lambda: sum(t.sum(dtype=torch.float32) for t in model(h0, x0, edges, ea))  # noqa: E731
    else:
        model = MPNN(in_node_nf=F0, hidden_nf=H, out_node_nf=H, in_edge_nf=FE, n_layers=L).to(dev, dt)
        loss = lambda: model(h0, edges, ea).sum(dtype=torch.float32)  # noqa: E731

    def step():
        model.zero_grad(set_to_none=True)
        loss().backward()

    # The library's event hook records the roofline's kernels (the fused backward edge kernel and the
    # factor products it hands weight-gradient work to) through the warm-up and the timed steps, on the
    # stream each kernel runs on; the warm-up fills its event pool so the timed steps create none.  Each
    # recorded event waits for the work before it, so the timed steps record only these classes (at
    # molecules-1024 recording the forward edge kernels as well cost ~20 us of a ~1.85 ms step).  Every
    # kernel class is timed in a separate untimed pass afterwards.
    edge_classes = [_capi.K_BWD_EDGE, _capi.K_EDGE_WGRAD]
    _capi.profile_enable(True, edge_classes)
    for _ in range(a.warmup):
        step()
    torch.cuda.synchronize()
    _capi.profile_enable(True, edge_classes)    # keep only the timed steps' records
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(a.steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / a.steps
    value = E * L / (ms / 1e3)
    timed = _capi.profile_read()
    nprof = max(2, min(a.steps, 5))
    _capi.profile_enable(True)
    for _ in range(nprof):
        step()
    torch.cuda.synchronize()
    prof = _capi.profile_read()
    _capi.profile_enable(False)
    for cls in ("bwd_edge", "edge_wgrad"):   # the roofline's kernels: the timed steps' own records
        prof[cls] = (timed[cls][0] * nprof / a.steps, timed[cls][1] * nprof / a.steps)

    s = 2 if dt == torch.bfloat16 else 4
    g1 = 1 if eq else 0
    path = "coop" if s == 2 and H == 128 and FE + 2 * g1 <= 32 else "wide" if s == 2 and H == 256 else "one"
    peak_mfma = PEAK["bf16_mfma_tflops"] if s == 2 else PEAK["fp32_mfma_tflops"]

    def executed_per_launch(cls, launches_per_step):
        fl, by = kernel_work(cls, path, N, E, H, H, H, H, FE, g1, s)
        if cls in ("wgrad", "edge_wgrad", "bwd_edge"):   # whole-layer work over the layer's launches
            return fl * L / launches_per_step, by * L / launches_per_step
        return fl, by

    def bound(fl, by, dur_s):
        t_hbm, t_mfma = by / (PEAK["hbm_gbs"] * 1e9), fl / (peak_mfma * 1e12)
        if t_hbm >= t_mfma:
            return dict(bound="hbm", achieved=by / dur_s / 1e9, peak=PEAK["hbm_gbs"], unit="GB/s",
                        frac=t_hbm / dur_s)
        return dict(bound="mfma", achieved=fl / dur_s / 1e12, peak=peak_mfma, unit="TFLOP/s", frac=t_mfma / dur_s)

    kern, portions = {}, {}
    for cls, (t, n) in prof.items():
        if not n:
            continue
        per = t / n
        kern[cls] = dict(ms_per_launch=per, launches_per_step=n / nprof, share=(t / nprof) / ms)
        fl, by = executed_per_launch(cls, n / nprof)
        if fl or by:
            portions[cls] = dict(mfma_frac=fl / (per / 1e3) / (peak_mfma * 1e12),
                                 hbm_frac=by / (per / 1e3) / (PEAK["hbm_gbs"] * 1e9), flops=fl, bytes=by)
    edge_cls = [c for c in ("bwd_edge", "fwd_edge") if c in kern]
    dom = max(edge_cls, key=lambda c: kern[c]["ms_per_launch"] * kern[c]["launches_per_step"])
    # one layer's launches of the class (one, or one per edge chunk of the one-wave-per-tile backward)
    per_layer = kern[dom]["launches_per_step"] / L
    dur_s = kern[dom]["ms_per_launch"] * per_layer / 1e3
    xf, xb = kernel_work(dom, path, N, E, H, H, H, H, FE, g1, s)     # the layer's work
    handed = dom == "bwd_edge" and "edge_wgrad" in kern
    if handed:   # the factor products finish the backward kernel's weight gradients: the same layer's work
        dur_s += kern["edge_wgrad"]["ms_per_launch"] * kern["edge_wgrad"]["launches_per_step"] / L / 1e3
        ef, eb = kernel_work("edge_wgrad", path, N, E, H, H, H, H, FE, g1, s)
        xf, xb = xf + ef, xb + eb
    fl, by = path_model(dom, N, E, H, H, H, H, FE, g1, s)
    roof = bound(fl, by, dur_s)
    name = DESCR[k].split(":")[0]
    traffic = [read_traffic(name, dtype, c) for c in ((dom, "edge_wgrad") if handed else (dom,))]
    roof["traffic"] = None if None in traffic else sum(traffic)
    roof.update(kernel=dom + ("+edge_wgrad" if handed else ""), ms_per_launch=kern[dom]["ms_per_launch"],
                launches_per_layer=per_layer, ms_per_layer=dur_s * 1e3, algorithmic_flops=fl, algorithmic_bytes=by,
                executed=dict(flops=xf, bytes=xb, **{kk: v for kk, v in bound(xf, xb, dur_s).items()
                                                     if kk in ("bound", "frac")}))
    # the whole step against the per-edge model of every layer's forward and backward
    fwf, fwb = path_model("fwd_edge", N, E, H, H, H, H, FE, g1, s)
    bwf, bwb = path_model("bwd_edge", N, E, H, H, H, H, FE, g1, s)
    step_roof = bound((fwf + bwf) * L, (fwb + bwb) * L, ms / 1e3)
    model_mfu = model_flops_per_edge(H, H, H, H, FE, g1) * E * L / (ms / 1e3) / (peak_mfma * 1e12)

    out = {
        "metric": METRIC, "value": value, "unit": "edges/s", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
        "ms_per_step": ms, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": dtype, "data": f"synthetic (seeded numpy PCG64 graphs, seeds {1000 + k}/{2000 + k}; "
                                f"random-init weights, seed {3000 + k})",
        "config": {"workload": DESCR[k] + ", fwd+bwd of the sum-of-outputs loss", "N": N, "E": E, "layers": L,
                   "H": H, "F_E": FE, "dtype": dtype},
        "roofline": roof,
        "step_roofline": {kk: step_roof[kk] for kk in ("bound", "frac")},
        "portions": portions,
        "model_flops_mfma_frac": model_mfu,
        "kernels": {c: {kk: round(vv, 5) for kk, vv in v.items()} for c, v in kern.items()},
        "kernel_ms_per_step": sum(t for t, _ in prof.values()) / nprof,
    }
    if not a.no_cpu:
        out["cpu_baseline"] = cpu_baseline(k, g, H, L, eq, a.cpu_frac, a.cpu_min_edges, a.cpu_repeats, 3000 + k)
    del model, edges, h0, ea
    torch.cuda.empty_cache()
    return out


def probe_identity(a, k=5):
    """Gather / segment-sum data movement of the MPNN layer alone: the edge-parallel kernels with the MLP
    replaced by identity (EGNN_FLAG_PROBE_IDENTITY, an instrument: the same kernels, the same gathers, row
    sums, stores and carries, without the products and elementwise work of the MLP), one layer forward +
    backward per step, on the full power-law graph.  Bytes per kernel, every gathered row counted once
    per edge:
      forward:      E (8 + 2 H s + F_E s) + N O s        (indices, P_i and Q_j, edge features; row sums out)
      backward:     E (8 + 2 H s + F_E s + O s + H s + H / 4) + N H s
                                                        (indices, P_i and Q_j, edge features, the row's
                                                        message gradient; dL/dpre1 out, its row sums: dP
                                                        rows and fp32 carries of the split rows)
      node reduce:  E (H s + 4) + N (8 + H s)           (dL/dpre1 by source, CSC ids; dQ out)
      fix-ups:      E H / 4 per step                    (the fp32 carries of the backward's split rows)
    The two fix-up launches of a step are timed together: the backward's completes every row split over
    tiles, the forward's only the rows that cross a wave's range of tiles (a few thousand rows, whose bytes
    are left out of the count, so its rate is understated)."""
    import torch
    from pymolecular_amd import _capi, fused, graphs
    g = graphs.make_workload(k)
    N, E, H, s = g.N, g.E, 128, 2
    FE = g.edge_attr.shape[1]
    dev = torch.device("cuda:0")
    gen = torch.Generator(device="cuda").manual_seed(11)
    h = torch.randn((N, H), generator=gen, device=dev).to(torch.bfloat16)
    ef = torch.from_numpy(g.edge_attr).to(dev, torch.bfloat16)
    w1 = (torch.randn((2 * H + FE, H), generator=gen, device=dev) * 0.05).to(torch.bfloat16)
    w2 = (torch.randn((H, H), generator=gen, device=dev) * 0.05).to(torch.bfloat16)
    gm = torch.randn((N, H), generator=gen, device=dev).to(torch.bfloat16)
    rowptr, col = torch.from_numpy(g.rowptr).to(dev), torch.from_numpy(g.col).to(dev)

    def step():
        fused.egnn_fused_forward(h, None, ef, rowptr, col, None, w1, w2, equivariant=False, probe_identity=True)
        fused.egnn_fused_backward(h, None, ef, rowptr, col, None, w1, w2, None, None, None, None, None, gm, None,
                                  equivariant=False, probe_identity=True)

    for _ in range(a.warmup):
        step()
    torch.cuda.synchronize()
    _capi.profile_enable(True, [_capi.K_FWD_EDGE, _capi.K_FWD_FIXUP, _capi.K_BWD_EDGE, _capi.K_NODE_REDUCE])
    for _ in range(a.steps):
        step()
    torch.cuda.synchronize()
    prof = _capi.profile_read()
    _capi.profile_enable(False)
    model = {"fwd_edge": E * (8 + 2 * H * s + FE * s) + N * H * s,
             "fwd_fixup": E * H / 4,
             "bwd_edge": E * (8 + 2 * H * s + FE * s + H * s + H * s + H / 4) + N * H * s,
             "node_reduce": E * (H * s + 4) + N * (8 + H * s)}
    out = {}
    tot_b = tot_t = 0.0
    for cls, nbytes in model.items():
        t, n = prof[cls]
        if cls == "fwd_fixup":   # both launches of a step (forward and backward), per step
            ms = t / max(a.steps, 1)
            key = "ms_per_step"
        else:
            ms = t / max(n, 1)
            key = "ms_per_launch"
        gbs = nbytes / (ms / 1e3) / 1e9
        out[cls] = {key: ms, "launches": n, "algorithmic_bytes": nbytes, "achieved_gbs": gbs,
                    "frac": gbs / PEAK["hbm_gbs"]}
        tot_b += nbytes
        tot_t += ms
    gbs = tot_b / (tot_t / 1e3) / 1e9
    return {"metric": "HBM fraction of the gather / segment-sum portion (identity-MLP instrument of the "
                      "edge-parallel MPNN kernels)", "value": gbs / PEAK["hbm_gbs"], "unit": "fraction of 8 TB/s",
            "achieved_gbs": gbs, "config": {"workload": DESCR[k], "N": N, "E": E, "steps": a.steps},
            "kernels": out}


def main():
    a = parse()
    if a.gpus != 1:
        print(f"bench.py measures one GPU (asked for --gpus {a.gpus}): every workload fits one MI355X, and the "
              "multi-GPU sharding of this layer is designed but not built", file=sys.stderr)
        sys.exit(2)
    import torch
    todo = [] if a.probe_only else ALL if a.all else [(a.workload, a.dtype)]
    for k, dtype in todo:
        out = run_workload(k, dtype, a)
        print(json.dumps(out), flush=True)
    if a.probe or a.probe_only:
        print(json.dumps(probe_identity(a)), flush=True)
    if a.copy_probe:
        src = torch.empty(64 << 20, dtype=torch.float32, device="cuda:0").fill_(1.0)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()


if __name__ == "__main__":
    main()
