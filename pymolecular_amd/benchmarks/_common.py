"""Shared pieces of the benchmark drivers: the eager comparison provider and HIP-event timing."""
from __future__ import annotations

import statistics
from typing import Callable, Sequence

import torch

# hyper-parameters of both reference drivers (test_speedup.py:25-30, test_mem.py:44-49)
DEFAULT_KWARGS = {
    'F_NODE': 32, 'F_EDGE': 16,
    'HIDDEN_FEATURES': 64, 'OUT_FEATURES': 32, 'HID_FEAT_MOV_MLP': 32,
    'MSG_BETA': 1.0, 'MOV_BETA': 1.0, 'MOV_ACT_TYPE': 0, 'MSG_ACT_TYPE': 0,
}


def eager_backward(h, coord, edge_feat, row_indices, col_indices, w1_msg, w2_msg, w1_mov, w2_mov, w_e, w_d, w_hl,
                   grad_out_msg, grad_out_mov):
    """The "PyTorch Native" provider of the drivers: the layer written as plain
    torch ops that materialise every per-edge tensor, forward then autograd
    backward (the computation of pytorch_baseline.py:18-48).  It is the
    comparison point of the speed and memory sweeps, never a substitute for
    the fused layer.  Returns (dL/dh, dL/dcoord)."""
    h = h.detach().requires_grad_(True)
    coord = coord.detach().requires_grad_(True)
    rows, cols = row_indices.long(), col_indices.long()
    delta = coord[rows, :3] - coord[cols, :3]
    sq = (delta * delta).sum(dim=1, keepdim=True)
    pre1 = h[rows] @ w1_msg + h[cols] @ w2_msg + sq * w_d + edge_feat @ w_e
    m = torch.nn.functional.silu(torch.nn.functional.silu(pre1) @ w_hl)
    force = (torch.nn.functional.silu(m @ w1_mov) * w2_mov).sum(dim=1, keepdim=True)
    n = h.shape[0]
    out_msg = torch.zeros(n, m.shape[1], device=h.device, dtype=m.dtype).index_add_(0, rows, m)
    out_mov = torch.zeros(n, 3, device=h.device, dtype=delta.dtype).index_add_(0, rows, delta * force)
    loss = (out_msg * grad_out_msg).sum() + (out_mov * grad_out_mov[:, :3]).sum()
    loss.backward()
    return h.grad, coord.grad


def do_bench(fn: Callable[[], object], quantiles: Sequence[float] = (0.5, 0.2, 0.8), warmup: int = 3,
             rep: int = 20) -> list:
    """Milliseconds per call at the given quantiles, timed with HIP events on
    the current stream (the role of triton.testing.do_bench in the reference)."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    times = []
    for _ in range(rep):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        fn()
        b.record()
        b.synchronize()
        times.append(a.elapsed_time(b))
    times.sort()
    out = []
    for q in quantiles:
        pos = q * (len(times) - 1)
        lo = int(pos)
        hi = min(lo + 1, len(times) - 1)
        out.append(times[lo] + (times[hi] - times[lo]) * (pos - lo))
    return out


def median(xs):
    return statistics.median(xs)
