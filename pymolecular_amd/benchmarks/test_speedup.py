"""Speed sweep of the reference's test_speedup.py on the HIP layer.

Same entry points: ``launch_triton(data_tuple, kwargs_dict)`` (the backward
kernel launch of test_mem.py:7-35, here the HIP kernel through its
reference-signature launcher) and ``benchmark_speed(num_nodes, avg_degree,
provider)`` returning ``(ms, min_ms, max_ms)`` at quantiles 0.5 / 0.2 / 0.8
(test_speedup.py:7-47), swept over the same node counts with
``benchmark_speed.run(print_data=True, ...)``.  Providers: ``'pytorch'`` (the
eager per-edge torch computation) and ``'triton'`` / ``'hip'`` (the fused
kernel).  Timing uses HIP events, not Triton.

Run: ``python -m pymolecular_amd.benchmarks.test_speedup``.
"""
from __future__ import annotations

import sys

import torch

from ..datasets_loaders import generate_graph_data
from ..models.EGNN import egnn_backward_kernel_node_parallel
from ._common import DEFAULT_KWARGS, do_bench, eager_backward

X_VALS = [1000, 5000, 10000, 20000, 40000, 80000]   # test_speedup.py:10
PROVIDERS = ['pytorch', 'triton']                    # test_speedup.py:12-13


def launch_triton(data_tuple, kwargs_dict):
    """test_mem.py:7-35: zeroed gradient buffers, one backward launch, return grad_h."""
    (h, coord, edge_feat, row_ptrs, col_indices, edge_ids,
     w1_msg, w2_msg_src, w_d, w_e, w_hl, w1_mov, w2_mov, packed_w1_msg,
     grad_out_msg, grad_out_mov) = data_tuple
    num_nodes = h.size(0)
    grad_h = torch.zeros_like(h)
    grad_coord = torch.zeros_like(coord)
    grad_w1_msg_ptr = torch.zeros_like(packed_w1_msg)
    grad_w2_msg_ptr = torch.zeros_like(w_hl)
    grad_w1_mov_ptr = torch.zeros_like(w1_mov)
    grad_w2_mov_ptr = torch.zeros_like(w2_mov)
    grid = (num_nodes,)
    egnn_backward_kernel_node_parallel[grid](
        h, coord, edge_feat, row_ptrs, col_indices, edge_ids, grad_out_msg, grad_out_mov,
        grad_h, grad_coord, grad_w1_msg_ptr, grad_w2_msg_ptr, grad_w1_mov_ptr, grad_w2_mov_ptr,
        packed_w1_msg, w_hl, w1_mov, w2_mov,
        h.stride(0), coord.stride(0), edge_feat.stride(0), grad_out_msg.stride(0), grad_out_mov.stride(0),
        num_nodes, **kwargs_dict)
    return grad_h


def _row_indices(data, num_nodes):
    return torch.repeat_interleave(torch.arange(num_nodes, device=data[0].device), data[3][1:] - data[3][:-1])


class _PerfReport:
    """The sweep object of triton.testing.perf_report: ``__call__`` runs one point, ``run`` the sweep."""

    def __init__(self, fn, x_vals, providers, avg_degree):
        self.fn, self.x_vals, self.providers, self.avg_degree = fn, list(x_vals), list(providers), avg_degree

    def __call__(self, num_nodes, avg_degree, provider):
        return self.fn(num_nodes, avg_degree, provider)

    def run(self, print_data=True, show_plots=False, save_path=None, x_vals=None):
        rows = []
        for n in (x_vals or self.x_vals):
            rows.append((n, [self.fn(n, self.avg_degree, p)[0] for p in self.providers]))
        if print_data:
            print("egnn-backward-performance (ms):")
            print(f"{'num_nodes':>10} " + " ".join(f"{p:>14}" for p in self.providers))
            for n, ms in rows:
                print(f"{n:>10} " + " ".join(f"{v:14.4f}" for v in ms))
        if show_plots or save_path:
            try:
                import matplotlib.pyplot as plt
            except ImportError:   # plotting is optional; the table above is the result
                return rows
            for k, p in enumerate(self.providers):
                plt.plot([n for n, _ in rows], [ms[k] for _, ms in rows], label=p)
            plt.xlabel('num_nodes')
            plt.ylabel('Execution Time (ms)')
            plt.legend()
            if save_path:
                plt.savefig(f"{save_path}/egnn-backward-performance.png")
            if show_plots:
                plt.show()
        return rows


def _benchmark_speed(num_nodes, avg_degree, provider):
    kwargs = dict(DEFAULT_KWARGS)
    data = generate_graph_data(num_nodes, avg_degree, kwargs['F_NODE'], kwargs['F_EDGE'],
                               kwargs['HIDDEN_FEATURES'], kwargs['OUT_FEATURES'], kwargs['HID_FEAT_MOV_MLP'])
    quantiles = [0.5, 0.2, 0.8]
    if provider == 'pytorch':
        rows = _row_indices(data, num_nodes)
        ms, min_ms, max_ms = do_bench(lambda: eager_backward(
            data[0], data[1], data[2], rows, data[4], data[6], data[7], data[11], data[12], data[9], data[8],
            data[10], data[14], data[15]), quantiles=quantiles)
    elif provider in ('triton', 'hip'):
        ms, min_ms, max_ms = do_bench(lambda: launch_triton(data, kwargs), quantiles=quantiles)
    else:
        raise ValueError(f"unknown provider {provider!r}")
    return ms, min_ms, max_ms


benchmark_speed = _PerfReport(_benchmark_speed, X_VALS, PROVIDERS, avg_degree=32)


if __name__ == "__main__":
    print("\n--- RUNNING SPEED BENCHMARK ---")
    benchmark_speed.run(print_data=True, show_plots=False, save_path=None)
    sys.exit(0)
