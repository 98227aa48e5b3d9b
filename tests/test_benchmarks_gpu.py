"""The benchmark drivers (test_speedup.py / test_mem.py counterparts) run and agree.

The eager provider and the fused kernel are compared on the driver's own
inputs (fp32, rel <= 1e-5), then each sweep runs at small sizes.
"""
import pytest
import torch

from oracle import egnn_oracle as orc

pytestmark = pytest.mark.gpu


def test_launch_triton_matches_eager_provider():
    from pymolecular_amd.benchmarks._common import DEFAULT_KWARGS, eager_backward
    from pymolecular_amd.benchmarks.test_speedup import _row_indices, launch_triton
    from pymolecular_amd.datasets_loaders import generate_graph_data
    k = DEFAULT_KWARGS
    data = generate_graph_data(700, 32, k['F_NODE'], k['F_EDGE'], k['HIDDEN_FEATURES'], k['OUT_FEATURES'],
                               k['HID_FEAT_MOV_MLP'])
    gh = launch_triton(data, k)
    gh_ref, _ = eager_backward(data[0], data[1], data[2], _row_indices(data, 700), data[4], data[6], data[7],
                               data[11], data[12], data[9], data[8], data[10], data[14], data[15])
    err = orc.normwise_rel_err(gh.double().cpu().numpy(), gh_ref.double().cpu().numpy())
    print(f"dh rel {err:.1e}")
    assert err <= 1e-5


def test_speed_sweep_small():
    from pymolecular_amd.benchmarks.test_speedup import benchmark_speed
    rows = benchmark_speed.run(print_data=True, x_vals=[1000, 5000])
    assert len(rows) == 2 and all(ms > 0 for _, v in rows for ms in v)


def test_memory_sweep_small():
    # peak device memory of one backward call, inputs included: the fused fp32 layer keeps its per-edge
    # state one edge chunk at a time, the eager provider every per-edge activation and its autograd saves;
    # at the reference sweep's sizes the fused peak is below the eager one, and at most half of it from
    # 25k nodes (test_mem.py:42)
    from pymolecular_amd.benchmarks.test_mem import run_memory_benchmark
    rows = run_memory_benchmark([1000, 25000])
    for n, e, pt, hip in rows:
        assert hip != "OOM" and float(hip) > 0
        assert pt == "OOM" or float(hip) <= float(pt), (n, hip, pt)
        if n == 25000:
            assert pt == "OOM" or float(hip) <= 0.5 * float(pt), (hip, pt)
