"""The allocation-free forward (egnn_fwd_static) against egnn_fwd, through the C-ABI.

Both entry points run the same kernels on the same inputs, so their outputs must agree
bit for bit.  Two calls in a row, the second on a smaller graph: the fixed scratch keeps
the first call's contents, and nothing in it may leak into the second call's results.
The call allocates nothing (torch's allocator and the device's free memory are unchanged
across it) and runs under HIP graph capture, replayed several times.
"""
import numpy as np
import pytest
import torch

from pymolecular_amd import _capi, fused, graphs
from pymolecular_amd._capi import EgnnStrides
from tests.cases import make_params

pytestmark = pytest.mark.gpu


def _layer(n_graphs, dtype, eq, FE, seed):
    g = graphs.molecule_batch(n_graphs, seed=seed, feat_seed=seed + 1)
    H = 128
    r = np.random.Generator(np.random.PCG64(seed))
    dev = torch.device("cuda:0")
    T = lambda a, dt=None: torch.from_numpy(np.ascontiguousarray(a)).to(dev, dt)  # noqa: E731
    p = make_params(r, H, FE, H, H, H, eq=eq)
    t = dict(h=T(r.standard_normal((g.N, H)).astype(np.float32), dtype),
             coord=T(g.coord) if eq else None,
             ef=T(r.standard_normal((g.E, FE)).astype(np.float32), dtype) if FE else None,
             rowptr=T(g.rowptr), col=T(g.col),
             **{k: T(v, dtype) for k, v in p.items()})
    return g, t


def _args(t, eq, mean):
    """(dims, strides, pointer arguments up to the schedule, out_msg, out_mov), outputs filled with NaN."""
    dims = fused._dims(t["h"], t["ef"], t["col"], t["w1_msg"], t["w2_msg"], t.get("w1_mov"), eq, mean)
    N = t["h"].shape[0]
    sched = fused.get_schedule(t["rowptr"], t["col"], N)
    out_msg = torch.full((N, dims.O), float("nan"), dtype=t["h"].dtype, device="cuda")
    out_mov = torch.full((N, 3), float("nan"), dtype=torch.float32, device="cuda") if eq else None
    strides = EgnnStrides(h=t["h"].stride(0), coord=3 if eq else 4,
                          edge=t["ef"].stride(0) if t["ef"] is not None else 0, msg=out_msg.stride(0), mov=3)
    P = fused._ptr
    args = [P(t["h"]), P(t["coord"]), P(t["ef"]), P(t["rowptr"]), P(t["col"]), None, P(t["w1_msg"]),
            P(t["w2_msg"]), P(t.get("w1_mov")), P(t.get("w2_mov")), P(t.get("b1")), P(t.get("b2")),
            P(t.get("bx1")), P(out_msg), P(out_mov), None, sched.buf.data_ptr()]
    return dims, strides, args, out_msg, out_mov


def _run(entry, t, eq, mean):
    L = _capi.lib()
    dims = fused._dims(t["h"], t["ef"], t["col"], t["w1_msg"], t["w2_msg"], t.get("w1_mov"), eq, mean)
    N = t["h"].shape[0]
    sched = fused.get_schedule(t["rowptr"], t["col"], N)
    out_msg = torch.full((N, dims.O), float("nan"), dtype=t["h"].dtype, device="cuda")
    out_mov = torch.full((N, 3), float("nan"), dtype=torch.float32, device="cuda") if eq else None
    strides = EgnnStrides(h=t["h"].stride(0), coord=3 if eq else 4,
                          edge=t["ef"].stride(0) if t["ef"] is not None else 0, msg=out_msg.stride(0), mov=3)
    P = fused._ptr
    args = [P(t["h"]), P(t["coord"]), P(t["ef"]), P(t["rowptr"]), P(t["col"]), None, P(t["w1_msg"]),
            P(t["w2_msg"]), P(t.get("w1_mov")), P(t.get("w2_mov")), P(t.get("b1")), P(t.get("b2")),
            P(t.get("bx1")), P(out_msg), P(out_mov), None, sched.buf.data_ptr()]
    stream = fused._stream(out_msg.device)
    if entry == "egnn_fwd":
        nbytes = L.egnn_fwd_workspace_bytes(dims)
        ws = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
        rc = L.egnn_fwd(dims, strides, *args, ws.data_ptr(), nbytes, stream)
    else:
        assert L.egnn_fwd_workspace_bytes(dims) <= _capi.FWD_STATIC_SCRATCH_BYTES
        rc = L.egnn_fwd_static(dims, strides, *args, stream)
    _capi.check(entry, rc)
    torch.cuda.synchronize()
    return out_msg, out_mov


@pytest.mark.parametrize("dtype,eq,FE,mean", [(torch.bfloat16, True, 0, True), (torch.bfloat16, False, 16, False),
                                             (torch.float32, True, 16, False)])
def test_static_forward_matches_egnn_fwd(dtype, eq, FE, mean):
    # the larger graph first, then a smaller one on the same scratch
    for n_graphs, seed in ((300, 61), (7, 62)):
        g, t = _layer(n_graphs, dtype, eq, FE, seed)
        print(f"[no_alloc] N={g.N} E={g.E} dtype={dtype} eq={eq} FE={FE} mean={mean}", flush=True)
        ref = _run("egnn_fwd", t, eq, mean)
        got = _run("egnn_fwd_static", t, eq, mean)
        assert torch.equal(got[0], ref[0]), "out_msg differs"
        assert not eq or torch.equal(got[1], ref[1]), "out_mov differs"
        assert torch.isfinite(got[0].float()).all()


def test_static_forward_allocates_nothing():
    L = _capi.lib()
    g, t = _layer(50, torch.bfloat16, True, 16, 64)
    ref = _run("egnn_fwd", t, True, False)
    dims, strides, args, out_msg, out_mov = _args(t, True, False)
    torch.cuda.synchronize()
    alloc0 = torch.cuda.memory_allocated()
    free0 = torch.cuda.mem_get_info()[0]
    _capi.check("egnn_fwd_static", L.egnn_fwd_static(dims, strides, *args, fused._stream(out_msg.device)))
    torch.cuda.synchronize()
    alloc1 = torch.cuda.memory_allocated()
    free1 = torch.cuda.mem_get_info()[0]
    print(f"[no_alloc] torch allocated {alloc0} -> {alloc1}; device free {free0} -> {free1}", flush=True)
    assert alloc1 == alloc0
    # the fixed array is resident from the library's code-object load on this GPU, not from this call
    assert free0 - free1 < _capi.FWD_STATIC_SCRATCH_BYTES
    assert torch.equal(out_msg, ref[0]) and torch.equal(out_mov, ref[1])


def test_static_forward_under_graph_capture():
    L = _capi.lib()
    g, t = _layer(40, torch.bfloat16, True, 16, 65)
    print(f"[no_alloc graph] N={g.N} E={g.E}", flush=True)
    ref = _run("egnn_fwd", t, True, True)
    _run("egnn_fwd_static", t, True, True)          # first call on the device outside the capture
    dims, strides, args, out_msg, out_mov = _args(t, True, True)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        rc = L.egnn_fwd_static(dims, strides, *args, fused._stream(out_msg.device))
    _capi.check("egnn_fwd_static (captured)", rc)
    for k in range(3):
        out_msg.fill_(float("nan"))                  # eager work between the replays
        out_mov.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out_msg, ref[0]), f"replay {k}: out_msg differs"
        assert torch.equal(out_mov, ref[1]), f"replay {k}: out_mov differs"
        other = _run("egnn_fwd", t, True, True)       # an eager call on its own workspace
        assert torch.equal(other[0], ref[0])
