"""Modules called on one graph, then on a different graph with the same edge count.

The second graph's edge tensors are allocated after the first's are freed, so the
device allocator hands them the same memory (same data pointer, version 0).
Each module must compute on the second graph, as the reference's modules do by
rebuilding from ``edge_index`` on every call (egnn_clean.py:95-101, layer.py:41-63).
Checked against the float64 CPU restatement (oracle/torch_ref.py, oracle/egnn_oracle.py).
"""
import gc

import numpy as np
import pytest
import torch

from oracle import egnn_oracle as orc
from oracle import torch_ref
from pymolecular_amd import graphs

pytestmark = pytest.mark.gpu

N, E = 300, 3000


def _edges(seed):
    r = np.random.Generator(np.random.PCG64(seed))
    dst = r.integers(0, N, E)
    src = (dst + r.integers(1, N, E)) % N     # no self loops
    return dst.astype(np.int64), src.astype(np.int64)


def _rel(a, b):
    return orc.normwise_rel_err(a.detach().double().cpu().numpy(), b.detach().double().cpu().numpy())


def _copy_weights(dst, src, rename=lambda n: n):
    pm = dict(dst.named_parameters())
    with torch.no_grad():
        for n, p in src.named_parameters():
            pm[rename(n)].copy_(p.to(pm[rename(n)].dtype))


def _device_pair(rows, cols):
    """Fresh device tensors holding one graph (allocated, then filled)."""
    a = torch.empty(E, dtype=torch.int64, device="cuda")
    b = torch.empty(E, dtype=torch.int64, device="cuda")
    a.copy_(torch.from_numpy(rows))
    b.copy_(torch.from_numpy(cols))
    return a, b


def _two_graphs(call):
    """call(rows, cols, dev_pair) on graph 1, free it, then on graph 2; returns graph 2's result
    and whether graph 2's edge tensors reused graph 1's memory."""
    r1, c1 = _edges(11)
    d1 = _device_pair(r1, c1)
    call(r1, c1, d1)
    torch.cuda.synchronize()
    p1 = tuple(t.data_ptr() for t in d1)
    del d1
    gc.collect()
    r2, c2 = _edges(12)
    d2 = _device_pair(r2, c2)
    reused = tuple(t.data_ptr() for t in d2) == p1
    out = call(r2, c2, d2)
    print(f"second graph's edge tensors at the first graph's addresses: {reused}", flush=True)
    return out, r2, c2


def test_egcl_second_graph():
    from pymolecular_amd.models.EGNN import E_GCL
    torch.manual_seed(4)
    H = 128
    ref = torch_ref.EGCLRef(H, H, H).double()
    torch.nn.init.xavier_uniform_(ref.coord_mlp[2].weight, gain=1.0)
    mod = E_GCL(H, H, H).cuda()
    _copy_weights(mod, ref)
    r = np.random.Generator(np.random.PCG64(5))
    h = torch.from_numpy(r.standard_normal((N, H)))
    x = torch.from_numpy(r.standard_normal((N, 3)))

    def call(rows, cols, dev):
        for p in mod.parameters():
            p.grad = None
        hd = h.float().cuda().requires_grad_()
        xd = x.float().cuda().requires_grad_()
        ho, xo, _ = mod(hd, dev, xd)
        (ho.sum() + xo.sum()).backward()
        return ho, xo, hd.grad, xd.grad, {n: p.grad.clone() for n, p in mod.named_parameters()}

    (ho, xo, gh, gx, gw), r2, c2 = _two_graphs(call)
    hr = h.clone().requires_grad_()
    xr = x.clone().requires_grad_()
    hor, xor_, _ = ref(hr, (torch.from_numpy(r2), torch.from_numpy(c2)), xr)
    (hor.sum() + xor_.sum()).backward()
    errs = {"h_out": _rel(ho, hor), "x_out": _rel(xo, xor_), "dh": _rel(gh, hr.grad), "dx": _rel(gx, xr.grad)}
    errs.update({"d" + n: _rel(gw[n], q.grad) for n, q in ref.named_parameters()})
    print({k: f"{v:.1e}" for k, v in errs.items()})
    assert all(v <= 1e-5 for v in errs.values()), errs


def test_egnn_stack_second_graph():
    from pymolecular_amd.models.EGNN import EGNN
    torch.manual_seed(5)
    H = 128
    ref = torch_ref.EGNNRef(5, H, 8, 0, n_layers=2).double()
    mod = EGNN(5, H, 8, 0, n_layers=2).cuda()
    _copy_weights(mod, ref, lambda n: n.replace("layers.", "gcl_"))
    r = np.random.Generator(np.random.PCG64(6))
    h = torch.from_numpy(r.standard_normal((N, 5)))
    x = torch.from_numpy(r.standard_normal((N, 3)))

    def call(rows, cols, dev):
        with torch.no_grad():
            return mod(h.float().cuda(), x.float().cuda(), list(dev), None)

    (ho, xo), r2, c2 = _two_graphs(call)
    with torch.no_grad():
        hor, xor_ = ref(h, x, [torch.from_numpy(r2), torch.from_numpy(c2)])
    e = {"h_out": _rel(ho, hor), "x_out": _rel(xo, xor_)}
    print({k: f"{v:.1e}" for k, v in e.items()})
    assert all(v <= 1e-5 for v in e.values()), e


def test_mpnn_stack_second_graph():
    from pymolecular_amd.models.EGNN import MPNN
    torch.manual_seed(6)
    H, FE = 128, 8
    ref = torch_ref.MPNNRef(16, H, 8, FE, n_layers=2).double()
    mod = MPNN(16, H, 8, FE, n_layers=2).cuda()
    _copy_weights(mod, ref, lambda n: n.replace("layers.", "gcl_"))
    r = np.random.Generator(np.random.PCG64(7))
    h = torch.from_numpy(r.standard_normal((N, 16)))
    ea = torch.from_numpy(r.standard_normal((E, FE)))

    def call(rows, cols, dev):
        with torch.no_grad():
            return mod(h.float().cuda(), list(dev), ea.float().cuda())

    ho, r2, c2 = _two_graphs(call)
    with torch.no_grad():
        hor = ref(h, [torch.from_numpy(r2), torch.from_numpy(c2)], ea)
    e = _rel(ho, hor)
    print(f"h_out {e:.1e}")
    assert e <= 1e-5


def test_egnn_triton_layer_second_graph():
    from pymolecular_amd.models.EGNN import EGNN_Triton_Layer
    torch.manual_seed(7)
    F, FE = 32, 16
    layer = EGNN_Triton_Layer(F, FE, 64, 32, 32, 48).cuda()
    r = np.random.Generator(np.random.PCG64(8))
    h = r.standard_normal((N, F)).astype(np.float32)
    x = r.standard_normal((N, 4)).astype(np.float32)
    ef = r.standard_normal((E, FE)).astype(np.float32)

    def call(rows, cols, dev):
        # (2, E) = (src, dst) as the reference layer reads it (layer.py:51-52); a new tensor per call,
        # freed when the call returns, so the second graph's lands at the first's address as well
        ei = torch.stack([dev[1], dev[0]])
        with torch.no_grad():
            return layer(torch.from_numpy(h).cuda(), torch.from_numpy(x).cuda(), ei, torch.from_numpy(ef).cuda())

    (hn, xn), dst, src = _two_graphs(call)
    rows = np.concatenate([dst, src])
    cols = np.concatenate([src, dst])
    eids = np.concatenate([np.arange(E), np.arange(E)])
    rowptr, col, perm = graphs.csr_from_rows(rows, cols, N)
    P = {k: getattr(layer, k).detach().cpu().numpy().astype(np.float64) for k in ["w1_msg", "w2_msg", "w1_mov"]}
    P["w2_mov"] = layer.w2_mov.detach().cpu().numpy().reshape(-1)
    om, ox = orc.fused_forward(h, x, ef, rowptr, col, eids[perm], P)
    deg = np.maximum(np.bincount(rows, minlength=N), 1)
    x_ref = x.astype(np.float64).copy()
    x_ref[:, :3] += ox / deg[:, None]
    with torch.no_grad():
        mlp = layer.node_mlp.double().cpu()
        h_ref = h + mlp(torch.cat([torch.from_numpy(h).double(), torch.from_numpy(om)], dim=1)).numpy()
    e_h = orc.normwise_rel_err(hn.cpu().numpy(), h_ref)
    e_x = orc.normwise_rel_err(xn.cpu().numpy(), x_ref)
    print(f"h {e_h:.1e} x {e_x:.1e}")
    assert e_h <= 1e-5 and e_x <= 1e-5
