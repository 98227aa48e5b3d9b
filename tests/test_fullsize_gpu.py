"""The fused layer at the workloads' full sizes, checked through properties that hold at any size.

The float64 oracle finishes in seconds only on small graphs, so on the full graphs of the
benchmark workloads (molecules-1024, proteins 64 x 512, the 2M-node power-law graph) these
tests check, in bf16:
  * row restriction: out_msg[i] and out_mov[i] depend only on the edges of row i, so the
    oracle run on the subgraph of a few sampled rows (the heaviest row among them) gives
    those rows (normwise 2e-2);
  * E(3) equivariance: rotating and translating the coordinates leaves out_msg unchanged and
    rotates out_mov;
  * exact linearity of the backward in the incoming gradients: doubling them doubles every
    gradient bit for bit (scaling by 2 is exact in bf16 and fp32);
  * bitwise determinism of the forward and the backward.
"""
import numpy as np
import pytest
import torch

from oracle import egnn_oracle as orc
from pymolecular_amd import graphs
from tests.cases import make_params

pytestmark = pytest.mark.gpu

BF = torch.bfloat16


_GRAPHS = {}


def _graph(k):
    # built once per session: the 2M-node power-law graph takes about 30 s of host work
    if k not in _GRAPHS:
        _GRAPHS[k] = graphs.make_workload(k)
    return _GRAPHS[k]


def _inputs(k, FE, eq, seed):
    g = _graph(k)
    N, E = g.N, g.E
    gen = torch.Generator(device="cuda").manual_seed(seed)
    h = torch.randn((N, 128), generator=gen, device="cuda").to(BF)
    ef = torch.randn((E, FE), generator=gen, device="cuda").to(BF) if FE else None
    coord = torch.from_numpy(g.coord).cuda() if eq else None
    p = make_params(np.random.Generator(np.random.PCG64(seed)), 128, FE, 128, 128, 128, eq=eq)
    pd = {key: torch.from_numpy(v).cuda().to(BF) for key, v in p.items()}
    rowptr = torch.from_numpy(g.rowptr).cuda()
    col = torch.from_numpy(g.col).cuda()
    print(f"[fullsize] workload {k} N={N} E={E} FE={FE} eq={eq}", flush=True)
    return g, h, ef, coord, pd, p, rowptr, col


def _fwd(h, coord, ef, rowptr, col, pd, eq, mean):
    from pymolecular_amd import fused
    return fused.egnn_fused_forward(h, coord, ef, rowptr, col, None, pd["w1_msg"], pd["w2_msg"], pd.get("w1_mov"),
                                    pd.get("w2_mov"), pd.get("b1"), pd.get("b2"), pd.get("bx1"), mean_agg=mean,
                                    equivariant=eq)


def _bwd(h, coord, ef, rowptr, col, pd, gm, gx, eq, mean):
    from pymolecular_amd import fused
    return fused.egnn_fused_backward(h, coord, ef, rowptr, col, None, pd["w1_msg"], pd["w2_msg"], pd.get("w1_mov"),
                                     pd.get("w2_mov"), pd.get("b1"), pd.get("b2"), pd.get("bx1"), gm, gx,
                                     mean_agg=mean, equivariant=eq)


@pytest.mark.parametrize("k,FE,eq,mean", [(2, 0, True, False), (3, 16, True, True), (5, 16, False, False)])
def test_row_restriction_against_oracle(k, FE, eq, mean):
    g, h, ef, coord, pd, p, rowptr, col = _inputs(k, FE, eq, seed=100 + k)
    out_msg, out_mov = _fwd(h, coord, ef, rowptr, col, pd, eq, mean)
    torch.cuda.synchronize()
    deg = np.diff(g.rowptr)
    r = np.random.Generator(np.random.PCG64(7 + k))
    rows = np.unique(np.concatenate([[int(np.argmax(deg))], r.choice(g.N, 47, replace=False)]))
    # the subgraph of the sampled rows, nodes relabelled: the rows first, then their other sources
    spans = [np.arange(g.rowptr[i], g.rowptr[i + 1]) for i in rows]
    eidx = np.concatenate(spans)
    nodes = np.unique(np.concatenate([rows, g.col[eidx]]))
    new = {int(v): q for q, v in enumerate(nodes)}
    order = np.argsort([new[int(i)] for i in rows], kind="stable")
    sub_rowptr = np.zeros(len(nodes) + 1, np.int64)
    for i, s in zip(rows, spans):
        sub_rowptr[new[int(i)] + 1] = len(s)
    sub_rowptr = np.cumsum(sub_rowptr)
    sub_col = np.concatenate([np.array([new[int(v)] for v in g.col[spans[q]]], np.int64) for q in order])
    sub_eidx = np.concatenate([spans[q] for q in order])
    nodes_t = torch.from_numpy(nodes).cuda()
    hs = h[nodes_t].float().cpu().numpy()
    cs = None if coord is None else coord[nodes_t].cpu().numpy()
    es = None if ef is None else ef[torch.from_numpy(sub_eidx).cuda()].float().cpu().numpy()
    P = {key: orc.round_bf16(v) for key, v in p.items()}
    ref_msg, ref_mov = orc.fused_forward(hs, cs, es, sub_rowptr, sub_col, None, P, mean_agg=mean, equivariant=eq)
    rows_new = np.array([new[int(i)] for i in rows])
    got = out_msg[torch.from_numpy(rows).cuda()].float().cpu().numpy()
    err = orc.normwise_rel_err(got, ref_msg[rows_new])
    print(f"[fullsize] rows {len(rows)} (max degree {deg.max()}) out_msg err {err:.2e}", flush=True)
    assert err <= 2e-2, err
    if eq:
        gmv = out_mov[torch.from_numpy(rows).cuda()].cpu().numpy()
        err = orc.normwise_rel_err(gmv, ref_mov[rows_new])
        print(f"[fullsize] out_mov err {err:.2e}", flush=True)
        assert err <= 2e-2, err


@pytest.mark.parametrize("k,FE,mean", [(2, 0, False), (3, 16, True)])
def test_equivariance(k, FE, mean):
    g, h, ef, coord, pd, p, rowptr, col = _inputs(k, FE, True, seed=200 + k)
    q, _ = np.linalg.qr(np.random.Generator(np.random.PCG64(k)).standard_normal((3, 3)))
    R = torch.from_numpy(q.astype(np.float32)).cuda()
    t = torch.tensor([3.0, -1.5, 0.25], device="cuda")
    m0, x0 = _fwd(h, coord, ef, rowptr, col, pd, True, mean)
    m1, x1 = _fwd(h, (coord @ R.T + t).contiguous(), ef, rowptr, col, pd, True, mean)
    torch.cuda.synchronize()
    e_msg = orc.normwise_rel_err(m1.float().cpu().numpy(), m0.float().cpu().numpy())
    e_mov = orc.normwise_rel_err(x1.cpu().numpy(), (x0 @ R.T).cpu().numpy())
    print(f"[fullsize] equivariance out_msg {e_msg:.2e} out_mov {e_mov:.2e}", flush=True)
    assert e_msg <= 2e-2 and e_mov <= 2e-2, (e_msg, e_mov)


@pytest.mark.parametrize("k,FE,eq", [(2, 0, True), (5, 16, False)])
def test_backward_exact_linearity_and_determinism(k, FE, eq):
    g, h, ef, coord, pd, p, rowptr, col = _inputs(k, FE, eq, seed=300 + k)
    gen = torch.Generator(device="cuda").manual_seed(5)
    gm = torch.randn((g.N, 128), generator=gen, device="cuda").to(BF)
    gx = torch.randn((g.N, 3), generator=gen, device="cuda") if eq else None
    f1 = _fwd(h, coord, ef, rowptr, col, pd, eq, False)
    f2 = _fwd(h, coord, ef, rowptr, col, pd, eq, False)
    a = _bwd(h, coord, ef, rowptr, col, pd, gm, gx, eq, False)
    b = _bwd(h, coord, ef, rowptr, col, pd, gm, gx, eq, False)
    c = _bwd(h, coord, ef, rowptr, col, pd, gm * 2, None if gx is None else gx * 2, eq, False)
    torch.cuda.synchronize()
    assert torch.equal(f1[0], f2[0]) and (not eq or torch.equal(f1[1], f2[1]))
    for key, v in a.items():
        if v is None:
            continue
        assert torch.equal(v, b[key]), key
        assert torch.equal(c[key], v * 2), key
