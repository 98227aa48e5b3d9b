"""The fused layer at the workloads' full sizes, checked against the oracle and through properties.

The float64 oracle finishes in seconds only on small graphs.  On the full graphs of the five
workloads (molecules-128 and -1024, proteins 64 x 512, slabs 256 x 80 at H = 256, the 2M-node
power-law graph) these tests check:
  * molecules-128 (E = 45,636, fp32, one layer): the whole graph, forward and backward, against
    the oracle at 1e-5;
  * forward row restriction: out_msg[i] and out_mov[i] depend only on the edges of row i, so the
    oracle on the subgraph of a few sampled rows (the heaviest row among them) gives those rows;
  * backward row restriction: with the incoming gradients zero outside the sampled rows, every
    weight gradient depends only on those rows' edges, and so do the gradients of h and x of the
    nodes they touch; the oracle's backward on the subgraph gives all of them, and every other
    node's gradient is exactly zero;
  * E(3) equivariance (rotation and translation of the coordinates);
  * exact linearity of the backward in the incoming gradients (scaling by 2 is exact) and
    bitwise determinism of the forward and the backward;
  * the schedule of the 2M-node power-law graph (per-edge rows, split rows, CSC, the rank tables of
    its ~580k 32-edge tiles) bit-exact against the numpy restatement.
Bounds: normwise 1e-5 (fp32), 2e-2 (bf16); the bf16 oracle runs in float64 on the bf16 inputs.
"""
import numpy as np
import pytest
import torch

from oracle import egnn_oracle as orc
from pymolecular_amd import graphs
from tests.cases import make_params

pytestmark = pytest.mark.gpu

BF, F32 = torch.bfloat16, torch.float32
TOL = {BF: 2e-2, F32: 1e-5}

# workload -> (H, equivariant); F = O = M = H, F_E from the workload's own edge inputs
SHAPE = {1: (128, True), 2: (128, True), 3: (128, True), 4: (256, True), 5: (128, False)}

_GRAPHS = {}


def _graph(k):
    # built once per session: the 2M-node power-law graph takes about 30 s of host work
    if k not in _GRAPHS:
        _GRAPHS[k] = graphs.make_workload(k)
    return _GRAPHS[k]


def _inputs(k, dtype, seed):
    g = _graph(k)
    H, eq = SHAPE[k]
    FE = 0 if g.edge_attr is None else g.edge_attr.shape[1]
    gen = torch.Generator(device="cuda").manual_seed(seed)
    h = torch.randn((g.N, H), generator=gen, device="cuda").to(dtype)
    ef = torch.from_numpy(g.edge_attr).cuda().to(dtype) if FE else None
    coord = torch.from_numpy(g.coord).cuda() if eq else None
    p = make_params(np.random.Generator(np.random.PCG64(seed)), H, FE, H, H, H, eq=eq)
    pd = {key: torch.from_numpy(v).cuda().to(dtype) for key, v in p.items()}
    rowptr = torch.from_numpy(g.rowptr).cuda()
    col = torch.from_numpy(g.col).cuda()
    print(f"[fullsize] workload {k} N={g.N} E={g.E} H={H} FE={FE} eq={eq} dtype={dtype}", flush=True)
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


def _sample_rows(g, k, n=47):
    """Rows checked by the row-restriction tests (ascending): n rows drawn without replacement
    (seeded), the 16 highest-degree rows, and the rows where the 32-edge tiling is hardest (where
    they exist): 16 drawn among the rows spread over three or more tiles, and up to 4 each of the
    rows whose first edge is the last of a tile and whose last edge is the first of a tile."""
    deg = np.diff(g.rowptr)
    r = np.random.Generator(np.random.PCG64(7 + k))
    first_t = g.rowptr[:-1] // 32
    last_t = (g.rowptr[1:] - 1) // 32
    straddle = np.flatnonzero((deg > 0) & (last_t - first_t >= 2))
    starts_late = np.flatnonzero((deg > 1) & (g.rowptr[:-1] % 32 == 31))
    ends_early = np.flatnonzero((deg > 1) & (g.rowptr[1:] % 32 == 1))
    pick = lambda a, m: r.choice(a, min(m, len(a)), replace=False) if len(a) else np.zeros(0, np.int64)  # noqa: E731
    parts = [r.choice(g.N, n, replace=False), np.argsort(deg, kind="stable")[-16:], pick(straddle, 16),
             pick(starts_late, 4), pick(ends_early, 4)]
    return np.unique(np.concatenate(parts).astype(np.int64))


def _subgraph(g, rows):
    """CSR of the edges of ``rows`` (ascending) over the nodes they touch, relabelled in ascending order.

    Returns (nodes, sub_rowptr, sub_col, eidx): ``nodes`` are the old ids of the new nodes, ``eidx``
    the old CSR positions of the subgraph's edges in its CSR order."""
    spans = [np.arange(g.rowptr[i], g.rowptr[i + 1], dtype=np.int64) for i in rows]
    eidx = np.concatenate(spans)
    nodes = np.unique(np.concatenate([rows, g.col[eidx]]))
    deg = np.zeros(len(nodes), np.int64)
    deg[np.searchsorted(nodes, rows)] = [len(s) for s in spans]
    sub_rowptr = np.concatenate([[0], np.cumsum(deg)])
    sub_col = np.searchsorted(nodes, g.col[eidx])
    return nodes, sub_rowptr, sub_col, eidx


def _oracle_inputs(h, coord, ef, p, nodes, eidx, dtype):
    """The subgraph's inputs in float64 (the device's bf16 values exactly, for bf16)."""
    nodes_t = torch.from_numpy(nodes).cuda()
    hs = h[nodes_t].double().cpu().numpy()
    cs = None if coord is None else coord[nodes_t].double().cpu().numpy()
    es = None if ef is None else ef[torch.from_numpy(eidx).cuda()].double().cpu().numpy()
    P = {key: (orc.round_bf16(v) if dtype == BF else v.astype(np.float64)) for key, v in p.items()}
    return nodes_t, hs, cs, es, P


ROW_CASES = [(2, BF, False), (2, F32, False), (3, BF, True), (4, BF, True), (5, BF, False)]


@pytest.mark.parametrize("k,dtype,mean", ROW_CASES)
def test_forward_row_restriction(k, dtype, mean, record_error):
    g, h, ef, coord, pd, p, rowptr, col = _inputs(k, dtype, seed=100 + k)
    eq = SHAPE[k][1]
    out_msg, out_mov = _fwd(h, coord, ef, rowptr, col, pd, eq, mean)
    torch.cuda.synchronize()
    rows = _sample_rows(g, k)
    nodes, sub_rowptr, sub_col, eidx = _subgraph(g, rows)
    _, hs, cs, es, P = _oracle_inputs(h, coord, ef, p, nodes, eidx, dtype)
    ref_msg, ref_mov = orc.fused_forward(hs, cs, es, sub_rowptr, sub_col, None, P, mean_agg=mean, equivariant=eq)
    rows_new = np.searchsorted(nodes, rows)
    rows_t = torch.from_numpy(rows).cuda()
    tol = TOL[dtype]
    print(f"[fullsize] rows {len(rows)}, subgraph E={len(eidx)} (max degree {np.diff(g.rowptr).max()})", flush=True)
    err = orc.normwise_rel_err(out_msg[rows_t].double().cpu().numpy(), ref_msg[rows_new])
    record_error("out_msg", err, tol)
    assert err <= tol, err
    if eq:
        err = orc.normwise_rel_err(out_mov[rows_t].double().cpu().numpy(), ref_mov[rows_new])
        record_error("out_mov", err, tol)
        assert err <= tol, err


@pytest.mark.parametrize("k,dtype,mean", ROW_CASES)
def test_backward_row_restriction(k, dtype, mean, record_error):
    g, h, ef, coord, pd, p, rowptr, col = _inputs(k, dtype, seed=400 + k)
    H, eq = SHAPE[k]
    rows = _sample_rows(g, k)
    rows_t = torch.from_numpy(rows).cuda()
    gen = torch.Generator(device="cuda").manual_seed(9 + k)
    gm = torch.zeros((g.N, H), dtype=dtype, device="cuda")
    gm[rows_t] = torch.randn((len(rows), H), generator=gen, device="cuda").to(dtype)
    gx = None
    if eq:
        gx = torch.zeros((g.N, 3), dtype=torch.float32, device="cuda")
        gx[rows_t] = torch.randn((len(rows), 3), generator=gen, device="cuda")
    grads = _bwd(h, coord, ef, rowptr, col, pd, gm, gx, eq, mean)
    torch.cuda.synchronize()
    nodes, sub_rowptr, sub_col, eidx = _subgraph(g, rows)
    nodes_t, hs, cs, es, P = _oracle_inputs(h, coord, ef, p, nodes, eidx, dtype)
    sub_gm = gm[nodes_t].double().cpu().numpy()
    sub_gx = None if gx is None else gx[nodes_t].double().cpu().numpy()
    ref = orc.fused_backward(hs, cs, es, sub_rowptr, sub_col, None, P, sub_gm, sub_gx, mean_agg=mean,
                             equivariant=eq)
    tol = TOL[dtype]
    print(f"[fullsize] backward: rows {len(rows)}, subgraph N={len(nodes)} E={len(eidx)}", flush=True)
    keys = ["w1_msg", "w2_msg", "b1", "b2"] + (["w1_mov", "w2_mov", "bx1"] if eq else [])
    for key in keys:
        err = orc.normwise_rel_err(grads[key].double().cpu().numpy().reshape(ref[key].shape), ref[key])
        record_error("d" + key, err, tol)
        assert err <= tol, (key, err)
    outside = torch.ones(g.N, dtype=torch.bool, device="cuda")
    outside[nodes_t] = False
    for key in ["h"] + (["coord"] if eq else []):
        err = orc.normwise_rel_err(grads[key][nodes_t].double().cpu().numpy(), ref[key])
        record_error("d" + key, err, tol)
        assert err <= tol, (key, err)
        nz = int(torch.count_nonzero(grads[key][outside]))
        assert nz == 0, f"d{key}: {nz} nonzero entries on nodes outside the sampled rows' edges"


@pytest.mark.parametrize("mean", [False, True])
def test_molecules128_whole_graph_fp32(mean, record_error):
    # the one-layer fp32 workload is small enough for the oracle to run whole
    g, h, ef, coord, pd, p, rowptr, col = _inputs(1, F32, seed=500 + int(mean))
    gen = torch.Generator(device="cuda").manual_seed(11)
    gm = torch.randn((g.N, 128), generator=gen, device="cuda")
    gx = torch.randn((g.N, 3), generator=gen, device="cuda")
    out_msg, out_mov = _fwd(h, coord, ef, rowptr, col, pd, True, mean)
    grads = _bwd(h, coord, ef, rowptr, col, pd, gm, gx, True, mean)
    torch.cuda.synchronize()
    P = {key: v.astype(np.float64) for key, v in p.items()}
    hn, cn = h.double().cpu().numpy(), coord.double().cpu().numpy()
    ref_msg, ref_mov = orc.fused_forward(hn, cn, None, g.rowptr, g.col, None, P, mean_agg=mean)
    ref = orc.fused_backward(hn, cn, None, g.rowptr, g.col, None, P, gm.double().cpu().numpy(),
                             gx.double().cpu().numpy(), mean_agg=mean)
    errs = {"out_msg": orc.normwise_rel_err(out_msg.double().cpu().numpy(), ref_msg),
            "out_mov": orc.normwise_rel_err(out_mov.double().cpu().numpy(), ref_mov)}
    for key in ("h", "coord", "w1_msg", "w2_msg", "w1_mov", "w2_mov", "b1", "b2", "bx1"):
        errs["d" + key] = orc.normwise_rel_err(grads[key].double().cpu().numpy().reshape(ref[key].shape), ref[key])
    for key, err in errs.items():
        record_error(key, err, 1e-5)
    bad = {key: v for key, v in errs.items() if not v <= 1e-5}
    assert not bad, bad


@pytest.mark.parametrize("k,mean", [(2, False), (3, True), (4, True)])
def test_equivariance(k, mean, record_error):
    g, h, ef, coord, pd, p, rowptr, col = _inputs(k, BF, seed=200 + k)
    q, _ = np.linalg.qr(np.random.Generator(np.random.PCG64(k)).standard_normal((3, 3)))
    R = torch.from_numpy(q.astype(np.float32)).cuda()
    t = torch.tensor([3.0, -1.5, 0.25], device="cuda")
    m0, x0 = _fwd(h, coord, ef, rowptr, col, pd, True, mean)
    m1, x1 = _fwd(h, (coord @ R.T + t).contiguous(), ef, rowptr, col, pd, True, mean)
    torch.cuda.synchronize()
    e_msg = orc.normwise_rel_err(m1.float().cpu().numpy(), m0.float().cpu().numpy())
    e_mov = orc.normwise_rel_err(x1.cpu().numpy(), (x0 @ R.T).cpu().numpy())
    record_error("out_msg", e_msg, 2e-2)
    record_error("out_mov", e_mov, 2e-2)
    assert e_msg <= 2e-2 and e_mov <= 2e-2, (e_msg, e_mov)


@pytest.mark.parametrize("k", [2, 4, 5])
def test_backward_exact_linearity_and_determinism(k):
    g, h, ef, coord, pd, p, rowptr, col = _inputs(k, BF, seed=300 + k)
    H, eq = SHAPE[k]
    gen = torch.Generator(device="cuda").manual_seed(5)
    gm = torch.randn((g.N, H), generator=gen, device="cuda").to(BF)
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


def test_powerlaw_schedule_bit_exact():
    # the degree-binning schedule at the size that needs it: 2M rows of degree 2..4096, ~18.6M edges
    from pymolecular_amd import fused
    from tests.test_schedule import schedule_ref
    g = _graph(5)
    print(f"[fullsize] schedule N={g.N} E={g.E} max degree {np.diff(g.rowptr).max()}", flush=True)
    rp = torch.from_numpy(g.rowptr).cuda()
    cl = torch.from_numpy(g.col).cuda()
    got = fused.schedule_arrays(fused.get_schedule(rp, cl, g.N))
    ref = schedule_ref(g.rowptr, g.col)
    for key, v in ref.items():
        np.testing.assert_array_equal(got[key].cpu().numpy(), v, err_msg=key)
