"""GPU parity of the fused EGNN/MPNN layer (HIP kernels through the C-ABI) against the oracle.

Tolerance: normwise max|y - ref| / max|ref| <= 1e-5 (fp32), <= 2e-2 (bf16); the
bf16 oracle runs in float64 on bf16-rounded inputs and weights.
"""
import numpy as np
import pytest
import torch

from oracle import egnn_oracle as orc
from pymolecular_amd import graphs
from tests.cases import Case, random_csr

pytestmark = pytest.mark.gpu

TOL = {"fp32": 1e-5, "bf16": 2e-2}
DT = {"fp32": torch.float32, "bf16": torch.bfloat16}


def _dev(a, dt=None):
    if a is None:
        return None
    t = torch.from_numpy(np.ascontiguousarray(a)).cuda()
    return t.to(dt) if dt is not None else t


def run_fused(case, dtype, backward=True, linear=False):
    """``linear``: pass w1_msg, w2_msg, w1_mov transposed (torch.nn.Linear layout); their
    gradients are transposed back, so results compare with the packed-layout run."""
    from pymolecular_amd import fused
    dt = DT[dtype]
    rowptr, col = _dev(case.rowptr), _dev(case.col)
    eids = _dev(case.edge_ids)
    h = _dev(case.h, dt)
    coord = _dev(case.coord) if case.eq else None
    ef = _dev(case.ef, dt)
    p = {k: _dev(v, dt) for k, v in case.p.items()}
    mats = ("w1_msg", "w2_msg", "w1_mov")
    if linear:
        p = {k: (v.t().contiguous() if k in mats and v is not None else v) for k, v in p.items()}
    print(f"[fused] N={case.N} E={case.E} F={case.F} FE={case.FE} H={case.H} O={case.O} M={case.M} "
          f"eq={case.eq} mean={case.mean} dtype={dtype} linear={linear}", flush=True)
    out_msg, out_mov = fused.egnn_fused_forward(h, coord, ef, rowptr, col, eids, p["w1_msg"], p["w2_msg"],
                                                p.get("w1_mov"), p.get("w2_mov"), p.get("b1"), p.get("b2"),
                                                p.get("bx1"), mean_agg=case.mean, equivariant=case.eq,
                                                linear_weights=linear)
    res = dict(out_msg=out_msg.float().cpu().numpy(), out_mov=None if out_mov is None else out_mov.cpu().numpy())
    if backward:
        g = fused.egnn_fused_backward(h, coord, ef, rowptr, col, eids, p["w1_msg"], p["w2_msg"], p.get("w1_mov"),
                                      p.get("w2_mov"), p.get("b1"), p.get("b2"), p.get("bx1"), _dev(case.gm, dt),
                                      _dev(case.gx) if case.eq else None, mean_agg=case.mean, equivariant=case.eq,
                                      linear_weights=linear)
        if linear:
            g = {k: (v.t() if k in mats and v is not None else v) for k, v in g.items()}
        res["grads"] = {k: (None if v is None else v.float().cpu().numpy()) for k, v in g.items()}
    torch.cuda.synchronize()
    return res


def check_case(case, dtype, backward=True):
    bf = dtype == "bf16"
    tol = TOL[dtype]
    res = run_fused(case, dtype, backward)
    ref_msg, ref_mov = case.forward_ref(bf)
    errs = {"out_msg": orc.normwise_rel_err(res["out_msg"], ref_msg)}
    if case.eq:
        errs["out_mov"] = orc.normwise_rel_err(res["out_mov"], ref_mov)
    if backward:
        gref = case.backward_ref(bf)
        for k, v in gref.items():
            if v is None or res["grads"].get(k) is None:
                continue
            errs["d" + k] = orc.normwise_rel_err(res["grads"][k].reshape(v.shape), v)
    print("errors:", {k: f"{v:.2e}" for k, v in errs.items()}, flush=True)
    bad = {k: v for k, v in errs.items() if not (v <= tol)}
    assert not bad, f"{dtype} parity failed (tol {tol}): {bad}"
    return errs


def molecule_case(n_graphs, F, FE, H, O, M, seed, **kw):
    g = graphs.molecule_batch(n_graphs, seed=seed, feat_seed=seed + 1)
    return Case(g.rowptr, g.col, F, FE, H, O, M, seed=seed, **kw)


@pytest.mark.parametrize("dtype", ["fp32", "bf16"])
def test_molecules_h128(dtype):
    check_case(molecule_case(6, 128, 0, 128, 128, 128, seed=11), dtype)


@pytest.mark.parametrize("dtype", ["fp32", "bf16"])
def test_molecules_h128_mean_agg(dtype):
    check_case(molecule_case(5, 128, 0, 128, 128, 128, seed=12, mean_agg=True), dtype)


@pytest.mark.parametrize("dtype", ["fp32", "bf16"])
def test_reference_sweep_dims(dtype):
    # F_NODE 32, F_EDGE 16, HIDDEN 64, OUT 32, HID_MOV 32 (test_mem.py:46-50)
    rowptr, col = random_csr(300, np.full(300, 32), seed=5)
    check_case(Case(rowptr, col, 32, 16, 64, 32, 32, seed=13, bias=False), dtype)


@pytest.mark.parametrize("dtype", ["fp32", "bf16"])
def test_skewed_rows_and_empty_rows(dtype):
    # rows crossing many 32-edge tiles, empty rows, and a final partial tile
    degs = np.array([0, 1, 100, 0, 3, 31, 32, 33, 0, 64, 2, 200, 5, 0, 17] * 4)
    rowptr, col = random_csr(len(degs), degs, seed=7)
    check_case(Case(rowptr, col, 128, 16, 128, 128, 128, seed=14), dtype)


@pytest.mark.parametrize("dtype", ["fp32", "bf16"])
def test_edge_ids_permutation(dtype):
    rowptr, col = random_csr(120, np.arange(120) % 40, seed=9)
    E = len(col)
    perm = np.random.Generator(np.random.PCG64(3)).permutation(E)
    check_case(Case(rowptr, col, 128, 32, 128, 128, 128, seed=15, edge_ids=perm), dtype)


@pytest.mark.parametrize("dtype", ["fp32", "bf16"])
def test_mpnn_variant(dtype):
    rowptr, col = random_csr(400, (np.arange(400) * 7) % 23 + 2, seed=21)
    check_case(Case(rowptr, col, 128, 16, 128, 128, 128, seed=16, eq=False), dtype)


@pytest.mark.parametrize("fe,skewed,eids", [(0, True, False), (8, False, True), (16, True, True), (24, True, False),
                                            (32, False, False)])
def test_mpnn_edge_parallel_cases(fe, skewed, eids):
    """The edge-parallel MPNN kernels (bf16, H = 128): every edge-feature width they instantiate (none, one and
    two 16-slot blocks of the dW_e product), rows across many 128-edge block tiles and 32-edge rank tables,
    empty rows, a partial last block tile, and edge ids that permute the feature rows."""
    if skewed:
        degs = np.array([0, 300, 1, 2, 0, 129, 3, 31, 33, 0, 64, 127, 128, 5, 2, 2, 2, 0, 17] * 6)
    else:
        degs = (np.arange(517) * 11) % 37
    rowptr, col = random_csr(len(degs), degs, seed=61 + fe)
    perm = np.random.Generator(np.random.PCG64(5)).permutation(len(col)) if eids else None
    print(f"[mpnn-ep] N={len(degs)} E={len(col)} fe={fe} skewed={skewed} eids={eids}", flush=True)
    check_case(Case(rowptr, col, 128, fe, 128, 128, 128, seed=22 + fe, eq=False, edge_ids=perm), "bf16")


@pytest.mark.parametrize("fe,ndeg", [(16, 14000), (0, 60000)])
def test_mpnn_forward_tile_ranges(fe, ndeg):
    """The edge-parallel MPNN forward gives each wave one contiguous range of 32-edge tiles: a row split over
    tiles of one range is summed by its wave, the pieces of a row that crosses range boundaries are summed
    by the fix-up.  With ~4,000 waves the 14,000-row graph has one tile per range, so every split row
    crosses range boundaries (the degree-3,000 row ~95 of them), and the 60,000-row graph three to four
    tiles per range, so rows also close inside their wave's range; next to short rows, empty rows and a
    partial last tile.  Every row is checked against the oracle, and the whole output at the usual
    tolerance."""
    r = np.random.Generator(np.random.PCG64(401 + fe))
    degs = r.integers(0, 20, size=ndeg)
    degs[r.choice(ndeg, 8, replace=False)] = [3000, 1000, 700, 300, 129, 65, 64, 33]
    degs[r.choice(ndeg, ndeg // 10, replace=False)] = 0
    rowptr, col = random_csr(len(degs), degs, seed=403 + fe)
    assert len(col) % 32 != 0
    case = Case(rowptr, col, 128, fe, 128, 128, 128, seed=405 + fe, eq=False)
    from pymolecular_amd import _capi
    ntt = (case.E + 31) // 32
    waves = 8 * max(1, min((case.E + 255) // 256, 512))
    print(f"[mpnn-ranges] N={case.N} E={case.E} tiles={ntt} waves={waves} tiles/range={ntt / waves:.2f}", flush=True)
    res = run_fused(case, "bf16", backward=False)
    ref_msg, _ = case.forward_ref(True)
    err = orc.normwise_rel_err(res["out_msg"], ref_msg)
    deg = np.diff(case.rowptr)
    num = np.abs(res["out_msg"] - ref_msg).max(axis=1)
    den = np.abs(ref_msg).max(axis=1)
    row_err = np.where(deg > 0, num / np.maximum(den, 1e-30), num)
    worst = int(np.argmax(row_err))
    print(f"[mpnn-ranges] out_msg err {err:.2e}, worst row {worst} (degree {deg[worst]}) {row_err[worst]:.2e}, "
          f"empty rows max |out| {np.abs(res['out_msg'][deg == 0]).max():.1e}", flush=True)
    assert err <= TOL["bf16"]
    assert row_err.max() <= 3e-2, (worst, deg[worst], row_err[worst])
    assert not np.any(res["out_msg"][deg == 0])


@pytest.mark.parametrize("mean", [False, True])
def test_egnn_h128_edge_features_24(mean):
    """The bf16 EGNN kernels at H = 128 (edge-parallel forward, cooperative backward) at F_E = 24: the forward's
    edge-input chunk of 24 features plus r^2 in the fourth 8-slot group, and the backward's second 16-slot dW_e
    block, which also holds the r^2 slots.  Skewed rows that cross many 32- and 64-edge tiles, empty rows, a
    partial last 64-edge tile (E % 64 != 0) and edge ids that permute the feature rows."""
    degs = np.array([0, 300, 1, 2, 0, 129, 3, 31, 33, 0, 64, 127, 128, 5, 2, 2, 2, 0, 17] * 5 + [7])
    rowptr, col = random_csr(len(degs), degs, seed=81)
    assert len(col) % 64 != 0
    perm = np.random.Generator(np.random.PCG64(9)).permutation(len(col))
    print(f"[egnn-fe24] N={len(degs)} E={len(col)} mean={mean}", flush=True)
    check_case(Case(rowptr, col, 128, 24, 128, 128, 128, seed=83, eq=True, mean_agg=mean, edge_ids=perm), "bf16")


@pytest.mark.parametrize("dtype", ["bf16", "fp32"])
@pytest.mark.parametrize("mean", [False, True])
def test_egnn_graph_smaller_than_a_tile(dtype, mean):
    """Seven edges: one partial 32-edge tile, so one wave of the edge-parallel forward works and most of its
    lanes hold edges past E (clamped loads, phi set to zero, outside every rank's span); empty rows too."""
    rowptr, col = random_csr(6, np.array([0, 3, 1, 0, 3, 0]), seed=95)
    assert len(col) == 7
    check_case(Case(rowptr, col, 128, 16, 128, 128, 128, seed=96, eq=True, mean_agg=mean), dtype)


def test_egnn_forward_many_tiles_per_wave():
    """The edge-parallel EGNN forward (bf16, H = 128) with more 32-edge tiles than the 2048 waves it runs, so
    each wave walks several tiles with the next tile's gathers and records in flight: skewed rows across
    tiles, empty rows, edge ids permuting the F_E = 16 features, mean aggregation, and the coordinate
    residual added to every row (whole rows stored by the kernel, split rows by the fix-up)."""
    from pymolecular_amd import fused
    r = np.random.Generator(np.random.PCG64(91))
    degs = r.integers(0, 48, 7000)
    degs[::97] = 300
    degs[::13] = 0
    rowptr_np, col_np = random_csr(len(degs), degs, seed=92)
    E = len(col_np)
    assert (E + 31) // 32 > 2 * 2048 and E % 32 != 0
    perm = r.permutation(E)
    case = Case(rowptr_np, col_np, 128, 16, 128, 128, 128, seed=93, eq=True, mean_agg=True, edge_ids=perm)
    print(f"[egnn-fwd-tiles] N={case.N} E={E} tiles={(E + 31) // 32}", flush=True)
    check_case(case, "bf16", backward=False)
    dt = torch.bfloat16
    h, coord, ef = _dev(case.h, dt), _dev(case.coord), _dev(case.ef, dt)
    p = {k: _dev(v, dt) for k, v in case.p.items()}
    fa = (h, coord, ef, _dev(case.rowptr), _dev(case.col), _dev(case.edge_ids), p["w1_msg"], p["w2_msg"],
          p["w1_mov"], p["w2_mov"], p.get("b1"), p.get("b2"), p.get("bx1"))
    kw = dict(mean_agg=True, equivariant=True)
    msg0, mov0 = fused.egnn_fused_forward(*fa, **kw)
    msg1, mov1 = fused.egnn_fused_forward(*fa, **kw, coord_residual=True)
    torch.cuda.synchronize()
    assert torch.equal(msg0, msg1)
    assert torch.equal(mov1, coord + mov0)   # one fp32 add of the same operands


@pytest.mark.parametrize("dims,eq,mean", [((32, 16, 64, 32, 32), True, False), ((128, 16, 128, 128, 128), True, True),
                                           ((128, 24, 128, 128, 128), False, False)])
def test_fp32_edge_chunks(dims, eq, mean):
    """The fp32 backward in edge chunks (more than 8,192 edges: at least two; Gh, Gx, r^2 and the factors
    held one chunk at a time, the node sums and weight gradients added in chunk order): rows that straddle
    the chunk boundaries, empty rows, a degree-1,500 row, edge ids that permute the feature rows."""
    from pymolecular_amd import _capi
    F, FE, H, O, M = dims
    degs = np.array([0, 1500, 3, 61, 0, 7, 33, 2, 90, 1, 31] * 60)
    rowptr, col = random_csr(len(degs), degs, seed=95)
    E = len(col)
    perm = np.random.Generator(np.random.PCG64(96)).permutation(E)
    d = _capi.EgnnDims(N=len(degs), E=E, F=F, FE=FE, H=H, O=O, M=M, equivariant=int(eq), mean_agg=int(mean), dtype=0)
    print(f"[fp32-chunks] N={len(degs)} E={E} dims={dims} eq={eq} mean={mean} "
          f"workspace {_capi.lib().egnn_bwd_workspace_bytes(d) / 2 ** 20:.1f} MB", flush=True)
    check_case(Case(rowptr, col, F, FE, H, O, M, seed=97, eq=eq, mean_agg=mean, edge_ids=perm), "fp32")


def test_mpnn_forward_wide_message_rows():
    """Message rows 2 MiB apart (an output of more than 2 GB in all): the MPNN forward leaves the edge-parallel
    kernel, whose stores use 32-bit offsets, for the cooperative kernel; both against the oracle."""
    from pymolecular_amd import fused
    degs = (np.arange(1100) * 7) % 29
    rowptr, col = random_csr(len(degs), degs, seed=71)
    case = Case(rowptr, col, 128, 16, 128, 128, 128, seed=23, eq=False)
    dt = DT["bf16"]
    p = {k: _dev(v, dt) for k, v in case.p.items()}
    row_elems = (1 << 20) + 128
    print(f"[wide-msg] N={case.N} E={case.E} row stride {row_elems}", flush=True)
    big = torch.zeros((case.N, row_elems), dtype=dt, device="cuda")
    outs = []
    for out in (None, big[:, :128]):
        o, _ = fused.egnn_fused_forward(_dev(case.h, dt), None, _dev(case.ef, dt), _dev(case.rowptr), _dev(case.col),
                                        None, p["w1_msg"], p["w2_msg"], None, None, p.get("b1"), p.get("b2"), None,
                                        equivariant=False, out_msg=out)
        outs.append(o.float().cpu().numpy())
    del big
    ref_msg, _ = case.forward_ref(True)
    for o in outs:
        err = orc.normwise_rel_err(o, ref_msg)
        print(f"[wide-msg] out_msg err {err:.1e}", flush=True)
        assert err <= TOL["bf16"]


@pytest.mark.parametrize("dtype", ["bf16", "fp32"])
def test_hidden_256(dtype):
    rowptr, col = random_csr(160, np.full(160, 40), seed=31)
    check_case(Case(rowptr, col, 256, 32, 256, 256, 256, seed=17, mean_agg=True), dtype)


@pytest.mark.parametrize("dtype", ["bf16", "fp32"])
@pytest.mark.parametrize("fe,eq,mean", [(16, True, False), (0, True, True), (16, False, False), (48, False, False),
                                        (40, True, True)])
def test_hidden_256_ragged(dtype, fe, eq, mean):
    # ragged degrees, a partial last tile, one or two 32-slot edge-input chunks (F_E + 2 > 32 for
    # EGNN, F_E > 32 for MPNN take two), EGNN and MPNN
    rowptr, col = random_csr(701, (np.arange(701) * 11) % 37, seed=33)
    check_case(Case(rowptr, col, 256, fe, 256, 256, 256, seed=19, mean_agg=mean, eq=eq), dtype)


def test_determinism_bitwise():
    rowptr, col = random_csr(500, (np.arange(500) * 13) % 50, seed=41)
    case = Case(rowptr, col, 128, 16, 128, 128, 128, seed=18)
    a = run_fused(case, "bf16")
    b = run_fused(case, "bf16")
    assert np.array_equal(a["out_msg"], b["out_msg"]) and np.array_equal(a["out_mov"], b["out_mov"])
    for k, v in a["grads"].items():
        if v is not None:
            assert np.array_equal(v, b["grads"][k]), k


@pytest.mark.parametrize("dtype,F,FE,H,O,M,eq", [
    ("bf16", 128, 0, 128, 128, 128, True),     # edge-parallel forward, cooperative backward
    ("bf16", 128, 16, 128, 128, 128, False),   # edge-parallel MPNN kernels
    ("bf16", 64, 8, 64, 32, 32, True),         # cooperative kernels, H = 64
    ("bf16", 256, 32, 256, 256, 256, True),    # wide kernels
    ("fp32", 128, 16, 128, 128, 128, True),    # one wave per tile
])
def test_linear_weight_layout(dtype, F, FE, H, O, M, eq):
    """Weights given in torch.nn.Linear layout give the packed-layout results bit for bit."""
    rowptr, col = random_csr(300, (np.arange(300) * 7) % 29, seed=52)
    case = Case(rowptr, col, F, FE, H, O, M, seed=23, eq=eq)
    a = run_fused(case, dtype)
    b = run_fused(case, dtype, linear=True)
    assert np.array_equal(a["out_msg"], b["out_msg"])
    if eq:
        assert np.array_equal(a["out_mov"], b["out_mov"])
    for k, v in a["grads"].items():
        if v is not None:
            assert np.array_equal(v, b["grads"][k]), k


@pytest.mark.parametrize("dtype", ["fp32", "bf16"])
@pytest.mark.parametrize("eq", [True, False])
def test_accumulate_grad_h(dtype, eq):
    # grad_h_into (EGNN_FLAG_ACCUMULATE_GRAD_H): the gradient of h is added to the buffer's contents,
    # here a strided view (row stride 2F) holding random values; everything else is unchanged
    from pymolecular_amd import fused
    dt = DT[dtype]
    case = molecule_case(6, 64, 0 if eq else 16, 128, 128, 128, seed=71, eq=eq, mean_agg=eq)
    rowptr, col = _dev(case.rowptr), _dev(case.col)
    h = _dev(case.h, dt)
    coord = _dev(case.coord) if case.eq else None
    ef = _dev(case.ef, dt)
    p = {k: _dev(v, dt) for k, v in case.p.items()}
    args = (h, coord, ef, rowptr, col, None, p["w1_msg"], p["w2_msg"], p.get("w1_mov"), p.get("w2_mov"),
            p.get("b1"), p.get("b2"), p.get("bx1"), _dev(case.gm, dt), _dev(case.gx) if case.eq else None)
    kw = dict(mean_agg=case.mean, equivariant=case.eq)
    print(f"[accumulate] N={case.N} E={case.E} eq={eq} dtype={dtype}", flush=True)
    g0 = fused.egnn_fused_backward(*args, **kw)
    buf = torch.randn((case.N, 2 * case.F), device="cuda").to(dt)
    base = buf[:, :case.F].float().clone()
    g1 = fused.egnn_fused_backward(*args, **kw, grad_h_into=buf[:, :case.F])
    torch.cuda.synchronize()
    assert g1["h"].data_ptr() == buf.data_ptr()
    expect = base + g0["h"].float()
    err = (buf[:, :case.F].float() - expect).abs().max().item() / expect.abs().max().item()
    assert err <= (1e-6 if dtype == "fp32" else 8e-3), err
    for k in ("w1_msg", "w2_msg", "coord", "b1"):
        if g0[k] is not None:
            assert torch.equal(g0[k], g1[k]), k


@pytest.mark.parametrize("dtype", ["fp32", "bf16"])
@pytest.mark.parametrize("shape", [(0, 128, 128, 128), (16, 128, 128, 128), (32, 256, 256, 256), (8, 64, 32, 32)])
def test_coord_residual(dtype, shape):
    # EGNN_FLAG_COORD_RESIDUAL: out_mov = coord + agg_x and grad_coord = grad_out_mov + the message
    # path's gradient, on every forward path (edge-parallel, cooperative, wide, one wave per tile), with mean
    # aggregation, empty rows and rows across many tiles (rows the fix-up writes)
    from pymolecular_amd import fused
    FE, H, O, M = shape
    dt = DT[dtype]
    degs = np.array([0, 1, 100, 0, 3, 31, 32, 33, 0, 64, 2, 200, 5, 0, 17] * 4)
    rowptr_np, col_np = random_csr(len(degs), degs, seed=8)
    case = Case(rowptr_np, col_np, 64, FE, H, O, M, seed=83, mean_agg=True)
    rowptr, col = _dev(case.rowptr), _dev(case.col)
    h, coord, ef = _dev(case.h, dt), _dev(case.coord), _dev(case.ef, dt)
    p = {k: _dev(v, dt) for k, v in case.p.items()}
    fa = (h, coord, ef, rowptr, col, None, p["w1_msg"], p["w2_msg"], p["w1_mov"], p["w2_mov"], p.get("b1"),
          p.get("b2"), p.get("bx1"))
    kw = dict(mean_agg=True, equivariant=True)
    print(f"[coord_residual] N={case.N} E={case.E} shape={shape} dtype={dtype}", flush=True)
    _, mov0 = fused.egnn_fused_forward(*fa, **kw)
    _, mov1 = fused.egnn_fused_forward(*fa, **kw, coord_residual=True)
    gx = _dev(case.gx)
    g0 = fused.egnn_fused_backward(*fa, _dev(case.gm, dt), gx, **kw)
    g1 = fused.egnn_fused_backward(*fa, _dev(case.gm, dt), gx, **kw, coord_residual=True)
    torch.cuda.synchronize()
    # one fp32 add of the same two operands in each direction: equal to the last bit
    assert torch.equal(mov1, coord + mov0)
    assert torch.equal(g1["coord"], g0["coord"] + gx)
    for k in ("h", "w1_msg", "w2_msg", "w1_mov", "b1"):
        if g0[k] is not None:
            assert torch.equal(g0[k], g1[k]), k


@pytest.mark.parametrize("dtype", ["fp32", "bf16"])
@pytest.mark.parametrize("eq,FE", [(True, 0), (True, 16), (False, 16)])
def test_no_edges(dtype, eq, FE):
    # a graph without edges: zero messages and coordinate updates, zero gradients (the edge kernels
    # launch nothing, every row is an empty fix-up row; torch hands the empty edge features over
    # as a NULL pointer)
    rowptr = np.zeros(41, np.int32)
    col = np.zeros(0, np.int32)
    case = Case(rowptr, col, 64, FE, 128, 128, 128, seed=91, eq=eq, mean_agg=eq)
    r = run_fused(case, dtype)
    assert not np.any(r["out_msg"])
    if eq:
        assert not np.any(r["out_mov"])
    for k, v in r["grads"].items():
        if v is not None:
            assert not np.any(v), k


@pytest.mark.parametrize("skewed", [False, True])
def test_identity_probe_instrument_computes_linear_sums(skewed):
    # the instrument of the gather / segment-sum timing (the edge-parallel kernels with the MLP replaced by
    # identity): messages P_i + Q_j + e W_e summed per row, dL/dpre1 = the row's message gradient summed by
    # row and by source into dh, and dW_e = sum_e e g_m,i
    from pymolecular_amd import fused
    degs = np.array([0, 300, 1, 2, 0, 129, 3, 31, 33, 0, 64, 127, 128, 5, 2, 17] * 8) if skewed else \
        (np.arange(900) * 5) % 41 + 2
    rowptr, col = random_csr(len(degs), degs, seed=51)
    case = Case(rowptr, col, 128, 16, 128, 128, 128, seed=52, eq=False, bias=False)
    bf = torch.bfloat16
    h, ef = _dev(case.h, bf), _dev(case.ef, bf)
    w1, w2 = _dev(case.p["w1_msg"], bf), _dev(case.p["w2_msg"], bf)
    gm = _dev(case.gm, bf)
    rp, cl = _dev(case.rowptr), _dev(case.col)
    out, _ = fused.egnn_fused_forward(h, None, ef, rp, cl, None, w1, w2, equivariant=False, probe_identity=True)
    g = fused.egnn_fused_backward(h, None, ef, rp, cl, None, w1, w2, None, None, None, None, None, gm, None,
                                  equivariant=False, probe_identity=True)
    torch.cuda.synchronize()
    H = 128
    hd, efd, W = orc.round_bf16(case.h), orc.round_bf16(case.ef), orc.round_bf16(case.p["w1_msg"])
    Wn1, Wn2, We = W[:H], W[H:2 * H], W[2 * H:]
    P, Q = orc.round_bf16(hd @ Wn1), orc.round_bf16(hd @ Wn2)   # stored per node in bf16
    rows = orc.csr_row_of_edge(case.rowptr)
    msg = P[rows] + Q[case.col] + efd @ We
    ref = np.zeros((case.N, H))
    np.add.at(ref, rows, msg)
    e_fwd = orc.normwise_rel_err(out.float().cpu().numpy(), ref)
    gmd = orc.round_bf16(case.gm)
    dP = np.zeros((case.N, H))
    dQ = np.zeros((case.N, H))
    np.add.at(dP, rows, gmd[rows])
    np.add.at(dQ, case.col, gmd[rows])
    dh = orc.round_bf16(dP) @ Wn1.T + orc.round_bf16(dQ) @ Wn2.T
    e_bwd = orc.normwise_rel_err(g["h"].float().cpu().numpy(), dh)
    dwe = efd.T @ gmd[rows]
    e_we = orc.normwise_rel_err(g["w1_msg"].float().cpu().numpy()[2 * H:], dwe)
    print(f"probe forward {e_fwd:.2e} backward dh {e_bwd:.2e} dW_e {e_we:.2e}", flush=True)
    assert e_fwd <= 2e-2 and e_bwd <= 2e-2 and e_we <= 2e-2, (e_fwd, e_bwd, e_we)
    assert not torch.any(g["w2_msg"].float()), "the instrument has no W_hl: its gradient is zero"
