"""Pins the CPU oracle (oracle/egnn_oracle.py) before the GPU tests trust it.

The reference ships no golden vectors, seeds or assertions, so the oracle is
pinned by what the mathematics fixes:
  * an independent formulation: the concat-form nn.Linear composition of
    E_GCL.edge_model / coord_model (oracle/torch_ref.py) for the forward and
    torch autograd for the backward;
  * central finite differences of the forward for the hand-written backward;
  * brute-force per-edge Python loops (math.exp, no numpy) on tiny graphs;
  * invariants: E(3) rotation/reflection equivariance, translation
    invariance, node relabelling, edge order within a row;
  * closed-form special cases: a single edge is the plain MLP, w2_mov = 0
    gives no coordinate update, empty rows give zeros, zero bias-free
    weights give zero messages.
Dimensions are all different (F != H != O != M) so a transposed operand fails.
"""
import math

import numpy as np
import pytest
import torch

from oracle import egnn_oracle as orc
from oracle import torch_ref
from tests.cases import make_params, random_csr, rng

F, FE, H, O, M = 6, 4, 10, 7, 5


def small_case(seed=0, N=14, eq=True, bias=True, with_eids=False, degs=None, FE_=FE):
    r = rng(seed)
    if degs is None:
        degs = r.integers(0, 6, size=N)
    rowptr, col = random_csr(N, degs, seed + 100)
    E = len(col)
    h = r.standard_normal((N, F))
    coord = r.standard_normal((N, 3)) * 1.3 if eq else None
    ef = r.standard_normal((E, FE_)) if FE_ else None
    p = {k: v.astype(np.float64) for k, v in make_params(r, F, FE_, H, O, M, eq=eq, bias=bias).items()}
    eids = r.permutation(E).astype(np.int32) if with_eids else None
    gm = r.standard_normal((N, O))
    gx = r.standard_normal((N, 3)) if eq else None
    return dict(rowptr=rowptr, col=col, h=h, coord=coord, ef=ef, p=p, eids=eids, gm=gm, gx=gx, N=N, E=E)


def concat_forward(c, mean_agg, eq, requires_grad=False):
    T = lambda a: None if a is None else torch.tensor(a, dtype=torch.float64, requires_grad=requires_grad)  # noqa
    rows = torch.tensor(orc.csr_row_of_edge(c["rowptr"]))
    col = torch.tensor(c["col"], dtype=torch.int64)
    ef = c["ef"]
    if ef is not None and c["eids"] is not None:
        ef = ef[c["eids"]]
    ts = {k: T(v) for k, v in c["p"].items()}
    h, coord = T(c["h"]), T(c["coord"])
    out = torch_ref.fused_concat(h, coord, None if ef is None else torch.tensor(ef), rows, col, ts["w1_msg"],
                                 ts["w2_msg"], ts.get("w1_mov"), ts.get("w2_mov"), ts.get("b1"), ts.get("b2"),
                                 ts.get("bx1"), mean_agg=mean_agg, equivariant=eq)
    return out, h, coord, ts


@pytest.mark.parametrize("eq", [True, False])
@pytest.mark.parametrize("mean_agg", [False, True])
@pytest.mark.parametrize("with_eids", [False, True])
def test_forward_equals_concat_form(eq, mean_agg, with_eids):
    c = small_case(1, eq=eq, with_eids=with_eids)
    om, ox = orc.fused_forward(c["h"], c["coord"], c["ef"], c["rowptr"], c["col"], c["eids"], c["p"],
                               mean_agg=mean_agg, equivariant=eq)
    (tm, tx), *_ = concat_forward(c, mean_agg, eq)
    np.testing.assert_allclose(om, tm.numpy(), rtol=1e-12, atol=1e-12)
    if eq:
        np.testing.assert_allclose(ox, tx.numpy(), rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("eq", [True, False])
@pytest.mark.parametrize("mean_agg", [False, True])
def test_backward_equals_autograd(eq, mean_agg):
    c = small_case(2, eq=eq, with_eids=True)
    g = orc.fused_backward(c["h"], c["coord"], c["ef"], c["rowptr"], c["col"], c["eids"], c["p"], c["gm"], c["gx"],
                           mean_agg=mean_agg, equivariant=eq)
    (tm, tx), h, coord, ts = concat_forward(c, mean_agg, eq, requires_grad=True)
    loss = (tm * torch.tensor(c["gm"])).sum()
    if eq:
        loss = loss + (tx * torch.tensor(c["gx"])).sum()
    loss.backward()
    np.testing.assert_allclose(g["h"], h.grad.numpy(), rtol=1e-10, atol=1e-12)
    for k in ["w1_msg", "w2_msg", "b1", "b2"] + (["w1_mov", "w2_mov", "bx1"] if eq else []):
        np.testing.assert_allclose(g[k].reshape(ts[k].shape), ts[k].grad.numpy(), rtol=1e-10, atol=1e-12, err_msg=k)
    if eq:
        np.testing.assert_allclose(g["coord"], coord.grad.numpy(), rtol=1e-10, atol=1e-12)


def test_backward_finite_differences():
    c = small_case(3, N=7, eq=True, with_eids=True)
    g = orc.fused_backward(c["h"], c["coord"], c["ef"], c["rowptr"], c["col"], c["eids"], c["p"], c["gm"], c["gx"],
                           mean_agg=True)

    def loss():
        om, ox = orc.fused_forward(c["h"], c["coord"], c["ef"], c["rowptr"], c["col"], c["eids"], c["p"],
                                   mean_agg=True)
        return float((om * c["gm"]).sum() + (ox * c["gx"]).sum())

    r = rng(9)
    eps = 1e-6
    targets = [("h", c["h"], g["h"]), ("coord", c["coord"], g["coord"])] + \
              [(k, c["p"][k], g[k].reshape(c["p"][k].shape)) for k in c["p"]]
    for name, arr, grad in targets:
        for _ in range(4):
            idx = tuple(int(r.integers(0, s)) for s in arr.shape)
            old = arr[idx]
            arr[idx] = old + eps
            lp = loss()
            arr[idx] = old - eps
            lm = loss()
            arr[idx] = old
            fd = (lp - lm) / (2 * eps)
            assert abs(fd - grad[idx]) <= 1e-6 * max(1.0, abs(fd)), (name, idx, fd, grad[idx])


def _silu(x):
    return x / (1.0 + math.exp(-x))


def test_brute_force_loops():
    c = small_case(4, N=6, eq=True, bias=True)
    W = c["p"]
    Wn1, Wn2, wd, We = orc.split_packed_w1(W["w1_msg"], F, FE)
    N = c["N"]
    msg = [[0.0] * O for _ in range(N)]
    mov = [[0.0] * 3 for _ in range(N)]
    for i in range(N):
        for e in range(c["rowptr"][i], c["rowptr"][i + 1]):
            j = int(c["col"][e])
            d = [float(c["coord"][i][k] - c["coord"][j][k]) for k in range(3)]
            r2 = sum(x * x for x in d)
            m1 = []
            for u in range(H):
                s = W["b1"][u] + r2 * wd[u]
                s += sum(c["h"][i][f] * Wn1[f][u] + c["h"][j][f] * Wn2[f][u] for f in range(F))
                s += sum(c["ef"][e][q] * We[q][u] for q in range(FE))
                m1.append(_silu(s))
            m = [_silu(W["b2"][o] + sum(m1[u] * W["w2_msg"][u][o] for u in range(H))) for o in range(O)]
            phi = sum(_silu(W["bx1"][k] + sum(m[o] * W["w1_mov"][o][k] for o in range(O))) * W["w2_mov"][k]
                      for k in range(M))
            for o in range(O):
                msg[i][o] += m[o]
            for k in range(3):
                mov[i][k] += d[k] * phi
    om, ox = orc.fused_forward(c["h"], c["coord"], c["ef"], c["rowptr"], c["col"], None, W)
    np.testing.assert_allclose(om, np.array(msg), rtol=1e-12, atol=1e-13)
    np.testing.assert_allclose(ox, np.array(mov), rtol=1e-12, atol=1e-13)


def _rotation(seed, reflect):
    q, _ = np.linalg.qr(rng(seed).standard_normal((3, 3)))
    if reflect and np.linalg.det(q) > 0:
        q[:, 0] = -q[:, 0]
    return q


@pytest.mark.parametrize("reflect", [False, True])
def test_e3_equivariance_and_translation(reflect):
    c = small_case(5)
    R = _rotation(6, reflect)
    t = np.array([3.0, -1.5, 0.25])
    om, ox = orc.fused_forward(c["h"], c["coord"], c["ef"], c["rowptr"], c["col"], None, c["p"])
    om2, ox2 = orc.fused_forward(c["h"], c["coord"] @ R + t, c["ef"], c["rowptr"], c["col"], None, c["p"])
    np.testing.assert_allclose(om2, om, rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(ox2, ox @ R, rtol=1e-10, atol=1e-12)


def test_node_relabelling():
    c = small_case(7)
    N = c["N"]
    pi = rng(8).permutation(N)           # new id of old node n is pi[n]
    inv = np.argsort(pi)
    rows = orc.csr_row_of_edge(c["rowptr"])
    new_rows, new_cols = pi[rows], pi[c["col"]]
    order = np.argsort(new_rows, kind="stable")
    rowptr2 = np.zeros(N + 1, np.int64)
    np.cumsum(np.bincount(new_rows, minlength=N), out=rowptr2[1:])
    om, ox = orc.fused_forward(c["h"], c["coord"], c["ef"], c["rowptr"], c["col"], None, c["p"])
    om2, ox2 = orc.fused_forward(c["h"][inv], c["coord"][inv], c["ef"][order], rowptr2, new_cols[order], None,
                                 c["p"])
    np.testing.assert_allclose(om2[pi], om, rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(ox2[pi], ox, rtol=1e-10, atol=1e-12)


def test_edge_order_within_row():
    c = small_case(10, degs=np.full(14, 5))
    r = rng(11)
    perm = np.concatenate([c["rowptr"][i] + r.permutation(5) for i in range(14)])
    om, ox = orc.fused_forward(c["h"], c["coord"], c["ef"], c["rowptr"], c["col"], None, c["p"])
    om2, ox2 = orc.fused_forward(c["h"], c["coord"], c["ef"][perm], c["rowptr"], c["col"][perm], None, c["p"])
    np.testing.assert_allclose(om2, om, rtol=1e-12, atol=1e-13)
    np.testing.assert_allclose(ox2, ox, rtol=1e-12, atol=1e-13)


def test_single_edge_is_plain_mlp():
    c = small_case(12, N=2, degs=np.array([1, 0]))
    W = c["p"]
    i, j = 0, int(c["col"][0])
    d = c["coord"][i] - c["coord"][j]
    x = np.concatenate([c["h"][i], c["h"][j], [d @ d], c["ef"][0]])
    lin1 = torch.nn.Linear(x.size, H).double()
    lin2 = torch.nn.Linear(H, O).double()
    lin3 = torch.nn.Linear(O, M).double()
    with torch.no_grad():
        lin1.weight.copy_(torch.tensor(W["w1_msg"].T)); lin1.bias.copy_(torch.tensor(W["b1"]))
        lin2.weight.copy_(torch.tensor(W["w2_msg"].T)); lin2.bias.copy_(torch.tensor(W["b2"]))
        lin3.weight.copy_(torch.tensor(W["w1_mov"].T)); lin3.bias.copy_(torch.tensor(W["bx1"]))
        m = torch.nn.functional.silu(lin2(torch.nn.functional.silu(lin1(torch.tensor(x)))))
        phi = float(torch.nn.functional.silu(lin3(m)) @ torch.tensor(W["w2_mov"]))
    om, ox = orc.fused_forward(c["h"], c["coord"], c["ef"], c["rowptr"], c["col"], None, W)
    np.testing.assert_allclose(om[0], m.numpy(), rtol=1e-12)
    np.testing.assert_allclose(ox[0], d * phi, rtol=1e-12)
    assert np.all(om[1] == 0) and np.all(ox[1] == 0)


def test_zero_w2mov_and_zero_weights():
    c = small_case(13)
    p = dict(c["p"])
    p["w2_mov"] = np.zeros_like(p["w2_mov"])
    _, ox = orc.fused_forward(c["h"], c["coord"], c["ef"], c["rowptr"], c["col"], None, p)
    assert np.all(ox == 0)
    z = {k: np.zeros_like(v) for k, v in c["p"].items() if not k.startswith("b")}
    om, ox = orc.fused_forward(c["h"], c["coord"], c["ef"], c["rowptr"], c["col"], None, z)
    assert np.all(om == 0) and np.all(ox == 0)


def test_empty_rows_give_zero():
    c = small_case(14, degs=np.array([0, 3, 0, 0, 2, 0, 1, 0, 0, 0, 4, 0, 0, 0]))
    om, ox = orc.fused_forward(c["h"], c["coord"], c["ef"], c["rowptr"], c["col"], None, c["p"], mean_agg=True)
    empty = np.diff(c["rowptr"]) == 0
    assert np.all(om[empty] == 0) and np.all(ox[empty] == 0)


def test_egcl_mapping_matches_module():
    # the packed mapping used by the product's E_GCL reproduces an E_GCL-style module
    torch.manual_seed(0)
    layer = torch_ref.EGCLRef(8, 8, 8, edges_in_d=3).double()
    c = small_case(15, N=9)
    rows = torch.tensor(orc.csr_row_of_edge(c["rowptr"]))
    col = torch.tensor(c["col"], dtype=torch.int64)
    h = torch.tensor(rng(1).standard_normal((9, 8)))
    x = torch.tensor(c["coord"])
    ea = torch.tensor(rng(2).standard_normal((len(col), 3)))
    h_out, x_out, _ = layer(h, (rows, col), x, ea)
    pk = {k: v.detach().numpy() for k, v in torch_ref.egcl_params_packed(layer).items()}
    om, ox = orc.fused_forward(h.numpy(), x.numpy(), ea.numpy(), c["rowptr"], c["col"], None, pk, mean_agg=True)
    with torch.no_grad():
        h_ref = h + layer.node_mlp(torch.cat([h, torch.tensor(om)], dim=1))
    np.testing.assert_allclose(x_out.detach().numpy(), x.numpy() + ox, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(h_out.detach().numpy(), h_ref.numpy(), rtol=1e-12, atol=1e-12)


def test_mpnn_mapping_matches_module():
    # the non-equivariant layer (no radial input, no coordinates) is the oracle with equivariant=False
    torch.manual_seed(1)
    layer = torch_ref.MPNNGCLRef(8, 8, 8, edges_in_d=3).double()
    c = small_case(17, N=11, eq=False)
    rows = torch.tensor(orc.csr_row_of_edge(c["rowptr"]))
    col = torch.tensor(c["col"], dtype=torch.int64)
    h = torch.tensor(rng(3).standard_normal((11, 8)))
    ea = torch.tensor(rng(4).standard_normal((len(col), 3)))
    h_out, _ = layer(h, (rows, col), ea)
    e0, e2 = layer.edge_mlp[0], layer.edge_mlp[2]
    pk = dict(w1_msg=e0.weight.t().detach().numpy(), b1=e0.bias.detach().numpy(),
              w2_msg=e2.weight.t().detach().numpy(), b2=e2.bias.detach().numpy())
    om, ox = orc.fused_forward(h.numpy(), None, ea.numpy(), c["rowptr"], c["col"], None, pk, equivariant=False)
    assert ox is None
    with torch.no_grad():
        h_ref = h + layer.node_mlp(torch.cat([h, torch.tensor(om)], dim=1))
    np.testing.assert_allclose(h_out.detach().numpy(), h_ref.numpy(), rtol=1e-12, atol=1e-12)


def test_round_bf16_matches_torch():
    a = rng(16).standard_normal(10000).astype(np.float32) * 100
    ref = torch.tensor(a).to(torch.bfloat16).to(torch.float64).numpy()
    np.testing.assert_array_equal(orc.round_bf16(a), ref)


def test_normwise_error():
    assert orc.normwise_rel_err(np.array([1.0, 2.0]), np.array([1.0, 2.0])) == 0.0
    assert abs(orc.normwise_rel_err(np.array([1.0, 2.1]), np.array([1.0, 2.0])) - 0.05) < 1e-12


def test_hoisted_first_layer_equals_concat_form():
    # the per-node products P[row] + Q[col] + W_x [r2, e] are the concat-form Linear in exact arithmetic:
    # outputs and every gradient agree to float64 roundoff, for the EGNN and the MPNN layer
    torch.manual_seed(5)
    c = small_case(18, N=13, eq=True)
    rows = torch.tensor(orc.csr_row_of_edge(c["rowptr"]))
    col = torch.tensor(c["col"], dtype=torch.int64)
    for layer in (torch_ref.EGCLRef(8, 8, 8, edges_in_d=3).double(), torch_ref.MPNNGCLRef(8, 8, 8, edges_in_d=3).double()):
        res = []
        for hoist in (False, True):
            layer.hoist_first_layer = hoist
            layer.zero_grad()
            h = torch.tensor(rng(3).standard_normal((13, 8)), requires_grad=True)
            x = torch.tensor(rng(4).standard_normal((13, 3)), requires_grad=True)
            ea = torch.tensor(rng(5).standard_normal((len(col), 3)))
            out = layer(h, (rows, col), x, ea) if isinstance(layer, torch_ref.EGCLRef) else layer(h, (rows, col), ea)
            loss = out[0].pow(2).sum() + (out[1].pow(2).sum() if isinstance(layer, torch_ref.EGCLRef) else 0)
            loss.backward()
            res.append([out[0].detach(), h.grad] + [p.grad.clone() for p in layer.parameters()]
                       + ([x.grad] if isinstance(layer, torch_ref.EGCLRef) else []))
        for a, b in zip(*res):
            np.testing.assert_allclose(b.numpy(), a.numpy(), rtol=1e-11, atol=1e-11)


def test_hoisted_first_layer_bf16_gradients():
    # bfloat16 on the CPU: the hoisted form's input gradients agree with float64 to bfloat16 resolution
    # (guards the contiguous weight slices: torch's CPU bfloat16 linear mishandles a strided weight)
    torch.manual_seed(6)
    lin = torch.nn.Linear(2 * 16 + 1, 32).double()
    rows = torch.tensor(rng(7).integers(0, 20, 200))
    col = torch.tensor(rng(8).integers(0, 20, 200))
    r2 = torch.tensor(rng(9).uniform(0, 30, (200, 1)))
    g = torch.tensor(rng(10).standard_normal((200, 32)))
    grads = []
    for dt in (torch.float64, torch.bfloat16):
        l2 = torch.nn.Linear(33, 32).to(dt)
        with torch.no_grad():
            l2.weight.copy_(lin.weight.to(torch.bfloat16))
            l2.bias.copy_(lin.bias.to(torch.bfloat16))
        h = torch.tensor(rng(11).standard_normal((20, 16))).to(torch.bfloat16).to(dt).requires_grad_()
        r = r2.float().requires_grad_()
        y = torch_ref.first_layer(l2, h, rows, col, [r], hoist=True)
        y.backward(g.to(y.dtype))
        grads.append((h.grad.double(), r.grad.double(), l2.weight.grad.double()))
    for a, b in zip(*grads):
        assert orc.normwise_rel_err(b.numpy(), a.numpy()) < 2e-2


def test_gather_rows_backward_accumulates_in_float32():
    t = torch.tensor(rng(12).standard_normal((5, 4))).to(torch.bfloat16).requires_grad_()
    idx = torch.tensor([0, 1, 1, 3] * 500)
    g = torch.full((len(idx), 4), 1.0 + 2.0 ** -7, dtype=torch.bfloat16)   # exact in bfloat16
    torch_ref.gather_rows(t, idx).backward(g)
    exact = torch.bincount(idx, minlength=5).double()[:, None] * (1.0 + 2.0 ** -7)
    np.testing.assert_array_equal(t.grad.double().numpy(), exact.to(torch.bfloat16).double().expand(5, 4).numpy())


def test_bf16_roundoff_realization_bounds():
    # every rounding point moves a value by at most the unit roundoff, and different seeds differ
    x = torch.linspace(-3, 3, 1000)
    a = torch_ref.bf16_roundoff(x, torch.Generator().manual_seed(0))
    b = torch_ref.bf16_roundoff(x, torch.Generator().manual_seed(1))
    rel = ((a.double() - x.double()).abs() / x.double().abs().clamp(min=1e-30)).max()
    assert rel <= torch_ref.BF16_UNIT_ROUNDOFF * (1 + 1e-6)
    assert not torch.equal(a, b)
    lin = torch.nn.Linear(4, 4)
    handles, act = torch_ref.bf16_rounding_realization(lin, torch.Generator().manual_seed(0))
    y = lin(torch.ones(2, 4))
    for hd in handles:
        hd.remove()
    y0 = lin(torch.ones(2, 4))
    assert 0 < (y - y0).abs().max() <= torch_ref.BF16_UNIT_ROUNDOFF * y0.abs().max() * 1.01
