"""The reference's Python surface on the HIP layer: E_GCL/EGNN, EGNN_Triton_Layer,
pytorch_egnn_baseline, the kernel-signature launchers and generate_graph_data.

Each is compared with the CPU oracle (oracle/torch_ref.py in float64, or the
numpy oracle) on the same seeded inputs.
"""
import numpy as np
import pytest
import torch

from oracle import egnn_oracle as orc
from oracle import torch_ref
from pymolecular_amd import graphs

pytestmark = pytest.mark.gpu


def _copy_weights(dst, src):
    with torch.no_grad():
        for (n1, p1), (n2, p2) in zip(dst.named_parameters(), src.named_parameters()):
            p1.copy_(p2.to(p1.dtype))


def _rel(a, b):
    return orc.normwise_rel_err(a.detach().double().cpu().numpy(), b.detach().double().cpu().numpy())


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-5), (torch.bfloat16, 2e-2)])
@pytest.mark.parametrize("edges_in_d", [0, 16])
def test_egcl_layer_forward_backward(dtype, tol, edges_in_d):
    from pymolecular_amd.models.EGNN import E_GCL
    torch.manual_seed(0)
    H = 128
    g = graphs.molecule_batch(12, seed=21, feat_seed=22)
    rows = torch.from_numpy(g.rows().astype(np.int64))
    cols = torch.from_numpy(g.col.astype(np.int64))
    ref = torch_ref.EGCLRef(H, H, H, edges_in_d=edges_in_d).double()
    torch.nn.init.xavier_uniform_(ref.coord_mlp[2].weight, gain=1.0)     # exercise the x path
    mod = E_GCL(H, H, H, edges_in_d=edges_in_d).cuda().to(dtype)
    _copy_weights(mod, ref)
    r = np.random.Generator(np.random.PCG64(5))
    h = torch.from_numpy(r.standard_normal((g.N, H)))
    x = torch.from_numpy(g.coord.astype(np.float64))
    ea = torch.from_numpy(r.standard_normal((g.E, edges_in_d))) if edges_in_d else None
    wh = torch.from_numpy(r.standard_normal((g.N, H)))
    wx = torch.from_numpy(r.standard_normal((g.N, 3)))
    # reference (fp64 CPU; for bf16, on bf16-rounded inputs and weights)
    rd = (lambda t: t.to(torch.bfloat16).double()) if dtype == torch.bfloat16 else (lambda t: t)
    with torch.no_grad():
        for p in ref.parameters():
            p.copy_(rd(p))
    hr = rd(h).detach().clone().requires_grad_()
    xr = x.detach().clone().requires_grad_()
    ho, xo, _ = ref(hr, (rows, cols), xr, None if ea is None else rd(ea))
    ((ho * wh).sum() + (xo * wx).sum()).backward()
    # device
    hd = h.detach().to(dtype).cuda().requires_grad_()
    xd = x.detach().float().cuda().requires_grad_()
    ho2, xo2, _ = mod(hd, (rows.cuda(), cols.cuda()), xd, None if ea is None else ea.to(dtype).cuda())
    ((ho2.float() * wh.float().cuda()).sum() + (xo2 * wx.float().cuda()).sum()).backward()
    errs = {"h_out": _rel(ho2, ho), "x_out": _rel(xo2, xo), "dh": _rel(hd.grad, hr.grad), "dx": _rel(xd.grad, xr.grad)}
    for (n, p), (_, q) in zip(mod.named_parameters(), ref.named_parameters()):
        errs["d" + n] = _rel(p.grad, q.grad)
    print({k: f"{v:.1e}" for k, v in errs.items()}, flush=True)
    bad = {k: v for k, v in errs.items() if not v <= tol}
    assert not bad, bad


def _grads_rel(mod_named, ref_named, rename=lambda n: n):
    refp = {rename(n): p for n, p in ref_named}
    return {"d" + n: _rel(p.grad, refp[n].grad) for n, p in mod_named}


def _loss_weights(N, F):
    """Seeded N(0, 1) weights of the stack tests' loss <h_out, w_h> + <x_out, w_x>.  With a constant
    upstream coordinate gradient (the all-ones sum-of-outputs loss) the coordinate MLP's weight
    gradients are sums of edge pairs that cancel almost exactly (delta_ij = -delta_ji while
    m_ij ~ m_ji), which leaves nothing to compare; random weights remove that pairing."""
    r = np.random.Generator(np.random.PCG64(77))
    return torch.from_numpy(r.standard_normal((N, F))), torch.from_numpy(r.standard_normal((N, 3)))


def _torch_lowp_errs(ref, dtype, run, n_realizations=8):
    """Errors of the same stack run in plain torch on the CPU at ``dtype`` against the float64 ``ref``
    (whose gradients are set), per quantity: the measured conditioning at that precision.

    fp32: the concat form.  bf16: the largest error of
      * the stack in torch bfloat16, concat form;
      * the same with the hoisted first layer (torch_ref.first_layer: the per-node products the fused
        layer forms, rounded where it rounds them) -- the same arithmetic rounded at other points;
      * ``n_realizations`` float32 runs that give every Linear and SiLU output, the activations
        between layers and all their gradients a random relative error of bfloat16's unit roundoff
        (torch_ref.bf16_rounding_realization, seeds 0..n-1).
    A quantity that is a sum of many terms of either sign (the coordinate MLP's weight gradients:
    the terms carry delta_ij . g_x,i) magnifies the rounding of its terms by the sum's condition
    number, and which realization of the rounding a run gets decides where in that range it lands.
    ``run(model, act_round)`` returns ``{name: (output, reference output)}`` after the backward."""
    import copy
    errs = []

    def measure(m, act_round=None):
        for p in m.parameters():
            p.grad = None
        outs = run(m, act_round)
        e = {k: _rel(o, r) for k, (o, r) in outs.items()}
        e.update(_grads_rel(m.named_parameters(), ref.named_parameters()))
        errs.append(e)

    if dtype == torch.float32:
        measure(copy.deepcopy(ref).float())
    else:
        for hoist in (False, True):
            measure(torch_ref.set_hoist(copy.deepcopy(ref).to(dtype), hoist))
        for seed in range(n_realizations):
            m = copy.deepcopy(ref).float()
            _, act_round = torch_ref.bf16_rounding_realization(m, torch.Generator().manual_seed(seed))
            measure(m, act_round)
    worst = {k: max(e[k] for e in errs) for k in errs[0]}
    return {k.replace("layers.", "gcl_"): v for k, v in worst.items()}


def _stack_bounds(errs_cpu, dtype):
    """Per-quantity bounds of the stack tests: the per-layer contract, or twice the error the same
    stack makes on the CPU at the same precision (_torch_lowp_errs) where that is larger -- a
    quantity whose sum largely cancels.  fp32: max(1e-5, 2 err_fp32); bf16: max(2e-2, 2 err_bf16)."""
    floor = 2e-2 if dtype == torch.bfloat16 else 1e-5
    return {k: max(floor, 2.0 * v) for k, v in errs_cpu.items()}


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_egnn_stack(dtype, record_error):
    from pymolecular_amd.models.EGNN import EGNN
    torch.manual_seed(1)
    H = 128
    g = graphs.molecule_batch(10, seed=31, feat_seed=32)
    edges = [torch.from_numpy(g.rows().astype(np.int64)), torch.from_numpy(g.col.astype(np.int64))]
    ref = torch_ref.EGNNRef(5, H, 16, 0, n_layers=4).double()
    mod = EGNN(5, H, 16, 0, n_layers=4).cuda().to(dtype)
    bf = dtype == torch.bfloat16
    with torch.no_grad():
        if bf:
            for p in ref.parameters():
                p.copy_(p.to(torch.bfloat16).double())
    # state dicts map 1:1 except the layer container name
    ren = lambda n: n.replace("layers.", "gcl_")  # noqa: E731
    pm = dict(mod.named_parameters())
    for n, p in ref.named_parameters():
        with torch.no_grad():
            pm[ren(n)].copy_(p.to(dtype))
    h = torch.from_numpy(g.node_feat.astype(np.float64))
    x = torch.from_numpy(g.coord.astype(np.float64))
    wh, wx = _loss_weights(g.N, 16)
    ho, xo = ref(h, x, edges, act_round=torch_ref.round_bf16_st if bf else None)
    ((ho * wh).sum() + (xo * wx).sum()).backward()

    def run_cpu(m, act_round):   # h in the model's dtype, coordinates in float32 (as on the device)
        hc, xc = m(h.to(next(m.parameters()).dtype), x.float(), edges, act_round=act_round)
        ((hc.float() * wh.float()).sum() + (xc.float() * wx.float()).sum()).backward()
        return {"h_out": (hc, ho), "x_out": (xc, xo)}

    ec = _torch_lowp_errs(ref, dtype, run_cpu)
    ho2, xo2 = mod(h.to(dtype).cuda(), x.float().cuda(), [e.cuda() for e in edges], None)
    ((ho2.float() * wh.float().cuda()).sum() + (xo2 * wx.float().cuda()).sum()).backward()
    errs = {"h_out": _rel(ho2, ho), "x_out": _rel(xo2, xo), **_grads_rel(mod.named_parameters(),
                                                                        ref.named_parameters(), ren)}
    bounds = _stack_bounds(ec, dtype)
    for k, v in errs.items():
        record_error(k, v, bounds[k])
        record_error(k + f" (torch {str(dtype)[6:]} cpu)", ec[k], bounds[k])
    bad = {k: v for k, v in errs.items() if not v <= bounds[k]}
    assert not bad, bad


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_mpnn_stack(dtype, record_error):
    # non-equivariant stack (2 layers, 16-dim edge features) on a skewed-degree graph
    from pymolecular_amd.models.EGNN import MPNN
    torch.manual_seed(3)
    H, FE = 128, 16
    g = graphs.powerlaw_graph(N=3000, dmax=400, seed=41, feat_seed=42, F=H, FE=FE)
    edges = [torch.from_numpy(g.rows().astype(np.int64)), torch.from_numpy(g.col.astype(np.int64))]
    ref = torch_ref.MPNNRef(H, H, 32, FE, n_layers=2).double()
    mod = MPNN(H, H, 32, FE, n_layers=2).cuda().to(dtype)
    bf = dtype == torch.bfloat16
    with torch.no_grad():
        if bf:
            for p in ref.parameters():
                p.copy_(p.to(torch.bfloat16).double())
    ren = lambda n: n.replace("layers.", "gcl_")  # noqa: E731
    pm = dict(mod.named_parameters())
    for n, p in ref.named_parameters():
        with torch.no_grad():
            pm[ren(n)].copy_(p.to(dtype))
    rd = (lambda t: t.to(torch.bfloat16).double()) if bf else (lambda t: t)
    h = rd(torch.from_numpy(g.node_feat.astype(np.float64)))
    ea = rd(torch.from_numpy(g.edge_attr.astype(np.float64)))
    wh, _ = _loss_weights(g.N, 32)
    ho = ref(h, edges, ea, act_round=torch_ref.round_bf16_st if bf else None)
    (ho * wh).sum().backward()

    def run_cpu(m, act_round):
        dt = next(m.parameters()).dtype
        hc = m(h.to(dt), edges, ea.to(dt), act_round=act_round)
        (hc.float() * wh.float()).sum().backward()
        return {"h_out": (hc, ho)}

    ec = _torch_lowp_errs(ref, dtype, run_cpu)
    ho2 = mod(h.to(dtype).cuda(), [e.cuda() for e in edges], ea.to(dtype).cuda())
    (ho2.float() * wh.float().cuda()).sum().backward()
    errs = {"h_out": _rel(ho2, ho), **_grads_rel(mod.named_parameters(), ref.named_parameters(), ren)}
    bounds = _stack_bounds(ec, dtype)
    for k, v in errs.items():
        record_error(k, v, bounds[k])
        record_error(k + f" (torch {str(dtype)[6:]} cpu)", ec[k], bounds[k])
    bad = {k: v for k, v in errs.items() if not v <= bounds[k]}
    assert not bad, bad


def _graph_data(n=600, deg=32, scaled=False):
    """generate_graph_data's 16-tuple (F 32, F_E 16, H 64, O = M = 32).

    scaled=False: its weights as the reference draws them (unscaled N(0, 1): most SiLU inputs of
    the layer are saturated).  scaled=True: the same draws divided by the square root of each
    layer's fan-in, so that the pre-activations are O(1) and the sigmoid's curved range is exercised;
    the packed w1_msg is rebuilt from the scaled parts."""
    from pymolecular_amd.datasets_loaders import generate_graph_data
    d = list(generate_graph_data(n, deg, 32, 16, 64, 32, 32, seed=7, device="cuda"))
    if scaled:
        F, FE, H, O, M = 32, 16, 64, 32, 32
        k1 = (2 * F + 1 + FE) ** -0.5
        for i in (6, 7, 8, 9):   # w1, w2src, wd, we: rows of the first layer's input
            d[i] = d[i] * k1
        d[10] = d[10] * H ** -0.5   # whl
        d[11] = d[11] * O ** -0.5   # w1m
        d[12] = d[12] * M ** -0.5   # w2m
        d[13] = torch.cat([d[6], d[7], d[8][None], d[9]]).reshape(-1).contiguous()
    return tuple(d)


def test_generate_graph_data_contract():
    d = _graph_data(100, 8)
    assert len(d) == 16
    h, coord, ef, rp, col, eids = d[:6]
    assert rp.dtype == torch.int32 and col.dtype == torch.int32 and eids.dtype == torch.int32
    assert rp.shape == (101,) and col.shape == (800,) and coord.shape == (100, 4)
    assert torch.all(coord[:, 3] == 0)
    packed = d[13]
    assert torch.equal(packed, torch.cat([d[6], d[7], d[8][None], d[9]]).reshape(-1))


def _oracle_inputs(d):
    (h, coord, ef, rp, col, eids, w1, w2src, wd, we, whl, w1m, w2m, packed, gm, gx) = [t.detach().cpu().numpy() for t in d]
    p = dict(w1_msg=np.concatenate([w1, w2src, wd[None], we]).astype(np.float64), w2_msg=whl, w1_mov=w1m, w2_mov=w2m)
    return h, coord, ef, rp, col, eids, p, gm, gx


@pytest.mark.parametrize("scaled", [False, True])
def test_pytorch_egnn_baseline_signature(scaled):
    from pymolecular_amd.models.EGNN import pytorch_egnn_baseline
    d = _graph_data(scaled=scaled)
    row_indices = torch.repeat_interleave(torch.arange(600, device="cuda"), d[3][1:] - d[3][:-1])
    gh, gc = pytorch_egnn_baseline(d[0], d[1], d[2], row_indices, d[4], d[6], d[7], d[11], d[12], d[9], d[8], d[10],
                                   d[14], d[15])
    h, coord, ef, rp, col, eids, p, gm, gx = _oracle_inputs(d)
    ref = orc.fused_backward(h, coord, ef, rp, col, None, p, gm, gx)
    e1, e2 = orc.normwise_rel_err(gh.cpu().numpy(), ref["h"]), orc.normwise_rel_err(gc[:, :3].cpu().numpy(), ref["coord"])
    print(f"dh {e1:.1e} dx {e2:.1e}")
    assert e1 <= 1e-5 and e2 <= 1e-5 and torch.all(gc[:, 3] == 0)


@pytest.mark.parametrize("scaled", [False, True])
def test_kernel_signature_launchers(scaled):
    from pymolecular_amd.models.EGNN import egnn_backward_kernel_node_parallel, egnn_forward_kernel_node_parallel
    d = _graph_data(scaled=scaled)
    (h, coord, ef, rp, col, eids, w1, w2src, wd, we, whl, w1m, w2m, packed, gm, gx) = d
    N = 600
    kw = dict(F_NODE=32, F_EDGE=16, HIDDEN_FEATURES=64, OUT_FEATURES=32, HID_FEAT_MOV_MLP=32)
    out_msg = torch.zeros((N, 32), device="cuda")
    out_mov = torch.zeros((N, 4), device="cuda")
    egnn_forward_kernel_node_parallel[(N,)](h, coord, ef, rp, col, eids, out_msg, out_mov, packed, whl, w1m, w2m,
                                           h.stride(0), coord.stride(0), ef.stride(0), out_msg.stride(0),
                                           out_mov.stride(0), N, BLOCK_SIZE_NEIGHBORS=32, **kw)
    grads = [torch.zeros_like(h), torch.zeros_like(coord), torch.zeros_like(packed), torch.zeros_like(whl),
             torch.zeros_like(w1m), torch.zeros_like(w2m)]
    egnn_backward_kernel_node_parallel[(N,)](h, coord, ef, rp, col, eids, gm, gx, *grads, packed, whl, w1m, w2m,
                                            h.stride(0), coord.stride(0), ef.stride(0), gm.stride(0), gx.stride(0), N,
                                            **kw)
    hn, cn, efn, rpn, coln, eidn, p, gmn, gxn = _oracle_inputs(d)
    om, ox = orc.fused_forward(hn, cn, efn, rpn, coln, eidn, p)
    g = orc.fused_backward(hn, cn, efn, rpn, coln, eidn, p, gmn, gxn)
    errs = dict(out_msg=orc.normwise_rel_err(out_msg.cpu().numpy(), om),
                out_mov=orc.normwise_rel_err(out_mov[:, :3].cpu().numpy(), ox),
                dh=orc.normwise_rel_err(grads[0].cpu().numpy(), g["h"]),
                dx=orc.normwise_rel_err(grads[1][:, :3].cpu().numpy(), g["coord"]),
                dw1=orc.normwise_rel_err(grads[2].cpu().numpy(), g["w1_msg"].reshape(-1)),
                dw2=orc.normwise_rel_err(grads[3].cpu().numpy(), g["w2_msg"]),
                dw1m=orc.normwise_rel_err(grads[4].cpu().numpy(), g["w1_mov"]),
                dw2m=orc.normwise_rel_err(grads[5].cpu().numpy(), g["w2_mov"]))
    print({k: f"{v:.1e}" for k, v in errs.items()})
    assert all(v <= 1e-5 for v in errs.values()), errs
    assert torch.all(out_mov[:, 3] == 0)


def test_egnn_triton_layer_bidirectional():
    from pymolecular_amd.models.EGNN import EGNN_Triton_Layer
    torch.manual_seed(2)
    F, FE = 32, 16
    layer = EGNN_Triton_Layer(F, FE, 64, 32, 32, 48).cuda()
    r = np.random.Generator(np.random.PCG64(11))
    N, E = 200, 900
    src, dst = r.integers(0, N, E), r.integers(0, N, E)
    h = r.standard_normal((N, F)).astype(np.float32)
    x = r.standard_normal((N, 4)).astype(np.float32)
    ef = r.standard_normal((E, FE)).astype(np.float32)
    ei = torch.from_numpy(np.stack([src, dst]).astype(np.int64)).cuda()
    hn, xn = layer(torch.from_numpy(h).cuda(), torch.from_numpy(x).cuda(), ei, torch.from_numpy(ef).cuda())
    # oracle: messages in both directions, coordinate sum over the incident degree
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
    e_h, e_x = orc.normwise_rel_err(hn.detach().cpu().numpy(), h_ref), orc.normwise_rel_err(xn.detach().cpu().numpy(), x_ref)
    print(f"h {e_h:.1e} x {e_x:.1e}")
    assert e_h <= 1e-5 and e_x <= 1e-5
