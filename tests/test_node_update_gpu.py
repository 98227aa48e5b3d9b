"""Fused node update (egnn_node_fwd / egnn_node_bwd) against a float64 CPU reference.

The reference is ``oracle.torch_ref.node_update_ref``: node_mlp(cat([x1, x2]))
(+ x1) as in egnn_clean.py:60-70, with torch autograd for the gradients.
"""
import numpy as np
import pytest
import torch

from oracle import egnn_oracle as orc
from oracle import torch_ref

pytestmark = pytest.mark.gpu


def _rel(a, b):
    return orc.normwise_rel_err(a.detach().double().cpu().numpy(), b.detach().double().cpu().numpy())


def _case(N, K1, K2, Hn, Fo, seed):
    r = np.random.Generator(np.random.PCG64(seed))
    t = lambda *s: torch.from_numpy(r.standard_normal(s))  # noqa: E731
    x1, x2 = t(N, K1), (t(N, K2) if K2 else None)
    w1, b1 = t(Hn, K1 + K2) / np.sqrt(K1 + K2), t(Hn) * 0.1
    w2, b2 = t(Fo, Hn) / np.sqrt(Hn), t(Fo) * 0.1
    gout = t(N, Fo)
    return x1, x2, w1, b1, w2, b2, gout


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-5), (torch.bfloat16, 2e-2)])
@pytest.mark.parametrize("N,K1,K2,Hn,Fo,residual,bias", [
    (1000, 128, 128, 128, 128, True, True),     # E_GCL at H = 128
    (777, 32, 32, 48, 32, True, True),          # EGNN_Triton_Layer test sizes, ragged N
    (300, 64, 0, 40, 24, False, False),         # no second input, no bias, no residual
    (50000, 128, 136, 128, 128, True, True),    # many split-K slices; node attributes appended
    (4099, 128, 128, 128, 128, True, True),     # bf16: the forward in one pass below the streaming threshold
])
def test_node_update_matches_reference(dtype, tol, N, K1, K2, Hn, Fo, residual, bias):
    from pymolecular_amd.node_update import NodeUpdateFn
    x1, x2, w1, b1, w2, b2, gout = _case(N, K1, K2, Hn, Fo, N + K2)
    if not bias:
        b1 = b2 = None
    rd = (lambda t: None if t is None else t.to(torch.bfloat16).double()) if dtype == torch.bfloat16 else \
        (lambda t: t)
    ref_in = [None if t is None else rd(t).clone().requires_grad_() for t in (x1, x2, w1, b1, w2, b2)]
    out_ref = torch_ref.node_update_ref(*ref_in, residual=residual)
    (out_ref * rd(gout)).sum().backward()
    dev_in = [None if t is None else t.to(dtype).cuda().requires_grad_() for t in (x1, x2, w1, b1, w2, b2)]
    out = NodeUpdateFn.apply(*dev_in, residual)
    (out.float() * gout.to(dtype).float().cuda()).sum().backward()
    errs = {"out": _rel(out, out_ref)}
    for name, a, b in zip(["x1", "x2", "w1", "b1", "w2", "b2"], dev_in, ref_in):
        if a is not None:
            errs["d" + name] = _rel(a.grad, b.grad)
    print({k: f"{v:.1e}" for k, v in errs.items()}, flush=True)
    bad = {k: v for k, v in errs.items() if not v <= tol}
    assert not bad, bad


@pytest.mark.parametrize("N,K2,residual,bias", [
    (300001, 128, True, True),    # the power-law layer's node update, a partial last 16-row tile
    (70001, 0, False, False),     # one input, no residual, no bias
    (65541, 128, False, True),    # just above the streaming threshold, no residual
])
def test_node_update_large_bf16(N, K2, residual, bias):
    # at 65,536 rows or more with K1 = Hn = Fo = 128 both products of each direction run in one streaming
    # pass (weights in LDS, the hidden activation handed from the first product to the second in
    # registers), followed by long split-K slices for the weight gradients
    test_node_update_matches_reference(torch.bfloat16, 2e-2, N, 128, K2, 128, 128, residual, bias)


def test_node_update_deterministic_and_empty():
    from pymolecular_amd.node_update import NodeUpdateFn
    x1, x2, w1, b1, w2, b2, gout = _case(20000, 128, 128, 128, 128, 9)
    ins = [t.to(torch.bfloat16).cuda() for t in (x1, x2, w1, b1, w2, b2)]
    res = []
    for _ in range(2):
        leaves = [t.clone().requires_grad_() for t in ins]
        out = NodeUpdateFn.apply(*leaves, True)
        out.backward(gout.to(torch.bfloat16).cuda())
        res.append([out.detach()] + [t.grad for t in leaves])
    for a, b in zip(*res):
        assert torch.equal(a, b)
    # no nodes: empty output, zero weight gradients
    leaves = [t[:0].clone().requires_grad_() if i < 2 else t.clone().requires_grad_() for i, t in enumerate(ins)]
    out = NodeUpdateFn.apply(*leaves, True)
    assert out.shape == (0, 128)
    out.sum().backward()
    assert torch.count_nonzero(leaves[2].grad) == 0 and torch.count_nonzero(leaves[5].grad) == 0


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-5), (torch.bfloat16, 2e-2)])
@pytest.mark.parametrize("N,K,Nout,bias", [(19363, 5, 128, True), (3000, 128, 128, False), (500, 20, 36, True),
                                         (0, 16, 24, True), (200003, 128, 128, True)])
def test_dense_weight_gradient(dtype, tol, N, K, Nout, bias):
    from pymolecular_amd.node_update import DenseFn
    r = np.random.Generator(np.random.PCG64(N + K))
    x = torch.from_numpy(r.standard_normal((N, K)))
    w = torch.from_numpy(r.standard_normal((Nout, K)) / np.sqrt(K))
    b = torch.from_numpy(r.standard_normal(Nout)) if bias else None
    gy = torch.from_numpy(r.standard_normal((N, Nout)))
    rd = (lambda t: None if t is None else t.to(torch.bfloat16).double()) if dtype == torch.bfloat16 else \
        (lambda t: t)
    ref = [None if t is None else rd(t).clone().requires_grad_() for t in (x, w, b)]
    (torch.nn.functional.linear(*ref) * rd(gy)).sum().backward()
    dev = [None if t is None else t.to(dtype).cuda().requires_grad_() for t in (x, w, b)]
    y = DenseFn.apply(*dev)
    (y.float() * gy.to(dtype).float().cuda()).sum().backward()
    errs = {"y": _rel(y, torch.nn.functional.linear(*[None if t is None else t.detach() for t in ref]))}
    for name, a, q in zip(["x", "w", "b"], dev, ref):
        if a is not None and N > 0:
            errs["d" + name] = _rel(a.grad, q.grad)
    if N == 0:
        assert torch.count_nonzero(dev[1].grad) == 0
    print({k: f"{v:.1e}" for k, v in errs.items()}, flush=True)
    bad = {k: v for k, v in errs.items() if not v <= tol}
    assert not bad, bad


@pytest.mark.parametrize("N,K2,residual,bias", [(70001, 128, True, True), (65541, 0, False, False)])
def test_node_update_without_activation_buffer(N, K2, residual, bias):
    # streaming sizes: egnn_node_act_required is 0, so act may be NULL; the forward then leaves it unwritten
    # and the backward's [act | 1]^T dout reads SiLU of pre on load.  Every output must equal the run with
    # the buffer, bit for bit; below the streaming rows a NULL act is refused.
    from pymolecular_amd import _capi
    from pymolecular_amd.node_update import _dims, _stream
    L = _capi.lib()
    x1, x2, w1, b1, w2, b2, gout = [None if t is None else t.to(torch.bfloat16).cuda()
                                    for t in _case(N, 128, K2, 128, 128, 17 + N)]
    if not bias:
        b1 = b2 = None
    d = _dims(x1, x2, w1, w2, residual)
    assert L.egnn_node_act_required(d) == 0
    p = lambda t: None if t is None else t.data_ptr()  # noqa: E731
    st = _stream(x1.device)
    runs = []
    for with_act in (True, False):
        pre = torch.full((N, 128), float("nan"), dtype=torch.bfloat16, device="cuda")
        act = torch.full_like(pre, float("nan")) if with_act else None
        out = torch.empty((N, 128), dtype=torch.bfloat16, device="cuda")
        rc = L.egnn_node_fwd(d, x1.data_ptr(), x1.stride(0), p(x2), 0 if x2 is None else x2.stride(0), w1.data_ptr(),
                             p(b1), w2.data_ptr(), p(b2), pre.data_ptr(), p(act), out.data_ptr(), out.stride(0), st)
        assert rc == 0, _capi.lib().egnn_status_string(rc)
        gx = torch.empty((N, 128 + K2), dtype=torch.bfloat16, device="cuda")
        gw1, gw2 = torch.empty_like(w1), torch.empty_like(w2)
        gb1 = torch.empty(128, dtype=torch.bfloat16, device="cuda") if bias else None
        gb2 = torch.empty(128, dtype=torch.bfloat16, device="cuda") if bias else None
        nb = L.egnn_node_bwd_workspace_bytes(d)
        ws = torch.empty(nb, dtype=torch.uint8, device="cuda")
        rc = L.egnn_node_bwd(d, x1.data_ptr(), x1.stride(0), p(x2), 0 if x2 is None else x2.stride(0), w1.data_ptr(),
                             w2.data_ptr(), pre.data_ptr(), p(act), gout.data_ptr(), gout.stride(0), gx.data_ptr(),
                             gw1.data_ptr(), p(gb1), gw2.data_ptr(), p(gb2), ws.data_ptr(), nb, st)
        assert rc == 0, _capi.lib().egnn_status_string(rc)
        torch.cuda.synchronize()
        if with_act:   # the stored act is SiLU of pre's bf16 value, rounded to bf16
            ref = torch.nn.functional.silu(pre.float()).to(torch.bfloat16)
            assert (act.float() - ref.float()).abs().max().item() <= 2 ** -8 * ref.float().abs().max().item()
        runs.append([t for t in (out, pre, gx, gw1, gb1, gw2, gb2) if t is not None])
    for name, a, b in zip(["out", "pre", "grad_x", "gw1", "gb1", "gw2", "gb2"], *runs):
        assert torch.equal(a, b), name
    small = _dims(x1[:1000], None if x2 is None else x2[:1000], w1, w2, residual)
    assert L.egnn_node_act_required(small) == 1
    pre = torch.empty((1000, 128), dtype=torch.bfloat16, device="cuda")
    out = torch.empty((1000, 128), dtype=torch.bfloat16, device="cuda")
    rc = L.egnn_node_fwd(small, x1.data_ptr(), x1.stride(0), p(x2), 0 if x2 is None else x2.stride(0), w1.data_ptr(),
                         p(b1), w2.data_ptr(), p(b2), pre.data_ptr(), None, out.data_ptr(), out.stride(0), st)
    assert rc == _capi.EGNN_ERR_NULL
