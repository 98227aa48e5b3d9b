"""Node update of a layer on the HIP library: ``[x1 | x2] -> Linear -> SiLU -> Linear (+ x1)``.

This is the per-node epilogue the reference runs as torch modules after the
message sum: ``E_GCL.node_model`` (egnn_clean.py:60-70: node_mlp on
``cat([h, agg])`` plus the residual) and ``EGNN_Triton_Layer.forward``
(layer.py:97-101: ``node_feat + node_mlp(cat([node_feat, total_msg]))``).
Here the concatenation is never materialised (the first GEMM reads both
inputs), bias, SiLU and residual are GEMM epilogues, and the backward's weight
gradients are split-K products summed in a fixed order (``egnn_node_fwd`` /
``egnn_node_bwd`` in include/egnn.h).  No CPU path: ROCm tensors only.
"""
from __future__ import annotations

from typing import Optional

import torch

from . import _capi
from ._capi import EgnnNodeDims, check
from .fused import _as, _stream

__all__ = ["NodeUpdateFn", "node_update", "node_update_forward", "node_update_backward", "DenseFn", "dense"]


def _rowmajor(t: torch.Tensor) -> torch.Tensor:
    """``t`` if its rows are unit-stride with 16-byte aligned row starts, else a contiguous copy."""
    esz = t.element_size()
    if t.stride(1) == 1 and (t.stride(0) * esz) % 16 == 0 and t.data_ptr() % 16 == 0:
        return t
    return t.contiguous()


def _dims(x1, x2, w1, w2, residual) -> EgnnNodeDims:
    if x1.dtype == torch.float32:
        dt = _capi.EGNN_F32
    elif x1.dtype == torch.bfloat16:
        dt = _capi.EGNN_BF16
    else:
        raise TypeError(f"unsupported dtype {x1.dtype}: the node update runs in float32 or bfloat16")
    N, K1 = x1.shape
    K2 = 0 if x2 is None else int(x2.shape[1])
    Hn, K = w1.shape
    Fo = int(w2.shape[0])
    if K != K1 + K2 or w2.shape[1] != Hn:
        raise ValueError(f"weight shapes {tuple(w1.shape)}, {tuple(w2.shape)} do not match inputs of width "
                         f"{K1} + {K2}")
    if K1 % 8 or K2 % 8 or Hn % 8 or Fo % 8:
        raise ValueError(f"the node update needs widths that are multiples of 8 (got {K1}, {K2}, {Hn}, {Fo})")
    if residual and Fo != K1:
        raise ValueError(f"residual update needs output width {Fo} == input width {K1}")
    return EgnnNodeDims(N=N, K1=K1, K2=K2, Hn=Hn, Fo=Fo, residual=1 if residual else 0, dtype=dt)


def _ptr(t: Optional[torch.Tensor]):
    return None if t is None else t.data_ptr()


def node_update_forward(x1, x2, w1, b1, w2, b2, residual=True):
    """``egnn_node_fwd``: returns ``(out, saved)``; ``saved`` is what :func:`node_update_backward` needs."""
    if not x1.is_cuda:
        raise RuntimeError("x1 must be a ROCm device tensor: the node update has no CPU path")
    dt = x1.dtype
    x1 = _rowmajor(x1)
    x2 = None if x2 is None else _rowmajor(x2 if x2.dtype == dt else x2.to(dt))
    w1c, b1c, w2c, b2c = _as(w1, dt), _as(b1, dt), _as(w2, dt), _as(b2, dt)
    d = _dims(x1, x2, w1c, w2c, residual)
    N = x1.shape[0]
    pre = torch.empty((N, d.Hn), dtype=dt, device=x1.device)
    L = _capi.lib()
    # the streaming passes recompute act from pre in the backward's weight-gradient product
    act = torch.empty_like(pre) if L.egnn_node_act_required(d) else None
    out = torch.empty((N, d.Fo), dtype=dt, device=x1.device)
    st = _stream(x1.device)
    rc = L.egnn_node_fwd(d, x1.data_ptr(), x1.stride(0), _ptr(x2), 0 if x2 is None else x2.stride(0),
                         w1c.data_ptr(), _ptr(b1c), w2c.data_ptr(), _ptr(b2c), pre.data_ptr(), _ptr(act),
                         out.data_ptr(), out.stride(0), st)
    check("egnn_node_fwd", rc)
    wdt = (w1.dtype, None if b1 is None else b1.dtype, w2.dtype, None if b2 is None else b2.dtype)
    return out, ((x1, x2, w1c, w2c, pre, act), residual, (b1 is not None, b2 is not None), wdt)


def node_update_backward(tensors, residual, has_b, wdt, gout):
    """``egnn_node_bwd``: returns ``(grad_x, gw1, gb1, gw2, gb2)``, ``grad_x`` the (N, K1 + K2)
    gradient of ``[x1 | x2]`` (a fresh buffer the caller may add into)."""
    x1, x2, w1, w2, pre, act = tensors
    dt = x1.dtype
    gout = _rowmajor(gout if gout.dtype == dt else gout.to(dt))
    d = _dims(x1, x2, w1, w2, residual)
    N = x1.shape[0]
    dev = x1.device
    grad_x = torch.empty((N, d.K1 + d.K2), dtype=dt, device=dev)
    gw1, gw2 = torch.empty_like(w1), torch.empty_like(w2)
    gb1 = torch.empty((d.Hn,), dtype=dt, device=dev) if has_b[0] else None
    gb2 = torch.empty((d.Fo,), dtype=dt, device=dev) if has_b[1] else None
    L = _capi.lib()
    nbytes = L.egnn_node_bwd_workspace_bytes(d)
    ws = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=dev)
    st = _stream(dev)
    rc = L.egnn_node_bwd(d, x1.data_ptr(), x1.stride(0), _ptr(x2), 0 if x2 is None else x2.stride(0),
                         w1.data_ptr(), w2.data_ptr(), pre.data_ptr(), _ptr(act), gout.data_ptr(),
                         gout.stride(0), grad_x.data_ptr(), gw1.data_ptr(), _ptr(gb1), gw2.data_ptr(),
                         _ptr(gb2), ws.data_ptr(), nbytes, st)
    check("egnn_node_bwd", rc)
    w1dt, b1dt, w2dt, b2dt = wdt
    return grad_x, _as(gw1, w1dt), _as(gb1, b1dt), _as(gw2, w2dt), _as(gb2, b2dt)


class NodeUpdateFn(torch.autograd.Function):
    """``out = NodeUpdateFn.apply(x1, x2, w1, b1, w2, b2, residual)``.

    ``w1`` (Hn, K1 + K2) and ``w2`` (Fo, Hn) in torch.nn.Linear layout; ``b1``
    and ``b2`` may be None.  Saves the pre-activation and, where the library
    needs it (``egnn_node_act_required``), the activation (N x Hn each) for the
    backward.
    """

    @staticmethod
    def forward(ctx, x1, x2, w1, b1, w2, b2, residual=True):
        out, (tensors, res, has_b, wdt) = node_update_forward(x1, x2, w1, b1, w2, b2, residual)
        ctx.save_for_backward(*tensors)
        ctx.residual, ctx.has_b, ctx.wdt = res, has_b, wdt
        ctx.has_x2 = x2 is not None
        return out

    @staticmethod
    def backward(ctx, gout):
        tensors = ctx.saved_tensors
        grad_x, gw1, gb1, gw2, gb2 = node_update_backward(tensors, ctx.residual, ctx.has_b, ctx.wdt, gout)
        K1 = tensors[0].shape[1]
        g_x2 = grad_x[:, K1:] if ctx.has_x2 else None
        return grad_x[:, :K1], g_x2, gw1, gb1, gw2, gb2, None


def node_update(x1: torch.Tensor, x2: Optional[torch.Tensor], lin1: torch.nn.Linear, lin2: torch.nn.Linear,
                residual: bool = True) -> torch.Tensor:
    """``x1 + lin2(SiLU(lin1(cat([x1, x2]))))`` (without ``x1 +`` when not residual)."""
    return NodeUpdateFn.apply(x1, x2, lin1.weight, lin1.bias, lin2.weight, lin2.bias, residual)


def _pad_to8(t: torch.Tensor, dim: int) -> torch.Tensor:
    """``t`` with zeros appended along ``dim`` up to a multiple of 8 (16-byte bf16 rows)."""
    n = t.shape[dim]
    if n % 8 == 0:
        return t
    pad = [0, 0] * (t.dim() - 1 - (dim % t.dim())) + [0, 8 - n % 8]
    return torch.nn.functional.pad(t, pad)


class DenseFn(torch.autograd.Function):
    """``y = DenseFn.apply(x, weight, bias)``: torch.nn.functional.linear on the
    library's GEMM (``egnn_dense_fwd``), with the weight gradient over the N
    rows as its deterministic split-K product (``egnn_dense_wgrad``); the
    stack's embedding layers use it (egnn_clean.py:127-128, 139-145).  Input and
    output widths that are not multiples of 8 are padded with zero columns."""

    @staticmethod
    def forward(ctx, x, weight, bias):
        if not x.is_cuda:
            raise RuntimeError("x must be a ROCm device tensor")
        dt = x.dtype
        if dt not in (torch.float32, torch.bfloat16):
            raise TypeError(f"unsupported dtype {dt}")
        Nout, Kin = weight.shape
        lead = x.shape[:-1]
        xp = _rowmajor(_pad_to8(x.reshape(-1, Kin), 1))
        wp = _as(_pad_to8(_pad_to8(_as(weight, dt), 1), 0), dt)
        bp = None if bias is None else _as(_pad_to8(_as(bias, dt), 0), dt)
        N, Kp = xp.shape
        Np = wp.shape[0]
        y = torch.empty((N, Np), dtype=dt, device=x.device)
        code = _capi.EGNN_F32 if dt == torch.float32 else _capi.EGNN_BF16
        st = _stream(x.device)
        rc = _capi.lib().egnn_dense_fwd(code, N, Kp, Np, xp.data_ptr() if N else None, xp.stride(0) if N else Kp,
                                        wp.data_ptr(), _ptr(bp), y.data_ptr() if N else None, Np, st)
        check("egnn_dense_fwd", rc)
        ctx.save_for_backward(xp, wp)
        ctx.dims = (Kin, Nout, lead)
        ctx.has_b = bias is not None
        ctx.wdt = (weight.dtype, None if bias is None else bias.dtype)
        return (y if Np == Nout else y[:, :Nout]).reshape(*lead, Nout)

    @staticmethod
    def backward(ctx, gy):
        xp, wp = ctx.saved_tensors
        Kin, Nout, lead = ctx.dims
        dt = xp.dtype
        N, Kp = xp.shape
        Np = wp.shape[0]
        gy2 = _rowmajor(_pad_to8((gy if gy.dtype == dt else gy.to(dt)).reshape(-1, Nout), 1))
        gx = None
        L = _capi.lib()
        code = _capi.EGNN_F32 if dt == torch.float32 else _capi.EGNN_BF16
        st = _stream(xp.device)
        if ctx.needs_input_grad[0]:   # gx = gy w, the padded weight read as it is
            gx = torch.empty((N, Kp), dtype=dt, device=xp.device)
            if N:
                check("egnn_dense_dgrad", L.egnn_dense_dgrad(code, N, Kp, Np, gy2.data_ptr(), gy2.stride(0),
                                                             wp.data_ptr(), gx.data_ptr(), Kp, st))
            gx = gx[:, :Kin].reshape(*lead, Kin)
        # the weight gradient at the layer's own widths (the padded columns of x and gy are not read),
        # so it is stored in the parameter's shape
        gw = torch.empty((Nout, Kin), dtype=dt, device=xp.device)
        gb = torch.empty((Nout,), dtype=dt, device=xp.device) if ctx.has_b else None
        nbytes = L.egnn_dense_wgrad_workspace_bytes(N, Kin, Nout)
        ws = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=xp.device)
        rc = L.egnn_dense_wgrad(code, N, Kin, Nout, xp.data_ptr() if N else None, xp.stride(0) if N else Kp,
                                gy2.data_ptr() if N else None, gy2.stride(0) if N else Np, gw.data_ptr(), _ptr(gb),
                                ws.data_ptr(), nbytes, st)
        check("egnn_dense_wgrad", rc)
        to = lambda t, d: t if t.dtype == d else t.to(d)  # noqa: E731
        return gx, to(gw, ctx.wdt[0]), None if gb is None else to(gb, ctx.wdt[1])


def dense(x: torch.Tensor, lin: torch.nn.Linear) -> torch.Tensor:
    """``lin(x)`` with the split-K weight gradient of :class:`DenseFn`."""
    return DenseFn.apply(x, lin.weight, lin.bias)
