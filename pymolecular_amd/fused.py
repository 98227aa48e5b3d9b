"""Host side of the fused EGNN/MPNN layer: schedule cache, workspaces, autograd.

Everything here is plumbing around the C-ABI (``include/egnn.h``): torch
provides device memory and the current stream, the HIP library does the work.
There is no CPU path: tensors must live on a ROCm device and the library must
be built, otherwise the calls raise.

Reference counterparts
  * the Triton launches ``egnn_forward_kernel_node_parallel[grid](...)``
    (models/EGNN/forward_kernel.py:14-43) and
    ``egnn_backward_kernel_node_parallel[grid](...)`` (backward_kernel.py:14-50)
    -> :func:`egnn_fused_forward` / :func:`egnn_fused_backward`;
  * the reference defines no ``autograd.Function`` for the layer, so
    :class:`EGNNFusedFn` is new; it saves only its inputs and recomputes in the
    backward, like backward_kernel.py:173-180.
"""
from __future__ import annotations

import weakref
from dataclasses import dataclass
from typing import Optional

import torch

from . import _capi
from ._capi import EgnnDims, EgnnStrides, check

__all__ = ["Schedule", "TensorCache", "get_schedule", "egnn_fused_forward", "egnn_fused_backward", "EGNNFusedFn",
           "egnn_fused", "coo_to_csr"]


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _stream(device: torch.device) -> int:
    """The raw handle of the device's current stream (the library's kernels are enqueued on it)."""
    return torch._C._cuda_getCurrentRawStream(device.index if device.index is not None else torch.cuda.current_device())


def _require_device(t: torch.Tensor, name: str) -> None:
    if not t.is_cuda:
        raise RuntimeError(f"{name} must be a ROCm device tensor: the fused EGNN layer has no CPU path")


@dataclass
class Schedule:
    """Per-graph schedule (row ids per edge, split-row list, CSC permutation)."""
    buf: torch.Tensor
    N: int
    E: int


def schedule_arrays(sched: Schedule) -> dict:
    """int32 views of a schedule buffer, in the layout egnn_schedule_build writes:
    erow [E], fix_rows [n_fix], csc_ptr [N+1], csc_eid [E], and the per-32-edge-tile rank tables
    tile_tab [ceil(E/32)][64] (each 256-byte aligned)."""
    N, E = sched.N, sched.E
    ntiles = max((E + 31) // 32, 1)
    off = 0
    out = {}
    for name, n in (("erow", max(E, 1)), ("fix_rows", N), ("n_fix", 1), ("csc_ptr", N + 1), ("csc_eid", max(E, 1)),
                    ("err", 1), ("tile_tab", ntiles * 64)):
        out[name] = sched.buf[off:off + 4 * n].view(torch.int32)
        off = (off + 4 * n + 255) // 256 * 256
    out.pop("err")
    out["tile_tab"] = out["tile_tab"].view(ntiles, 64)[:(E + 31) // 32]
    nf = int(out.pop("n_fix")[0])
    out["fix_rows"] = out["fix_rows"][:nf]
    out["erow"] = out["erow"][:E]
    out["csc_eid"] = out["csc_eid"][:E]
    return out


class TensorCache:
    """Values derived from tensors, kept while those very tensors live unmodified.

    An entry holds weak references to the root tensors (the ``_base`` of a view)
    of its keys plus each key's device, dtype, shape, strides, storage offset and
    in-place version counter.  A lookup hits only when every key's root *is* the
    remembered object: a freed tensor whose memory (same data pointer, version 0)
    is handed to a new tensor of the same size therefore never matches, and a
    tensor edited in place has a new version.  Fresh views of a live tensor (the
    ``row, col = edge_index`` unpacking of a (2, E) tensor) share its root and hit.
    """

    def __init__(self, maxsize: int = 8):
        self.maxsize = maxsize
        self._entries: list = []

    @staticmethod
    def _root(t: torch.Tensor) -> torch.Tensor:
        return t if t._base is None else t._base

    @staticmethod
    def _meta(t: torch.Tensor) -> tuple:
        return (t.device, t.dtype, tuple(t.shape), tuple(t.stride()), t.storage_offset(), t._version)

    def get(self, tensors, extra, make):
        """The value for ``tensors`` (and the hashable ``extra``), computed by ``make()`` on a miss."""
        roots = [self._root(t) for t in tensors]
        meta = (tuple(self._meta(t) for t in tensors), extra)
        live = []
        hit = None
        for refs, m, val in self._entries:
            objs = [r() for r in refs]
            if any(o is None for o in objs):
                continue   # a key tensor died: its memory may belong to another tensor now
            live.append((refs, m, val))
            if hit is None and m == meta and all(o is r for o, r in zip(objs, roots)):
                hit = val
        self._entries = live
        if hit is not None:
            return hit
        val = make()
        self._entries.append(([weakref.ref(r) for r in roots], meta, val))
        del self._entries[:-self.maxsize]
        return val

    def clear(self):
        self._entries = []


_SCHED_CACHE = TensorCache(maxsize=16)


def get_schedule(row_ptrs: torch.Tensor, col_indices: torch.Tensor, num_nodes: int) -> Schedule:
    """Build (or fetch from the cache) the schedule of a dst-sorted int32 CSR graph.

    Cached per (``row_ptrs``, ``col_indices``) tensor pair by :class:`TensorCache`:
    a different or edited graph gets a new schedule.
    """
    _require_device(row_ptrs, "row_ptrs")
    if row_ptrs.dtype != torch.int32 or col_indices.dtype != torch.int32:
        raise TypeError("row_ptrs and col_indices must be int32 (datasets_loaders.py CSR contract)")
    if row_ptrs.numel() != num_nodes + 1:
        raise ValueError(f"row_ptrs has {row_ptrs.numel()} entries, expected num_nodes + 1 = {num_nodes + 1}")
    return _SCHED_CACHE.get((row_ptrs, col_indices), int(num_nodes),
                            lambda: _build_schedule(row_ptrs, col_indices, int(num_nodes)))


def _build_schedule(row_ptrs: torch.Tensor, col_indices: torch.Tensor, N: int) -> Schedule:
    row_ptrs = row_ptrs.contiguous()
    col_indices = col_indices.contiguous()
    E = int(col_indices.numel())
    L = _capi.lib()
    nbytes = L.egnn_schedule_bytes(N, E)
    tbytes = L.egnn_schedule_tmp_bytes(N, E)
    buf = torch.empty(nbytes, dtype=torch.uint8, device=row_ptrs.device)
    tmp = torch.empty(max(tbytes, 1), dtype=torch.uint8, device=row_ptrs.device)
    rc = L.egnn_schedule_build(row_ptrs.data_ptr(), col_indices.data_ptr() if E else None, N, E, buf.data_ptr(),
                               nbytes, tmp.data_ptr(), tbytes, _stream(row_ptrs.device))
    check("egnn_schedule_build", rc)
    return Schedule(buf, N, E)


def coo_to_csr(row: torch.Tensor, col: torch.Tensor, num_nodes: int):
    """COO (row = destination) -> dst-sorted int32 CSR plus the permutation.

    A stable sort by destination keeps the original order of edges within a
    row; ``edge_ids[k]`` is the COO position of CSR edge ``k`` (the indirection
    of forward_kernel.py:19-21 / explanation.txt:113).
    """
    row = row.to(torch.int64)
    order = torch.sort(row, stable=True).indices
    counts = torch.bincount(row, minlength=num_nodes)
    row_ptrs = torch.zeros(num_nodes + 1, dtype=torch.int64, device=row.device)
    row_ptrs[1:] = torch.cumsum(counts, 0)
    return (row_ptrs.to(torch.int32), col.to(torch.int64)[order].to(torch.int32).contiguous(),
            order.to(torch.int32).contiguous())


def _dtype_code(dt: torch.dtype) -> int:
    if dt == torch.float32:
        return _capi.EGNN_F32
    if dt == torch.bfloat16:
        return _capi.EGNN_BF16
    raise TypeError(f"unsupported dtype {dt}: the fused layer runs in float32 or bfloat16")


def _dims(h, edge_feat, col, w1, w2, w1m, equivariant, mean_agg, linear=False) -> EgnnDims:
    """Dimensions of the layer; ``linear``: weights in torch.nn.Linear (out, in) layout."""
    N, F = h.shape
    FE = 0 if edge_feat is None else int(edge_feat.shape[1])
    io = (lambda t: (int(t.shape[1]), int(t.shape[0]))) if linear else (lambda t: (int(t.shape[0]), int(t.shape[1])))  # noqa: E731
    K1, H = io(w1)
    O = io(w2)[1]
    M = io(w1m)[1] if (equivariant and w1m is not None) else O
    g = 1 if equivariant else 0
    if K1 != 2 * F + g + FE:
        raise ValueError(f"w1_msg has {K1} input rows, expected 2*F + {g} + F_E = {2 * F + g + FE}")
    return EgnnDims(N=N, E=int(col.numel()), F=F, FE=FE, H=H, O=O, M=M, equivariant=g,
                    mean_agg=1 if mean_agg else 0, dtype=_dtype_code(h.dtype),
                    weight_layout=_capi.WEIGHTS_LINEAR if linear else _capi.WEIGHTS_PACKED)


def _as(t: Optional[torch.Tensor], dt: torch.dtype) -> Optional[torch.Tensor]:
    """``t`` in dtype ``dt`` with contiguous storage: ``t`` itself (no torch call) when it already is."""
    if t is None:
        return None
    if t.dtype != dt:
        t = t.to(dt)
    return t if t.is_contiguous() else t.contiguous()


def _prep_inputs(h, coord, edge_feat, w1, w2, w1m, w2m, b1, b2, bx1, equivariant):
    _require_device(h, "h")
    dt = h.dtype
    h = h if h.is_contiguous() else h.contiguous()
    w1, w2, w1m, b1, b2, bx1 = _as(w1, dt), _as(w2, dt), _as(w1m, dt), _as(b1, dt), _as(b2, dt), _as(bx1, dt)
    if w2m is not None:
        w2m = _as(w2m.reshape(-1), dt)
    if edge_feat is not None:
        edge_feat = _as(edge_feat, dt)
        if edge_feat.shape[1] == 0:
            edge_feat = None
        elif edge_feat.shape[0] == 0:   # no edges: a fresh empty tensor has unit-stride rows of F_E
            edge_feat = torch.empty((0, edge_feat.shape[1]), dtype=dt, device=edge_feat.device)
    if equivariant:
        coord = _as(coord, torch.float32)
    return h, coord, edge_feat, w1, w2, w1m, w2m, b1, b2, bx1


def egnn_fused_forward(h, coord, edge_feat, row_ptrs, col_indices, edge_ids, w1_msg, w2_msg, w1_mov=None,
                       w2_mov=None, b1=None, b2=None, bx1=None, *, mean_agg: bool = False,
                       equivariant: bool = True, node_proj: Optional[torch.Tensor] = None,
                       linear_weights: bool = False, coord_residual: bool = False, probe_identity: bool = False,
                       out_msg: Optional[torch.Tensor] = None):
    """One fused layer forward.  Returns ``(out_msg (N, O), out_mov (N, 3) or None)``.

    ``out_msg``: when given, an (N, O) tensor of h's dtype on h's device with unit column stride (its rows
    may lie further apart, e.g. a column slice of a wider buffer); the message sums are written into it.

    ``probe_identity`` (EGNN_FLAG_PROBE_IDENTITY): an instrument, not the layer -- the edge kernels
    with the MLP replaced by identity, to time the gather / segment-sum data movement alone.

    ``coord_residual`` (equivariant only, EGNN_FLAG_COORD_RESIDUAL): ``out_mov`` is
    the updated coordinate ``coord + agg_x`` instead of ``agg_x``.

    ``node_proj`` (uint8 device buffer of ``egnn_node_proj_bytes``): when given,
    receives the per-node projections so that a following backward can reuse them.
    ``linear_weights``: w1_msg, w2_msg, w1_mov in torch.nn.Linear (out, in) layout
    instead of the packed (in, out) layout of layer.py:24-28.
    """
    h, coord, edge_feat, w1, w2, w1m, w2m, b1, b2, bx1 = _prep_inputs(
        h, coord, edge_feat, w1_msg, w2_msg, w1_mov, w2_mov, b1, b2, bx1, equivariant)
    return _fused_forward(h, coord, edge_feat, row_ptrs, col_indices, edge_ids, w1, w2, w1m, w2m, b1, b2, bx1,
                          mean_agg=mean_agg, equivariant=equivariant, node_proj=node_proj,
                          linear_weights=linear_weights, coord_residual=coord_residual,
                          probe_identity=probe_identity, out_msg=out_msg)


def _fused_forward(h, coord, edge_feat, row_ptrs, col_indices, edge_ids, w1, w2, w1m, w2m, b1, b2, bx1, *,
                   mean_agg, equivariant, node_proj=None, linear_weights=False, coord_residual=False,
                   probe_identity=False, out_msg=None, dims=None, sched=None):
    """:func:`egnn_fused_forward` on inputs :func:`_prep_inputs` returned; ``dims`` (without flags) and
    ``sched`` when the caller has them."""
    dims = (_dims(h, edge_feat, col_indices, w1, w2, w1m, equivariant, mean_agg, linear_weights) if dims is None
            else EgnnDims.from_buffer_copy(dims))
    if coord_residual and equivariant:
        dims.flags |= _capi.FLAG_COORD_RESIDUAL
    if probe_identity:
        dims.flags |= _capi.FLAG_PROBE_IDENTITY
    if sched is None:
        sched = get_schedule(row_ptrs, col_indices, h.shape[0])
    dev = h.device
    N, O = h.shape[0], dims.O
    if out_msg is None:
        out_msg = torch.empty((N, O), dtype=h.dtype, device=dev)
    elif (tuple(out_msg.shape) != (N, O) or out_msg.dtype != h.dtype or out_msg.device != dev or
          (N > 0 and out_msg.stride(1) != 1)):
        raise ValueError("out_msg must be an (N, O) tensor of h's dtype and device with unit column stride")
    out_mov = torch.empty((N, 3), dtype=torch.float32, device=dev) if equivariant else None
    L = _capi.lib()
    ws_bytes = L.egnn_fwd_workspace_bytes(dims)
    if ws_bytes == 0:
        raise ValueError(f"unsupported dimensions F={dims.F} FE={dims.FE} H={dims.H} O={dims.O} M={dims.M}")
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    strides = EgnnStrides(h=h.stride(0), coord=coord.stride(0) if equivariant else 4,
                          edge=edge_feat.stride(0) if edge_feat is not None else 0, msg=out_msg.stride(0), mov=3)
    eids = _as(edge_ids, torch.int32)
    rc = L.egnn_fwd(dims, strides, _ptr(h), _ptr(coord) if equivariant else None, _ptr(edge_feat),
                    _ptr(_as(row_ptrs, torch.int32)), _ptr(_as(col_indices, torch.int32)), _ptr(eids), _ptr(w1), _ptr(w2),
                    _ptr(w1m) if equivariant else None, _ptr(w2m) if equivariant else None, _ptr(b1), _ptr(b2),
                    _ptr(bx1) if equivariant else None, _ptr(out_msg), _ptr(out_mov), _ptr(node_proj),
                    sched.buf.data_ptr(), ws.data_ptr(), ws_bytes, _stream(dev))
    check("egnn_fwd", rc)
    return out_msg, out_mov


def egnn_fused_backward(h, coord, edge_feat, row_ptrs, col_indices, edge_ids, w1_msg, w2_msg, w1_mov, w2_mov,
                        b1, b2, bx1, grad_out_msg, grad_out_mov, *, mean_agg: bool = False,
                        equivariant: bool = True, node_proj: Optional[torch.Tensor] = None,
                        linear_weights: bool = False, grad_h_into: Optional[torch.Tensor] = None,
                        coord_residual: bool = False, probe_identity: bool = False):
    """Backward by recomputation.  Returns a dict of gradients (None where absent),
    weight gradients in the layout of the weights.

    ``node_proj``: the buffer a forward with the same inputs filled (skips the
    per-node projection GEMM), or None.  ``grad_h_into``: an (N, F) tensor of h's
    dtype with unit column stride; the gradient of h is added to it in place
    (EGNN_FLAG_ACCUMULATE_GRAD_H) and it is returned as the gradient of h.
    ``coord_residual`` (equivariant only, EGNN_FLAG_COORD_RESIDUAL): the coordinate
    output was ``coord + agg_x``, so the returned gradient of coord includes
    ``grad_out_mov`` (the residual path).
    """
    w2m_shape = None if w2_mov is None else tuple(w2_mov.shape)
    h, coord, edge_feat, w1, w2, w1m, w2m, b1, b2, bx1 = _prep_inputs(
        h, coord, edge_feat, w1_msg, w2_msg, w1_mov, w2_mov, b1, b2, bx1, equivariant)
    g = _fused_backward(h, coord, edge_feat, row_ptrs, col_indices, edge_ids, w1, w2, w1m, w2m, b1, b2, bx1,
                        grad_out_msg, grad_out_mov, mean_agg=mean_agg, equivariant=equivariant, node_proj=node_proj,
                        linear_weights=linear_weights, grad_h_into=grad_h_into, coord_residual=coord_residual,
                        probe_identity=probe_identity)
    if g["w2_mov"] is not None and w2m_shape is not None:
        g["w2_mov"] = g["w2_mov"].reshape(w2m_shape)
    return g


def _fused_backward(h, coord, edge_feat, row_ptrs, col_indices, edge_ids, w1, w2, w1m, w2m, b1, b2, bx1,
                    grad_out_msg, grad_out_mov, *, mean_agg, equivariant, node_proj=None, linear_weights=False,
                    grad_h_into=None, coord_residual=False, probe_identity=False, dims=None, sched=None):
    """:func:`egnn_fused_backward` on inputs :func:`_prep_inputs` returned (w2_mov's gradient flat);
    ``dims`` (without flags) and ``sched`` when the caller has them."""
    dims = (_dims(h, edge_feat, col_indices, w1, w2, w1m, equivariant, mean_agg, linear_weights) if dims is None
            else EgnnDims.from_buffer_copy(dims))
    if sched is None:
        sched = get_schedule(row_ptrs, col_indices, h.shape[0])
    dev, dt = h.device, h.dtype
    N = h.shape[0]
    gm = grad_out_msg.to(dt)
    if gm.stride(1) != 1 or (gm.stride(0) * gm.element_size()) % 16 or gm.data_ptr() % 16:
        gm = gm.contiguous()   # the kernels read 8- and 16-byte pieces of unit-stride rows
    gx = _as(grad_out_mov, torch.float32) if equivariant else None
    if grad_h_into is not None:
        gh = grad_h_into
        if (gh.dtype != dt or tuple(gh.shape) != tuple(h.shape) or gh.stride(1) != 1
                or (gh.stride(0) * gh.element_size()) % 16 or gh.data_ptr() % 16):
            raise ValueError("grad_h_into must be an (N, F) tensor of h's dtype with 16-byte aligned unit-stride rows")
        dims.flags |= _capi.FLAG_ACCUMULATE_GRAD_H
        grad_h = gh
    else:
        grad_h = torch.empty_like(h)
    if coord_residual and equivariant:
        dims.flags |= _capi.FLAG_COORD_RESIDUAL
    if probe_identity:   # the identity-MLP instrument (see egnn_fused_forward)
        dims.flags |= _capi.FLAG_PROBE_IDENTITY
    grad_coord = torch.empty((N, 3), dtype=torch.float32, device=dev) if equivariant else None
    g_w1 = torch.empty_like(w1)
    g_w2 = torch.empty_like(w2)
    g_w1m = torch.empty_like(w1m) if equivariant else None
    g_w2m = torch.empty_like(w2m) if equivariant else None
    g_b1 = torch.empty_like(b1) if b1 is not None else None
    g_b2 = torch.empty_like(b2) if b2 is not None else None
    g_bx1 = torch.empty_like(bx1) if (bx1 is not None and equivariant) else None
    L = _capi.lib()
    ws_bytes = L.egnn_bwd_workspace_bytes(dims)
    if ws_bytes == 0:
        raise ValueError(f"unsupported dimensions F={dims.F} FE={dims.FE} H={dims.H} O={dims.O} M={dims.M}")
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    strides = EgnnStrides(h=h.stride(0), coord=3, edge=edge_feat.stride(0) if edge_feat is not None else 0,
                          msg=gm.stride(0), mov=gx.stride(0) if equivariant else 3, grad_h=grad_h.stride(0))
    if equivariant and coord.stride(0) != 3:
        coord = coord[:, :3].contiguous()
    eids = _as(edge_ids, torch.int32)
    rc = L.egnn_bwd(dims, strides, _ptr(h), _ptr(coord) if equivariant else None, _ptr(edge_feat),
                    _ptr(_as(row_ptrs, torch.int32)), _ptr(_as(col_indices, torch.int32)), _ptr(eids), _ptr(w1), _ptr(w2),
                    _ptr(w1m) if equivariant else None, _ptr(w2m) if equivariant else None, _ptr(b1), _ptr(b2),
                    _ptr(bx1) if equivariant else None, _ptr(gm), _ptr(gx), _ptr(grad_h), _ptr(grad_coord),
                    _ptr(g_w1), _ptr(g_w2), _ptr(g_w1m), _ptr(g_w2m), _ptr(g_b1), _ptr(g_b2), _ptr(g_bx1),
                    _ptr(node_proj), sched.buf.data_ptr(), ws.data_ptr(), ws_bytes, _stream(dev))
    check("egnn_bwd", rc)
    return dict(h=grad_h, coord=grad_coord, w1_msg=g_w1, w2_msg=g_w2, w1_mov=g_w1m, w2_mov=g_w2m, b1=g_b1,
                b2=g_b2, bx1=g_bx1)


def _node_proj_buffer(h, edge_feat, col, w1, w2, w1m, equivariant, mean_agg, linear=False, dims=None):
    if dims is None:
        ef = None if (edge_feat is None or edge_feat.shape[1] == 0) else edge_feat
        dims = _dims(h, ef, col, w1, w2, w1m, equivariant, mean_agg, linear)
    n = _capi.lib().egnn_node_proj_bytes(dims)
    return torch.empty(max(n, 16), dtype=torch.uint8, device=h.device)


class EGNNFusedFn(torch.autograd.Function):
    """Autograd wrapper: ``(out_msg, out_mov) = EGNNFusedFn.apply(h, coord, edge_feat, row_ptrs,
    col_indices, edge_ids, w1_msg, w2_msg, w1_mov, w2_mov, b1, b2, bx1, mean_agg, equivariant)``.

    Saves only the inputs; the backward recomputes the messages.  No gradient
    flows to ``edge_feat`` or the CSR (the reference computes none).
    """

    @staticmethod
    def forward(ctx, h, coord, edge_feat, row_ptrs, col_indices, edge_ids, w1_msg, w2_msg, w1_mov, w2_mov,
                b1=None, b2=None, bx1=None, mean_agg=False, equivariant=True, linear_weights=False):
        # dtype/layout conversion once; the backward reuses the converted tensors
        ctx.shapes = [None if t is None else tuple(t.shape) for t in (w1_msg, w2_msg, w1_mov, w2_mov, b1, b2, bx1)]
        h, coord_p, edge_feat, w1_msg, w2_msg, w1_mov, w2_mov, b1, b2, bx1 = _prep_inputs(
            h, coord, edge_feat, w1_msg, w2_msg, w1_mov, w2_mov, b1, b2, bx1, equivariant)
        pq = _node_proj_buffer(h, edge_feat, col_indices, w1_msg, w2_msg, w1_mov, equivariant, mean_agg,
                               linear_weights)
        out_msg, out_mov = egnn_fused_forward(h, coord_p, edge_feat, row_ptrs, col_indices, edge_ids, w1_msg,
                                              w2_msg, w1_mov, w2_mov, b1, b2, bx1, mean_agg=mean_agg,
                                              equivariant=equivariant, node_proj=pq, linear_weights=linear_weights)
        ctx.save_for_backward(h, coord_p, edge_feat, row_ptrs, col_indices, edge_ids, w1_msg, w2_msg, w1_mov,
                              w2_mov, b1, b2, bx1, pq)
        ctx.mean_agg = mean_agg
        ctx.equivariant = equivariant
        ctx.linear_weights = linear_weights
        ctx.coord_shape = None if coord is None else tuple(coord.shape)
        ctx.coord_dtype = None if coord is None else coord.dtype
        if out_mov is None:
            out_mov = torch.zeros((h.shape[0], 3), dtype=torch.float32, device=h.device)
        return out_msg, out_mov

    @staticmethod
    def backward(ctx, g_msg, g_mov):
        (h, coord, edge_feat, row_ptrs, col_indices, edge_ids, w1, w2, w1m, w2m, b1, b2, bx1, pq) = ctx.saved_tensors
        if g_msg is None:
            O = w2.shape[0] if ctx.linear_weights else w2.shape[1]
            g_msg = torch.zeros((h.shape[0], O), dtype=h.dtype, device=h.device)
        if g_mov is None:
            g_mov = torch.zeros((h.shape[0], 3), dtype=torch.float32, device=h.device)
        g = egnn_fused_backward(h, coord, edge_feat, row_ptrs, col_indices, edge_ids, w1, w2, w1m, w2m, b1, b2,
                                bx1, g_msg, g_mov, mean_agg=ctx.mean_agg, equivariant=ctx.equivariant,
                                node_proj=pq, linear_weights=ctx.linear_weights)
        gc = g["coord"]
        if gc is not None and ctx.coord_shape is not None and ctx.coord_shape[1] != 3:
            full = torch.zeros(ctx.coord_shape, dtype=torch.float32, device=gc.device)
            full[:, :3] = gc
            gc = full
        if gc is not None and ctx.coord_dtype is not None:
            gc = gc.to(ctx.coord_dtype)
        wg = [g[k] for k in ("w1_msg", "w2_msg", "w1_mov", "w2_mov", "b1", "b2", "bx1")]
        wg = [None if (t is None or shp is None) else t.reshape(shp) for t, shp in zip(wg, ctx.shapes)]
        return (g["h"], gc, None, None, None, None, *wg, None, None, None)


def egnn_fused(h, coord, edge_feat, row_ptrs, col_indices, edge_ids, w1_msg, w2_msg, w1_mov=None, w2_mov=None,
               b1=None, b2=None, bx1=None, *, mean_agg=False, equivariant=True, linear_weights=False):
    """Differentiable fused layer (see :class:`EGNNFusedFn`).

    ``linear_weights``: w1_msg (H, 2F+g+F_E), w2_msg (O, H), w1_mov (M, O) as
    torch.nn.Linear stores them, used in place (no transposed copies) and with
    gradients in the same layout; else the packed (in, out) layout.
    Edge-feature widths that are not a multiple of 8 are zero-padded (with
    matching zero W_e entries) outside the Function, so gradients stay exact.
    """
    if edge_feat is not None and edge_feat.shape[1] % 8:
        pad = 8 - edge_feat.shape[1] % 8
        edge_feat = torch.nn.functional.pad(edge_feat, (0, pad))
        if linear_weights:
            w1_msg = torch.cat([w1_msg, w1_msg.new_zeros((w1_msg.shape[0], pad))], dim=1)
        else:
            w1_msg = torch.cat([w1_msg, w1_msg.new_zeros((pad, w1_msg.shape[1]))], dim=0)
    return EGNNFusedFn.apply(h, coord, edge_feat, row_ptrs, col_indices, edge_ids, w1_msg, w2_msg, w1_mov, w2_mov,
                             b1, b2, bx1, mean_agg, equivariant, linear_weights)
