"""The C-ABI library loads and exports every symbol include/egnn.h declares (no GPU needed)."""
import ctypes
import re
from pathlib import Path

import pytest

from pymolecular_amd import _capi

HEADER = Path(__file__).resolve().parents[1] / "include" / "egnn.h"


def declared_symbols():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(egnn_\w+)\s*\(", text)))


def test_header_and_binding_agree():
    assert declared_symbols() == sorted(_capi.EXPORTED)


def test_library_exports_every_declared_symbol():
    L = _capi.lib()
    for name in declared_symbols():
        assert hasattr(L, name), name
        assert ctypes.cast(getattr(L, name), ctypes.c_void_p).value


def test_host_only_entry_points():
    L = _capi.lib()
    assert L.egnn_abi_version() == _capi.ABI_VERSION
    assert _capi.status_string(0) == "ok"
    assert "CSR" in _capi.status_string(6)
    assert L.egnn_schedule_bytes(100, 1000) > 4 * 1000
    d = _capi.EgnnDims(N=100, E=1000, F=128, FE=16, H=128, O=128, M=128, equivariant=1, mean_agg=0, dtype=1)
    assert L.egnn_fwd_workspace_bytes(d) > 0
    assert L.egnn_bwd_workspace_bytes(d) > L.egnn_fwd_workspace_bytes(d)


@pytest.mark.parametrize("field,value", [("H", 96), ("FE", 12), ("F", 24), ("dtype", 7), ("O", 64)])
def test_unsupported_dims_rejected(field, value):
    L = _capi.lib()
    kw = dict(N=100, E=1000, F=128, FE=16, H=128, O=128, M=128, equivariant=1, mean_agg=0, dtype=0)
    kw[field] = value
    assert L.egnn_fwd_workspace_bytes(_capi.EgnnDims(**kw)) == 0


def test_bad_arguments_return_status_not_crash():
    L = _capi.lib()
    d = _capi.EgnnDims(N=10, E=20, F=128, FE=0, H=128, O=128, M=128, equivariant=1, mean_agg=0, dtype=0)
    s = _capi.EgnnStrides(h=128, coord=3, edge=0, msg=128, mov=3)
    # NULL inputs are reported before anything touches the device
    rc = L.egnn_fwd(d, s, *([None] * 18), 0, None)
    assert rc == 1
    s_bad = _capi.EgnnStrides(h=16, coord=3, edge=0, msg=128, mov=3)
    assert L.egnn_fwd(d, s_bad, *([None] * 18), 0, None) == 3
    assert L.egnn_schedule_build(None, None, 10, 20, None, 0, None, 0, None) == 1
    assert L.egnn_schedule_build(1, 1, 0, 20, 1, 0, 1, 0, None) == 2


def test_node_activation_buffer_requirement():
    # act may be NULL exactly where both node-update passes stream the rows: bf16, K1 = Hn = Fo = 128,
    # K2 in {0, 128}, at least 65,536 rows; invalid dims return minus their status code
    L = _capi.lib()
    nd = lambda **kw: _capi.EgnnNodeDims(**{**dict(N=65536, K1=128, K2=128, Hn=128, Fo=128, residual=1,  # noqa: E731
                                                    dtype=_capi.EGNN_BF16), **kw})
    assert L.egnn_node_act_required(nd()) == 0
    assert L.egnn_node_act_required(nd(K2=0, residual=0, N=1 << 21)) == 0
    assert L.egnn_node_act_required(nd(N=65535)) == 1
    assert L.egnn_node_act_required(nd(dtype=_capi.EGNN_F32)) == 1
    assert L.egnn_node_act_required(nd(Hn=64)) == 1
    assert L.egnn_node_act_required(nd(K2=136)) == 1
    assert L.egnn_node_act_required(nd(K1=12)) == -_capi.EGNN_ERR_DIMS


def test_flags_validated():
    L = _capi.lib()
    kw = dict(N=100, E=1000, F=128, FE=16, H=128, O=128, M=128, equivariant=1, mean_agg=0, dtype=1)
    for flags in (0, _capi.FLAG_ACCUMULATE_GRAD_H, _capi.FLAG_COORD_RESIDUAL,
                  _capi.FLAG_ACCUMULATE_GRAD_H | _capi.FLAG_COORD_RESIDUAL):
        assert L.egnn_bwd_workspace_bytes(_capi.EgnnDims(**kw, flags=flags)) > 0, flags
    assert L.egnn_fwd_workspace_bytes(_capi.EgnnDims(**kw, flags=4)) == 0          # unknown flag
    kw["equivariant"] = 0                                                            # no coordinates in the MPNN layer
    assert L.egnn_fwd_workspace_bytes(_capi.EgnnDims(**kw, flags=_capi.FLAG_COORD_RESIDUAL)) == 0
    assert L.egnn_fwd_workspace_bytes(_capi.EgnnDims(**kw, flags=_capi.FLAG_ACCUMULATE_GRAD_H)) > 0


def test_graph_builder_arguments_checked_on_the_host():
    # every check below returns before the library touches the device
    L = _capi.lib()
    assert L.egnn_graph_tmp_bytes(0) == 0 and L.egnn_graph_tmp_bytes(1000) > 4000
    ne = ctypes.c_int64(0)
    buf = 1 << 12   # a non-NULL stand-in address, never dereferenced by these calls
    call = lambda k, cap, tmpb, pos=buf: L.egnn_knn_graph(pos, 100, buf, 2, 64, k, buf, buf, cap, buf, tmpb,  # noqa: E731
                                                           ctypes.byref(ne), None)
    big = L.egnn_graph_tmp_bytes(100)
    assert call(8, 800, big, pos=None) == 1        # NULL positions
    assert call(65, 6500, big) == 2                 # k above 64
    assert call(0, 800, big) == 2                   # k below 1
    assert call(8, 799, big) == 5                   # col capacity below N * k
    assert call(8, 800, 16) == 5                    # short tmp
    assert call(8, 800, big, pos=buf + 4) == 4      # positions not 8-byte aligned
    assert L.egnn_radius_graph(buf, 100, buf, 2, 64, ctypes.c_double(-1.0), 8, buf, buf, 800, buf, big,
                               ctypes.byref(ne), None) == 2   # negative cutoff
    assert L.egnn_knn_graph(buf, 100, buf, 2, 4096, 8, buf, buf, 800, buf, big, ctypes.byref(ne), None) == 2


def test_static_forward_rejects_graphs_beyond_its_scratch():
    # the size check comes before any device access: a 2M-node layer needs 1 GB of node projections
    L = _capi.lib()
    d = _capi.EgnnDims(N=2_000_000, E=18_000_000, F=128, FE=16, H=128, O=128, M=128, equivariant=0, mean_agg=0,
                       dtype=1)
    assert L.egnn_fwd_workspace_bytes(d) > _capi.FWD_STATIC_SCRATCH_BYTES
    s = _capi.EgnnStrides(h=128, coord=4, edge=16, msg=128, mov=3)
    assert L.egnn_fwd_static(d, s, *([None] * 18)) == _capi.EGNN_ERR_SCRATCH
    assert "scratch" in _capi.status_string(_capi.EGNN_ERR_SCRATCH)
    bad = _capi.EgnnDims(N=10, E=20, F=128, FE=0, H=96, O=96, M=96, equivariant=1, mean_agg=0, dtype=1)
    assert L.egnn_fwd_static(bad, s, *([None] * 18)) == 2


def test_identity_probe_flag_only_for_bf16_mpnn_h128():
    L = _capi.lib()
    kw = dict(N=100, E=1000, F=128, FE=16, H=128, O=128, M=128, equivariant=0, mean_agg=0, dtype=1,
              flags=_capi.FLAG_PROBE_IDENTITY)
    assert L.egnn_fwd_workspace_bytes(_capi.EgnnDims(**kw)) > 0
    for field, value in (("equivariant", 1), ("dtype", 0), ("H", 256)):
        bad = dict(kw, **{field: value})
        if field == "H":
            bad.update(O=256, M=256)
        assert L.egnn_fwd_workspace_bytes(_capi.EgnnDims(**bad)) == 0, field
    # beyond the edge-parallel kernels' 32-bit node-projection offsets (N * 4H >= 2^32) the layer runs other
    # kernels; the instrument is refused rather than silently timing the real layer
    big = dict(kw, N=1 << 23)
    assert L.egnn_fwd_workspace_bytes(_capi.EgnnDims(**big)) == 0
    assert L.egnn_bwd_workspace_bytes(_capi.EgnnDims(**big)) == 0
    assert L.egnn_fwd_workspace_bytes(_capi.EgnnDims(**dict(big, flags=0))) > 0


def test_fp32_backward_scratch_is_bounded():
    # the fp32 backward keeps its per-edge rows (factors, dL/dpre1, dL/ddelta, r^2) one edge chunk at a
    # time: its workspace grows with the nodes, not with the edges, past the chunk budget
    L = _capi.lib()
    kw = dict(F=32, FE=16, H=64, O=32, M=32, equivariant=1, mean_agg=0, dtype=0)
    small = L.egnn_bwd_workspace_bytes(_capi.EgnnDims(N=250_000, E=8_000_000, **kw))
    big = L.egnn_bwd_workspace_bytes(_capi.EgnnDims(N=250_000, E=32_000_000, **kw))
    assert big - small < 32 << 20, (small >> 20, big >> 20)          # 4x the edges, about the same scratch
    assert small < (256 << 20) + 2 * 250_000 * 2 * 64 * 4 + (32 << 20), small >> 20   # chunk + node rows
    # graphs of 8,192 edges or more take at least two chunks: the scratch is about half the per-edge state
    one = L.egnn_bwd_workspace_bytes(_capi.EgnnDims(N=1000, E=8000, **kw))
    two = L.egnn_bwd_workspace_bytes(_capi.EgnnDims(N=1000, E=32_000, **kw))
    per_edge = (64 + 2 * 32 + 2 * 32) * 4 + 64 * 4 + 16 + 4
    assert two < 0.6 * 32_000 * per_edge + one, (one, two)
