"""ctypes binding of the C-ABI in ``include/egnn.h`` (``libpymolecular_egnn.so``).

The library is built in-tree by ``pymolecular_amd._build`` (``__graft_entry__.build``).
There is no fallback: if the library is missing every entry point raises.
"""
from __future__ import annotations

import ctypes
from ctypes import c_int32, c_int64, c_size_t, c_void_p, c_char_p
from pathlib import Path

LIB_PATH = Path(__file__).resolve().with_name("libpymolecular_egnn.so")

EGNN_OK = 0
EGNN_ERR_NULL = 1
EGNN_ERR_DIMS = 2
EGNN_ERR_SCRATCH = 8
FWD_STATIC_SCRATCH_BYTES = 128 << 20   # include/egnn.h EGNN_FWD_STATIC_SCRATCH_BYTES
EGNN_F32 = 0
EGNN_BF16 = 1

# every symbol include/egnn.h declares
EXPORTED = (
    "egnn_abi_version", "egnn_status_string", "egnn_schedule_bytes", "egnn_schedule_tmp_bytes",
    "egnn_schedule_build", "egnn_fwd_workspace_bytes", "egnn_bwd_workspace_bytes", "egnn_node_proj_bytes",
    "egnn_fwd", "egnn_fwd_static", "egnn_bwd",
    "egnn_node_bwd_workspace_bytes", "egnn_node_act_required", "egnn_node_fwd", "egnn_node_bwd",
    "egnn_dense_fwd", "egnn_dense_dgrad", "egnn_dense_wgrad_workspace_bytes", "egnn_dense_wgrad",
    "egnn_profile_enable", "egnn_profile_read",
    "egnn_graph_tmp_bytes", "egnn_knn_graph", "egnn_radius_graph",
)

# kernel classes of the instrumentation hook
(K_FWD_EDGE, K_FWD_FIXUP, K_BWD_EDGE, K_NODE_GEMM, K_WGRAD, K_NODE_REDUCE, K_PREP, K_NODE_UPDATE,
 K_EDGE_WGRAD) = range(9)
K_NAMES = ("fwd_edge", "fwd_fixup", "bwd_edge", "node_gemm", "wgrad", "node_reduce", "prep", "node_update",
           "edge_wgrad")


WEIGHTS_PACKED, WEIGHTS_LINEAR = 0, 1   # include/egnn.h EGNN_WEIGHTS_*
FLAG_ACCUMULATE_GRAD_H = 1              # include/egnn.h EGNN_FLAG_ACCUMULATE_GRAD_H
FLAG_COORD_RESIDUAL = 2                 # include/egnn.h EGNN_FLAG_COORD_RESIDUAL
FLAG_PROBE_IDENTITY = 4                 # include/egnn.h EGNN_FLAG_PROBE_IDENTITY (instrument only)


class EgnnDims(ctypes.Structure):
    _fields_ = [("N", c_int64), ("E", c_int64), ("F", c_int32), ("FE", c_int32), ("H", c_int32),
                ("O", c_int32), ("M", c_int32), ("equivariant", c_int32), ("mean_agg", c_int32),
                ("dtype", c_int32), ("weight_layout", c_int32), ("flags", c_int32)]


class EgnnStrides(ctypes.Structure):
    _fields_ = [("h", c_int64), ("coord", c_int64), ("edge", c_int64), ("msg", c_int64), ("mov", c_int64),
                ("grad_h", c_int64)]


class EgnnNodeDims(ctypes.Structure):
    _fields_ = [("N", c_int64), ("K1", c_int32), ("K2", c_int32), ("Hn", c_int32), ("Fo", c_int32),
                ("residual", c_int32), ("dtype", c_int32)]


_lib = None

ABI_VERSION = 9   # include/egnn.h egnn_abi_version()


def _check_stamp() -> None:
    """Refuse a library that was not built from the sources in this tree.

    The build writes the SHA-256 of its sources next to the library; a missing
    or different stamp means the library is stale (or foreign)."""
    from . import _build
    stamp = _build.STAMP
    if not stamp.exists():
        raise RuntimeError(f"{stamp} is missing: rebuild the library with `python -m pymolecular_amd._build`")
    built = stamp.read_text().strip()
    now = _build.source_hash()
    if built != now:
        raise RuntimeError(f"{LIB_PATH} was built from other sources (sha256 {built[:16]}, tree {now[:16]}): "
                           "rebuild it with `python -m pymolecular_amd._build`")


class EgnnError(RuntimeError):
    """A C-ABI call returned a non-zero status."""

    def __init__(self, fn: str, status: int):
        self.status = status
        super().__init__(f"{fn} failed with status {status}: {status_string(status)}")


def lib() -> ctypes.CDLL:
    """Load the HIP library once; raise if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise RuntimeError(f"{LIB_PATH} is missing: build it with `python -m pymolecular_amd._build` "
                           "(or __graft_entry__.build()); there is no CPU fallback")
    _check_stamp()
    L = ctypes.CDLL(str(LIB_PATH))
    P = c_void_p
    L.egnn_abi_version.restype = c_int32
    L.egnn_abi_version.argtypes = []
    if L.egnn_abi_version() != ABI_VERSION:
        raise RuntimeError(f"{LIB_PATH} implements ABI {L.egnn_abi_version()}, these bindings expect {ABI_VERSION}: "
                           "rebuild it with `python -m pymolecular_amd._build`")
    L.egnn_status_string.restype = c_char_p
    L.egnn_status_string.argtypes = [c_int32]
    L.egnn_schedule_bytes.restype = c_size_t
    L.egnn_schedule_bytes.argtypes = [c_int64, c_int64]
    L.egnn_schedule_tmp_bytes.restype = c_size_t
    L.egnn_schedule_tmp_bytes.argtypes = [c_int64, c_int64]
    L.egnn_schedule_build.restype = c_int32
    L.egnn_schedule_build.argtypes = [P, P, c_int64, c_int64, P, c_size_t, P, c_size_t, P]
    L.egnn_fwd_workspace_bytes.restype = c_size_t
    L.egnn_fwd_workspace_bytes.argtypes = [ctypes.POINTER(EgnnDims)]
    L.egnn_bwd_workspace_bytes.restype = c_size_t
    L.egnn_bwd_workspace_bytes.argtypes = [ctypes.POINTER(EgnnDims)]
    L.egnn_node_proj_bytes.restype = c_size_t
    L.egnn_node_proj_bytes.argtypes = [ctypes.POINTER(EgnnDims)]
    L.egnn_fwd.restype = c_int32
    L.egnn_fwd.argtypes = [ctypes.POINTER(EgnnDims), ctypes.POINTER(EgnnStrides)] + [P] * 18 + [c_size_t, P]
    L.egnn_fwd_static.restype = c_int32
    L.egnn_fwd_static.argtypes = [ctypes.POINTER(EgnnDims), ctypes.POINTER(EgnnStrides)] + [P] * 18
    L.egnn_bwd.restype = c_int32
    L.egnn_bwd.argtypes = [ctypes.POINTER(EgnnDims), ctypes.POINTER(EgnnStrides)] + [P] * 27 + [c_size_t, P]
    ND = ctypes.POINTER(EgnnNodeDims)
    L.egnn_node_bwd_workspace_bytes.restype = c_size_t
    L.egnn_node_bwd_workspace_bytes.argtypes = [ND]
    L.egnn_node_act_required.restype = c_int32
    L.egnn_node_act_required.argtypes = [ND]
    L.egnn_node_fwd.restype = c_int32
    L.egnn_node_fwd.argtypes = [ND, P, c_int64, P, c_int64, P, P, P, P, P, P, P, c_int64, P]
    L.egnn_node_bwd.restype = c_int32
    L.egnn_node_bwd.argtypes = [ND, P, c_int64, P, c_int64, P, P, P, P, P, c_int64, P, P, P, P, P, P, c_size_t, P]
    L.egnn_dense_fwd.restype = c_int32
    L.egnn_dense_fwd.argtypes = [c_int32, c_int64, c_int32, c_int32, P, c_int64, P, P, P, c_int64, P]
    L.egnn_dense_dgrad.restype = c_int32
    L.egnn_dense_dgrad.argtypes = [c_int32, c_int64, c_int32, c_int32, P, c_int64, P, P, c_int64, P]
    L.egnn_dense_wgrad_workspace_bytes.restype = c_size_t
    L.egnn_dense_wgrad_workspace_bytes.argtypes = [c_int64, c_int32, c_int32]
    L.egnn_dense_wgrad.restype = c_int32
    L.egnn_dense_wgrad.argtypes = [c_int32, c_int64, c_int32, c_int32, P, c_int64, P, c_int64, P, P, P, c_size_t, P]
    L.egnn_graph_tmp_bytes.restype = c_size_t
    L.egnn_graph_tmp_bytes.argtypes = [c_int64]
    L.egnn_knn_graph.restype = c_int32
    L.egnn_knn_graph.argtypes = [P, c_int64, P, c_int32, c_int32, c_int32, P, P, c_int64, P, c_size_t,
                                 ctypes.POINTER(c_int64), P]
    L.egnn_radius_graph.restype = c_int32
    L.egnn_radius_graph.argtypes = [P, c_int64, P, c_int32, c_int32, ctypes.c_double, c_int32, P, P, c_int64, P,
                                    c_size_t, ctypes.POINTER(c_int64), P]
    L.egnn_profile_enable.restype = c_int32
    L.egnn_profile_enable.argtypes = [c_int32]
    L.egnn_profile_read.restype = c_int32
    L.egnn_profile_read.argtypes = [c_int32, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(c_int64)]
    _lib = L
    return L


PROFILE_ALL = 0xFF   # include/egnn.h EGNN_PROFILE_ALL


def profile_enable(on: bool, classes=None) -> None:
    """Record the launches of every kernel class (or of ``classes``, a list of K_* values); clears
    earlier records.  ``on=False`` stops recording."""
    mask = 0 if not on else (PROFILE_ALL if classes is None else sum(1 << k for k in classes))
    check("egnn_profile_enable", lib().egnn_profile_enable(mask))


def profile_read() -> dict:
    """{kernel class name: (total ms, launches)} of the records since profile_enable(True)."""
    out = {}
    for k, name in enumerate(K_NAMES):
        t, n = ctypes.c_double(0.0), c_int64(0)
        check("egnn_profile_read", lib().egnn_profile_read(k, ctypes.byref(t), ctypes.byref(n)))
        out[name] = (t.value, n.value)
    return out


def status_string(status: int) -> str:
    try:
        return lib().egnn_status_string(int(status)).decode()
    except Exception:  # pragma: no cover - only when the library itself is unusable
        return "unknown"


def check(fn: str, status: int) -> None:
    if status != EGNN_OK:
        raise EgnnError(fn, status)
