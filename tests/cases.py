"""Seeded inputs for the parity tests (numpy on the CPU, then moved to the device)."""
from __future__ import annotations

import numpy as np

from oracle import egnn_oracle as orc
from pymolecular_amd import graphs


def rng(seed):
    return np.random.Generator(np.random.PCG64(seed))


def random_csr(N, degs, seed, self_loops=True):
    """CSR with the given in-degrees and uniform sources (duplicates allowed)."""
    r = rng(seed)
    degs = np.asarray(degs, dtype=np.int64)
    rowptr = np.zeros(N + 1, dtype=np.int64)
    np.cumsum(degs, out=rowptr[1:])
    E = int(rowptr[-1])
    col = r.integers(0, N, size=E)
    rows = np.repeat(np.arange(N), degs)
    if not self_loops:
        bad = col == rows
        col[bad] = (col[bad] + 1) % N
    return rowptr.astype(np.int32), col.astype(np.int32)


def make_params(r, F, FE, H, O, M, eq=True, bias=True, scale=1.0):
    g = 1 if eq else 0
    p = dict(
        w1_msg=graphs.xavier_uniform(r, 2 * F + g + FE, H) * scale,
        w2_msg=graphs.xavier_uniform(r, H, O) * scale,
    )
    if eq:
        p["w1_mov"] = graphs.xavier_uniform(r, O, M) * scale
        p["w2_mov"] = (r.uniform(-1, 1, size=M) * np.sqrt(6.0 / (M + 1))).astype(np.float32)
    if bias:
        p["b1"] = (r.standard_normal(H) * 0.1).astype(np.float32)
        p["b2"] = (r.standard_normal(O) * 0.1).astype(np.float32)
        if eq:
            p["bx1"] = (r.standard_normal(M) * 0.1).astype(np.float32)
    return p


class Case:
    """Inputs of one fused-layer call, in numpy (float32) plus bf16-rounded float64 views."""

    def __init__(self, rowptr, col, F, FE, H, O, M, *, eq=True, bias=True, seed=0, edge_ids=None, coord_scale=1.5,
                 mean_agg=False):
        r = rng(seed)
        self.rowptr, self.col = np.asarray(rowptr, np.int32), np.asarray(col, np.int32)
        self.N, self.E = len(rowptr) - 1, len(col)
        self.F, self.FE, self.H, self.O, self.M, self.eq, self.mean = F, FE, H, O, M, eq, mean_agg
        self.h = r.standard_normal((self.N, F)).astype(np.float32)
        self.coord = (r.standard_normal((self.N, 3)) * coord_scale).astype(np.float32) if eq else None
        self.ef = r.standard_normal((self.E, FE)).astype(np.float32) if FE > 0 else None
        self.edge_ids = None if edge_ids is None else np.asarray(edge_ids, np.int32)
        self.p = make_params(r, F, FE, H, O, M, eq=eq, bias=bias)
        self.gm = r.standard_normal((self.N, O)).astype(np.float32)
        self.gx = r.standard_normal((self.N, 3)).astype(np.float32) if eq else None

    def oracle_inputs(self, bf16):
        rd = orc.round_bf16 if bf16 else (lambda a: np.asarray(a, np.float64))
        h = rd(self.h)
        ef = None if self.ef is None else rd(self.ef)
        p = {k: rd(v) for k, v in self.p.items()}
        gm = rd(self.gm)
        return h, ef, p, gm

    def forward_ref(self, bf16):
        h, ef, p, _ = self.oracle_inputs(bf16)
        return orc.fused_forward(h, self.coord, ef, self.rowptr, self.col, self.edge_ids, p, mean_agg=self.mean,
                                 equivariant=self.eq)

    def backward_ref(self, bf16):
        h, ef, p, gm = self.oracle_inputs(bf16)
        return orc.fused_backward(h, self.coord, ef, self.rowptr, self.col, self.edge_ids, p, gm, self.gx,
                                  mean_agg=self.mean, equivariant=self.eq)
