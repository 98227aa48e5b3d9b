"""Seeded synthetic graphs for the five workloads of the fused EGNN/MPNN layer.

All generation runs on the CPU with numpy's PCG64, so the bytes are the same
on every machine; the arrays are moved to the device afterwards.  Every graph
is returned in the dst-sorted int32 CSR contract of datasets_loaders.py:7-11
(``row_ptrs`` (N+1), ``col_indices`` (E) = source of each edge, rows are the
receiving node), with source ids ascending inside each row -- the order of
egnn_clean.py:167-173 (``get_edges``: i outer, j inner).

Workloads (seeds: graph 1000+k, features 2000+k, weights 3000+k):
  1 molecules   128 graphs, atoms ~ U{9..29}, fully connected, no self loops,
                coords N(0, 1.5^2) per axis, one-hot(5) atom types, F_E = 0
  2 molecules   the same generator with 1024 graphs
  3 proteins    64 chains x 512 residues, 3.8 A random-walk steps with a 3 A
                self-avoidance radius, kNN k = 30 inside a chain (ties by
                index), one-hot(20), 16 Gaussian RBFs on [0, 15] A
  4 slabs       256 systems x 80 atoms, uniform in a cube at 0.08 atoms/A^3
                (side 10 A), radius graph 6 A capped at the 50 nearest,
                one-hot(50), 32 RBFs on [0, 6] A
  5 power law   one graph, N = 2,000,000, in-degree ~ d^-2.1 on [2, 4096]
                (inverse CDF), uniform sources (self loops resampled),
                h ~ N(0, 1) (N, 128), e ~ N(0, 1) (E, 16), MPNN (no geometry)
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Optional

import numpy as np

__all__ = ["Graph", "molecule_batch", "protein_chains", "catalyst_slabs", "powerlaw_graph", "rbf",
           "protein_positions", "knn_rows", "slab_positions", "radius_rows",
           "csr_from_rows", "WORKLOADS", "make_workload", "xavier_uniform"]


def _rng(seed: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(seed))


@dataclass
class Graph:
    """A CSR graph plus the node/edge inputs of one workload."""
    rowptr: np.ndarray            # int32 (N+1)
    col: np.ndarray               # int32 (E)
    coord: Optional[np.ndarray]   # float32 (N, 3) or None (MPNN)
    node_feat: np.ndarray         # float32 (N, in_nf): one-hot types or dense features
    edge_attr: Optional[np.ndarray]  # float32 (E, F_E) or None
    info: dict = field(default_factory=dict)

    @property
    def N(self) -> int:
        return int(self.rowptr.shape[0] - 1)

    @property
    def E(self) -> int:
        return int(self.col.shape[0])

    def rows(self) -> np.ndarray:
        return np.repeat(np.arange(self.N, dtype=np.int64), np.diff(self.rowptr)).astype(np.int32)


def csr_from_rows(rows: np.ndarray, cols: np.ndarray, N: int):
    """COO -> dst-sorted CSR (stable in the given order).  Returns (rowptr, col, perm)."""
    rows = np.asarray(rows, dtype=np.int64)
    perm = np.argsort(rows, kind="stable")
    counts = np.bincount(rows, minlength=N)
    rowptr = np.zeros(N + 1, dtype=np.int64)
    np.cumsum(counts, out=rowptr[1:])
    return rowptr.astype(np.int32), np.asarray(cols, dtype=np.int64)[perm].astype(np.int32), perm.astype(np.int64)


def rbf(d: np.ndarray, n: int, dmax: float) -> np.ndarray:
    """Gaussian radial basis exp(-(d - mu_k)^2 / (2 sigma^2)), mu = linspace(0, dmax, n), sigma = spacing."""
    mu = np.linspace(0.0, dmax, n)
    sigma = mu[1] - mu[0]
    return np.exp(-((d[:, None] - mu[None, :]) ** 2) / (2.0 * sigma * sigma)).astype(np.float32)


def _one_hot(types: np.ndarray, k: int) -> np.ndarray:
    out = np.zeros((types.shape[0], k), dtype=np.float32)
    out[np.arange(types.shape[0]), types] = 1.0
    return out


def molecule_batch(n_graphs: int, seed: int = 1001, feat_seed: int = 2001, lo: int = 9, hi: int = 29,
                   sigma: float = 1.5, n_types: int = 5) -> Graph:
    """Fully connected molecules without self loops (egnn_clean.py:167-191 edge order)."""
    r = _rng(seed)
    sizes = r.integers(lo, hi + 1, size=n_graphs)
    offs = np.zeros(n_graphs + 1, dtype=np.int64)
    np.cumsum(sizes, out=offs[1:])
    N = int(offs[-1])
    local = {}
    for n in np.unique(sizes):
        i, j = np.meshgrid(np.arange(n), np.arange(n), indexing="ij")
        mask = i != j
        local[int(n)] = (i[mask], j[mask])
    rows = np.concatenate([local[int(n)][0] + o for n, o in zip(sizes, offs[:-1])])
    cols = np.concatenate([local[int(n)][1] + o for n, o in zip(sizes, offs[:-1])])
    coord = (r.standard_normal((N, 3)) * sigma).astype(np.float32)
    types = _rng(feat_seed).integers(0, n_types, size=N)
    rowptr, col, _ = csr_from_rows(rows, cols, N)
    return Graph(rowptr, col, coord, _one_hot(types, n_types), None,
                 dict(name="molecules", n_graphs=n_graphs, graph_offsets=offs))


def protein_positions(n_chains: int = 64, n_res: int = 512, seed: int = 1003, step: float = 3.8,
                      min_dist: float = 3.0, max_tries: int = 200) -> np.ndarray:
    """Self-avoiding 3-D random-walk chains, float64 (n_chains, n_res, 3)."""
    r = _rng(seed)
    X = np.zeros((n_chains, n_res, 3))
    for t in range(1, n_res):
        need = np.ones(n_chains, dtype=bool)
        prop = np.zeros((n_chains, 3))
        for _ in range(max_tries):
            idx = np.flatnonzero(need)
            if idx.size == 0:
                break
            v = r.standard_normal((idx.size, 3))
            v /= np.linalg.norm(v, axis=1, keepdims=True)
            cand = X[idx, t - 1] + step * v
            d2 = ((X[idx, :t] - cand[:, None, :]) ** 2).sum(-1)
            ok = d2.min(axis=1) >= min_dist * min_dist
            prop[idx[ok]] = cand[ok]
            prop[idx[~ok]] = cand[~ok]     # kept if every try is rejected
            need[idx[ok]] = False
        X[:, t] = prop
    return X


def knn_rows(X: np.ndarray, k: int):
    """Host kNN inside each segment of X (n_seg, n, 3): (rows, cols) with each node's k nearest
    others (ties broken by index), sources ascending."""
    n_seg, n = X.shape[:2]
    rows_l, cols_l = [], []
    for cidx in range(n_seg):
        P = X[cidx]
        d2 = ((P[:, None, :] - P[None, :, :]) ** 2).sum(-1)
        np.fill_diagonal(d2, np.inf)
        nb = np.argsort(d2, axis=1, kind="stable")[:, :k]      # ties broken by index
        nb = np.sort(nb, axis=1)
        base = cidx * n
        rows_l.append(np.repeat(np.arange(n), nb.shape[1]) + base)
        cols_l.append(nb.reshape(-1) + base)
    return np.concatenate(rows_l), np.concatenate(cols_l)


def protein_chains(n_chains: int = 64, n_res: int = 512, k: int = 30, seed: int = 1003, feat_seed: int = 2003,
                   step: float = 3.8, min_dist: float = 3.0, n_types: int = 20, n_rbf: int = 16,
                   rbf_max: float = 15.0, max_tries: int = 200) -> Graph:
    """Self-avoiding 3-D random-walk chains with an in-chain kNN graph (k = 30)."""
    X = protein_positions(n_chains, n_res, seed, step, min_dist, max_tries)
    rows, cols = knn_rows(X, k)
    N = n_chains * n_res
    coord = X.reshape(N, 3).astype(np.float32)
    rowptr, col, _ = csr_from_rows(rows, cols, N)
    d = np.linalg.norm(coord[np.repeat(np.arange(N), np.diff(rowptr))] - coord[col], axis=1)
    types = _rng(feat_seed).integers(0, n_types, size=N)
    return Graph(rowptr, col, coord, _one_hot(types, n_types), rbf(d, n_rbf, rbf_max), dict(name="proteins"))


def slab_positions(n_sys: int = 256, n_atoms: int = 80, density: float = 0.08, seed: int = 1004) -> np.ndarray:
    """Uniform atoms in open cubes of side (n_atoms / density)^(1/3), float64 (n_sys, n_atoms, 3)."""
    side = (n_atoms / density) ** (1.0 / 3.0)
    return _rng(seed).uniform(0.0, side, size=(n_sys, n_atoms, 3))


def radius_rows(X: np.ndarray, cutoff: float, max_nb: int):
    """Host radius graph inside each segment of X (n_seg, n, 3): (rows, cols) with each node's
    nearest max_nb others (ties broken by index) within the cutoff, sources ascending."""
    n_sys, n_atoms = X.shape[:2]
    rows_l, cols_l = [], []
    for s in range(n_sys):
        P = X[s]
        d2 = ((P[:, None, :] - P[None, :, :]) ** 2).sum(-1)
        np.fill_diagonal(d2, np.inf)
        order = np.argsort(d2, axis=1, kind="stable")
        for i in range(n_atoms):
            cand = order[i, :max_nb]
            cand = cand[d2[i, cand] <= cutoff * cutoff]
            cand = np.sort(cand)
            rows_l.append(np.full(cand.size, i + s * n_atoms))
            cols_l.append(cand + s * n_atoms)
    return np.concatenate(rows_l), np.concatenate(cols_l)


def catalyst_slabs(n_sys: int = 256, n_atoms: int = 80, density: float = 0.08, cutoff: float = 6.0,
                   max_nb: int = 50, seed: int = 1004, feat_seed: int = 2004, n_types: int = 50,
                   n_rbf: int = 32) -> Graph:
    """Uniform atoms in open cubes, radius graph capped at the nearest ``max_nb``."""
    X = slab_positions(n_sys, n_atoms, density, seed)
    rows, cols = radius_rows(X, cutoff, max_nb)
    N = n_sys * n_atoms
    coord = X.reshape(N, 3).astype(np.float32)
    rowptr, col, _ = csr_from_rows(rows, cols, N)
    d = np.linalg.norm(coord[np.repeat(np.arange(N), np.diff(rowptr))] - coord[col], axis=1)
    types = _rng(feat_seed).integers(0, n_types, size=N)
    return Graph(rowptr, col, coord, _one_hot(types, n_types), rbf(d, n_rbf, cutoff), dict(name="slabs"))


def powerlaw_graph(N: int = 2_000_000, alpha: float = 2.1, dmin: int = 2, dmax: int = 4096, seed: int = 1005,
                   feat_seed: int = 2005, F: int = 128, FE: int = 16, with_features: bool = True) -> Graph:
    """Power-law in-degree graph for the MPNN stress workload."""
    r = _rng(seed)
    ks = np.arange(dmin, dmax + 1, dtype=np.float64)
    pmf = ks ** (-alpha)
    cdf = np.cumsum(pmf / pmf.sum())
    deg = ks[np.minimum(np.searchsorted(cdf, r.random(N), side="right"), ks.size - 1)].astype(np.int64)
    rowptr = np.zeros(N + 1, dtype=np.int64)
    np.cumsum(deg, out=rowptr[1:])
    E = int(rowptr[-1])
    rows = np.repeat(np.arange(N, dtype=np.int64), deg)
    src = r.integers(0, N, size=E)
    bad = src == rows
    while bad.any():
        src[bad] = r.integers(0, N, size=int(bad.sum()))
        bad = src == rows
    # sources ascending within each row
    key = rows * N + src
    src = src[np.argsort(key, kind="stable")]
    h = e = None
    if with_features:
        fr = _rng(feat_seed)
        h = fr.standard_normal((N, F), dtype=np.float32)
        e = fr.standard_normal((E, FE), dtype=np.float32)
    return Graph(rowptr.astype(np.int32), src.astype(np.int32), None, h, e, dict(name="powerlaw"))


def xavier_uniform(r: np.random.Generator, fan_in: int, fan_out: int, gain: float = 1.0) -> np.ndarray:
    """Xavier-uniform (in, out) matrix: U(-a, a), a = gain * sqrt(6 / (fan_in + fan_out))."""
    a = gain * np.sqrt(6.0 / (fan_in + fan_out))
    return r.uniform(-a, a, size=(fan_in, fan_out)).astype(np.float32)


# workload k -> (generator, H, layers, dtype, equivariant, F_E)
WORKLOADS = {
    1: dict(name="molecules-128", H=128, layers=1, dtypes=("fp32",), eq=True),
    2: dict(name="molecules-1024", H=128, layers=4, dtypes=("fp32", "bf16"), eq=True),
    3: dict(name="proteins-64x512", H=128, layers=4, dtypes=("bf16",), eq=True),
    4: dict(name="slabs-256x80", H=256, layers=6, dtypes=("bf16",), eq=True),
    5: dict(name="powerlaw-2M", H=128, layers=2, dtypes=("bf16",), eq=False),
}


def make_workload(k: int, **kw) -> Graph:
    """Graph and inputs of workload ``k`` (1..5) with its fixed seeds."""
    if k == 1:
        return molecule_batch(128, seed=1001, feat_seed=2001, **kw)
    if k == 2:
        return molecule_batch(1024, seed=1002, feat_seed=2002, **kw)
    if k == 3:
        return protein_chains(seed=1003, feat_seed=2003, **kw)
    if k == 4:
        return catalyst_slabs(seed=1004, feat_seed=2004, **kw)
    if k == 5:
        return powerlaw_graph(seed=1005, feat_seed=2005, **kw)
    raise ValueError(k)
