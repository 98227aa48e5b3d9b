"""The per-graph caches of the module path (CPU only: the caches are host logic).

The modules convert the COO ``edge_index`` to a dst-sorted CSR once per graph
(the reference rebuilds it on every call: egnn_clean.py:95-101, layer.py:41-63).
The cache must follow the graph, not the address of its tensor: a freed edge
tensor's memory is handed to the next tensor of the same size, with a fresh
version counter, so an address-keyed cache would return the old graph's CSR.
"""
import gc

import numpy as np
import torch

from pymolecular_amd import graphs
from pymolecular_amd.fused import TensorCache, coo_to_csr
from pymolecular_amd.models.EGNN.egnn_clean import _CSRCache
from pymolecular_amd.models.EGNN.layer import EGNN_HIP_Layer


def _graph(seed, N=50, E=400):
    r = np.random.Generator(np.random.PCG64(seed))
    return r.integers(0, N, E), r.integers(0, N, E)


def _expected(rows, cols, N):
    rowptr, col, perm = graphs.csr_from_rows(np.asarray(rows), np.asarray(cols), N)
    return rowptr, col, perm


def _same(csr, rows, cols, N):
    rp, cl, pm = _expected(rows, cols, N)
    return (np.array_equal(csr[0].numpy(), rp) and np.array_equal(csr[1].numpy(), cl)
            and np.array_equal(csr[2].numpy(), pm))


def test_tensor_cache_hits_live_tensor_and_views():
    c = TensorCache()
    calls = []
    t = torch.arange(10).reshape(2, 5)
    make = lambda: calls.append(1) or len(calls)  # noqa: E731
    assert c.get((t,), 0, make) == 1
    assert c.get((t,), 0, make) == 1                 # same live tensor: hit
    a, b = t                                         # fresh views each unpacking
    assert c.get((a, b), 0, make) == 2
    a2, b2 = t
    assert c.get((a2, b2), 0, make) == 2             # views of the same root and offsets: hit
    assert c.get((b2, a2), 0, make) == 3             # swapped: different offsets
    assert c.get((t,), 1, make) == 4                 # different extra key
    t.add_(1)                                        # in-place edit bumps the version
    assert c.get((t,), 0, make) == 5


def test_tensor_cache_same_address_new_tensor_misses():
    # Two distinct tensors over one storage at the same offset, each written once (version 1):
    # the same data pointer, shape, strides and version -- what an address-keyed cache confuses.
    N, E = 50, 400
    storage = torch.empty((2, E), dtype=torch.int64).untyped_storage()
    A = torch.empty(0, dtype=torch.int64).set_(storage, 0, (2, E))
    ra, ca = _graph(1, N, E)
    A.copy_(torch.from_numpy(np.stack([ra, ca])))
    cache = _CSRCache()
    assert _same(cache.get(A[0], A[1], N), ra, ca, N)
    ptr_a, ver_a = A.data_ptr(), A._version
    del A
    gc.collect()
    B = torch.empty(0, dtype=torch.int64).set_(storage, 0, (2, E))
    rb, cb = _graph(2, N, E)
    B.copy_(torch.from_numpy(np.stack([rb, cb])))
    assert (B.data_ptr(), B._version) == (ptr_a, ver_a)
    assert _same(cache.get(B[0], B[1], N), rb, cb, N)


def test_csr_cache_freed_and_reallocated_edges():
    # the scenario of a training loop over graphs of equal E: free, allocate, fill, call
    N, E = 60, 500
    cache = _CSRCache()
    reused = 0
    prev = None
    for k in range(20):
        r, c = _graph(100 + k, N, E)
        row = torch.empty(E, dtype=torch.int64)
        col = torch.empty(E, dtype=torch.int64)
        row.copy_(torch.from_numpy(r))
        col.copy_(torch.from_numpy(c))
        reused += prev == (row.data_ptr(), col.data_ptr())
        assert _same(cache.get(row, col, N), r, c, N), k
        assert _same(cache.get(row, col, N), r, c, N), k       # and the hit returns the same graph
        prev = (row.data_ptr(), col.data_ptr())
        del row, col
    print(f"addresses reused in {reused} of 19 reallocations")


def test_both_ways_cache_follows_the_graph():
    N, E = 40, 300
    layer = EGNN_HIP_Layer(16, 0, 32, 32, 32, 32)
    for k in range(10):
        s, d = _graph(200 + k, N, E)
        ei = torch.empty((2, E), dtype=torch.int64)
        ei.copy_(torch.from_numpy(np.stack([s, d])))
        rp, cl, eids, deg = layer._both_ways(ei, N)
        rows = np.concatenate([d, s])
        cols = np.concatenate([s, d])
        erp, ecl, eperm = _expected(rows, cols, N)
        assert np.array_equal(rp.numpy(), erp) and np.array_equal(cl.numpy(), ecl), k
        assert np.array_equal(eids.numpy(), eperm % E), k
        assert layer._both_ways(ei, N) is layer._both_ways(ei, N)
        del ei


def test_coo_to_csr_matches_numpy():
    r, c = _graph(5, 30, 200)
    rp, cl, pm = coo_to_csr(torch.from_numpy(r), torch.from_numpy(c), 30)
    assert _same((rp, cl, pm), r, c, 30)
