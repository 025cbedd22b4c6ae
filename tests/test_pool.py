"""Slab state pool bookkeeping (kdn_pool_*) on the host, as the reference's own test exercises it
(serving/test_hybrid_memory_pool.cpp:8-81: allocate 100 of 128 streams, fork 20, release everything,
zero bytes left allocated), plus ordering, capacity and error cases.  A CPU slab makes the pool skip
its device work (zeroing, fork copies), which the GPU tests cover."""
import pytest

from kdn import ops
from serving import HybridMemoryPool


def test_reference_pool_scenario():
    pool = HybridMemoryPool(128, 16384, num_layers=1, num_heads=1, val_dim=16, lifted_dim=64, device="cpu")
    per = pool.recurrent_bytes_per_stream
    ids = [pool.allocate_stream(2048) for _ in range(100)]
    assert ids == list(range(100))  # lowest free slot first
    kids = [pool.fork_stream(s) for s in ids[:20]]
    assert kids == list(range(100, 120))
    assert pool.get_total_allocated_bytes() == 120 * per
    assert pool.get_free_bytes() == 8 * per
    for s in kids + ids:
        pool.release_stream(s)
    assert pool.get_total_allocated_bytes() == 0
    assert pool.get_free_bytes() == 128 * per


def test_capacity_reuse_and_errors():
    p = ops.StatePool(3, 1, 1, 64, 16, device="cpu")
    assert [p.allocate() for _ in range(3)] == [0, 1, 2]
    assert p.allocate() == -1          # full
    assert p.fork(1) == -1             # no free slot for the child
    p.release(1)
    assert p.active == 2
    assert p.allocate() == 1           # the released slot comes back first
    with pytest.raises(RuntimeError):
        p.release(7)                   # out of range
    p.release(2)
    with pytest.raises(RuntimeError):
        p.release(2)                   # not active any more
    with pytest.raises(RuntimeError):
        p.fork(2)                      # inactive parent
    assert p.fork(0) == 2
    assert p.allocated_bytes() == 3 * p.slot_bytes


def test_pool_create_rejects_bad_sizes():
    import ctypes
    from kdn import _native as N
    h = ctypes.c_void_p()
    assert N.lib().kdn_pool_create(0, 64, ctypes.byref(h)) == -1
    assert N.lib().kdn_pool_create(4, 20, ctypes.byref(h)) == -1   # not a multiple of 16 bytes
    assert N.lib().kdn_pool_create(4, 64, ctypes.byref(h)) == 0
    N.lib().kdn_pool_destroy(h)


def test_ragged_workspace_query_needs_no_device():
    import ctypes
    import numpy as np
    from kdn import _native as N
    a = N.RaggedArgs()
    cu = np.array([0, 1, 2, 70, 70, 200], dtype=np.int64)
    a.num_seqs, a.H, a.d_k, a.D, a.d_v = 5, 16, 64, 512, 64
    a.num_slots = 8
    a.in_dtype = a.out_dtype = 1
    a.inv_tau = 0.35
    a.cu_seqlens_host = cu.ctypes.data
    assert N.lib().kdn_ragged_workspace_bytes(ctypes.byref(a)) > 0
    bad = np.array([0, 5, 3, 4, 6, 9], dtype=np.int64)   # decreasing offsets
    a.cu_seqlens_host = bad.ctypes.data
    assert N.lib().kdn_ragged_workspace_bytes(ctypes.byref(a)) == 0
    a.cu_seqlens_host = cu.ctypes.data
    a.d_v = 48
    assert N.lib().kdn_ragged_workspace_bytes(ctypes.byref(a)) == 0
