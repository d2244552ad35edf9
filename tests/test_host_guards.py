"""Host-side guards (CPU): a KV cache refuses a call that would pass its
capacity (the kernels would drop those writes), caches driven by a captured
cycle refuse host edits except during capture, recurrent rollback is bounded by
the last call's width, and cache clones are independent."""

import numpy as np
import pytest
import torch

from qvex import _C
from qvex.model import Attention, CacheCounters, KVCache, LayerCaches, RecurrentCache


def attention_stub(H=2, Hkv=1, D=64):
    att = Attention.__new__(Attention)
    att.cfg = None
    att.n_heads, att.n_kv, att.head_dim = H, Hkv, D
    return att


def test_kv_cache_refuses_to_overflow():
    counters = CacheCounters(1, "cpu")
    cache = KVCache(counters, 0, n_kv=1, head_dim=64, capacity=256, device="cpu")
    assert cache.capacity == 256
    cache.offset = 254
    att = attention_stub()
    with pytest.raises(_C.QvexError, match="KV cache full"):
        att(torch.zeros((4, 128)), cache)
    assert cache.offset == 254                      # nothing advanced


def test_graph_mode_refuses_host_edits_except_while_capturing():
    counters = CacheCounters(3, "cpu")
    caches = LayerCaches([KVCache(counters, i, n_kv=1, head_dim=64, capacity=256, device="cpu") for i in range(3)],
                         counters)
    caches[1].offset = 7
    counters.graph_mode = True
    with pytest.raises(_C.QvexError, match="captured cycle"):
        caches[0].rollback(1)
    with pytest.raises(_C.QvexError, match="captured cycle"):
        counters.sync()
    counters.capturing = True
    caches[2].offset = 5                            # model code edits the mirror during capture
    counters.sync()
    counters.capturing = False
    counters.graph_mode = False
    assert counters.host.tolist() == [0, 7, 5]


def test_recurrent_rollback_bounded_and_clone_independent():
    counters = CacheCounters(2, "cpu")
    rc = RecurrentCache(counters, 0, conv_dim=8, kernel=4, hv=1, dv=4, dk=4, max_width=4, device="cpu",
                        prefill_width=8)
    kv = KVCache(counters, 1, n_kv=1, head_dim=64, capacity=256, device="cpu")
    caches = LayerCaches([rc, kv], counters)
    rc.offset, rc.last_width = 10, 3
    rc.rollback(2)
    with pytest.raises(_C.QvexError, match="only the last 1"):
        rc.rollback(2)
    twin = caches.clone()
    twin[0].offset = 99
    twin[0].ssm_ring.fill_(1.0)
    kv.k.fill_(2.0)
    assert rc.offset == 8 and twin[0].offset == 99
    assert float(rc.ssm_ring.abs().sum()) == 0.0 and float(twin[1].k.abs().sum()) == 0.0
    assert twin[0].counters is twin[1].counters and twin.counters is not counters
    assert np.array_equal(counters.host, np.array([8, 0], np.int32))
