"""Host-side guards (CPU): a KV cache grows in 256-token steps and keeps its
keys where the kernels read them, caches driven by a captured
cycle refuse host edits except during capture, recurrent rollback is bounded by
the last call's width, and cache clones are independent."""

import numpy as np
import pytest
import torch

from qvex import _C
from qvex.model import CacheCounters, KVCache, LayerCaches, RecurrentCache


def test_kv_cache_grows_in_steps_keeping_its_keys():
    """KVCache.grow (engine/model.py:156-170 grows by 256-token steps): the
    capacity rounds up to a step, every kept tile stays where the attention
    kernels read it (a head's tiles are key-major), the new tiles are zero, and
    a cache driven by a captured cycle refuses to move."""
    counters = CacheCounters(1, "cpu")
    cache = KVCache(counters, 0, n_kv=2, head_dim=64, capacity=256, device="cpu")
    cache.k.copy_(torch.arange(cache.k.numel(), dtype=torch.float32).reshape(cache.k.shape))
    cache.v.copy_(-torch.arange(cache.v.numel(), dtype=torch.float32).reshape(cache.v.shape))
    k0, v0 = cache.k.clone(), cache.v.clone()
    cache.offset = 254
    assert not cache.grow(256)
    assert cache.grow(254 + 4)
    assert cache.capacity == 512
    assert cache.k.shape == (2, 512 // 16, 2, 64, 8) and cache.v.shape == (2, 512 // 32, 64, 32)
    assert torch.equal(cache.k[:, :16], k0) and torch.equal(cache.v[:, :8], v0)
    assert float(cache.k[:, 16:].abs().sum()) == 0.0 and float(cache.v[:, 8:].abs().sum()) == 0.0
    assert cache.offset == 254
    assert cache.grow(1000) and cache.capacity == 1024
    assert torch.equal(cache.k[:, :16], k0)
    counters.graph_mode = True
    with pytest.raises(_C.QvexError, match="captured cycle"):
        cache.grow(2000)
    assert cache.capacity == 1024


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
