"""Deferred eviction (the cache's decode steps): rows handed to
ColdKVStore.evict_deferred are written by the next retrieval (inside its
coarse scan launch when they stay in the partial page, by the eviction
kernels otherwise) or by any other use of the store.  Two stores fed the
same rows, one deferring and one evicting at once, must hold the same rows
and summaries and return the same selections, rows and telemetry."""

from __future__ import annotations

import pytest
import torch

from kiv_amd import ColdKVStore, KIVConfig, ModelTopology
from kiv_amd.synthetic import Workload, generate

pytestmark = pytest.mark.gpu


def _pair(w, data, cuda, cold0, cfg):
    topo = ModelTopology.manual(global_layer_indices=(0,), num_query_heads=w.num_q_heads,
                                num_kv_heads=w.num_kv_heads, head_dim=w.head_dim, num_hidden_layers=1)
    a, b = ColdKVStore(cfg, topo, cuda), ColdKVStore(cfg, topo, cuda)
    if cold0:
        for s in (a, b):
            s.evict_from_hot(data["cold_k"][:, :, :cold0].to(cuda), data["cold_v"][:, :, :cold0].to(cuda))
    return a, b


def _same(a, b, q, w, cfg, step=-1):
    ka, va = a.retrieve_top_kv(q, w.scaling, cfg, step=step)
    kb, vb = b.retrieve_top_kv(q, w.scaling, cfg, step=step)
    assert torch.equal(ka, kb) and torch.equal(va, vb)
    ra, rb = a.telemetry_snapshot()["recent"][-2:], b.telemetry_snapshot()["recent"][-2:]
    assert ra == rb
    assert a.cold_length == b.cold_length and a.num_pages == b.num_pages


@pytest.mark.parametrize("tier", ["host", "hbm"])
@pytest.mark.parametrize("pruning", [False, True])
def test_deferred_matches_immediate_over_decode_steps(cuda, tier, pruning):
    """300 decode steps of one row each from 1,000 cold tokens: the rows
    cross two page ends (kiv_evict path) and otherwise ride on the coarse
    scan; every step's retrieval agrees, and so do the stored rows."""
    w = Workload("deferred", 8, 2, 64, torch.bfloat16, hot=400, cold=1000, top_pages=4, top_p=64, segment=128)
    data = generate(w, seed=91)
    cfg = KIVConfig(hot_budget=w.hot, top_p=w.top_p, top_pages=w.top_pages, cold_tier=tier, fine_pruning=pruning)
    a, b = _pair(w, data, cuda, w.cold, cfg)
    hk, hv = data["hot_k"].to(cuda), data["hot_v"].to(cuda)
    q = data["q"].to(cuda)
    for t in range(300):
        a.evict_deferred(hk[:, :, t:t + 1], hv[:, :, t:t + 1])
        b.evict_from_hot(hk[:, :, t:t + 1], hv[:, :, t:t + 1])
        assert a.cold_length == b.cold_length == w.cold + t + 1
        if t % 7 == 0:
            _same(a, b, q, w, cfg)
        else:
            out_a = a.retrieve_attend(q, w.scaling, cfg, hk[:, :, t + 1:], hv[:, :, t + 1:], None)
            out_b = b.retrieve_attend(q, w.scaling, cfg, hk[:, :, t + 1:], hv[:, :, t + 1:], None)
            assert torch.equal(out_a, out_b)
    ka, va = a.read_tokens()
    kb, vb = b.read_tokens()
    assert torch.equal(ka, kb) and torch.equal(va, vb)
    assert torch.equal(ka.cpu(), torch.cat([data["cold_k"], data["hot_k"][:, :, :300]], 2))
    assert torch.equal(a.read_summaries()[1], b.read_summaries()[1])


def test_deferred_edges(cuda):
    """No finished page yet (written at once), several rows at a time, a
    shared-layer reuse after a deferred row (the eviction drops the union,
    so the call is fresh), and every other use of the store writing the
    rows first: read_tokens, memory_bytes, reset (drops them)."""
    w = Workload("deferred_edges", 8, 2, 64, torch.bfloat16, hot=64, cold=300, top_pages=2, top_p=32, segment=64)
    data = generate(w, seed=92)
    cfg = KIVConfig(hot_budget=w.hot, top_p=w.top_p, top_pages=w.top_pages)
    hk, hv = data["hot_k"].to(cuda), data["hot_v"].to(cuda)
    q = data["q"].to(cuda)
    a, b = _pair(w, data, cuda, 0, cfg)
    # no pages: immediate
    a.evict_deferred(data["cold_k"][:, :, :100].to(cuda), data["cold_v"][:, :, :100].to(cuda))
    b.evict_from_hot(data["cold_k"][:, :, :100].to(cuda), data["cold_v"][:, :, :100].to(cuda))
    assert a._pending is None
    _same(a, b, q, w, cfg)
    a.evict_from_hot(data["cold_k"][:, :, 100:300].to(cuda), data["cold_v"][:, :, 100:300].to(cuda))
    b.evict_from_hot(data["cold_k"][:, :, 100:300].to(cuda), data["cold_v"][:, :, 100:300].to(cuda))
    # three rows at once, then retrieval at a step, then a reuse call
    a.evict_deferred(hk[:, :, :3], hv[:, :, :3])
    b.evict_from_hot(hk[:, :, :3], hv[:, :, :3])
    assert a._pending is not None
    _same(a, b, q, w, cfg, step=4)
    _same(a, b, q, w, cfg, step=4)
    assert a.telemetry_snapshot()["recent"][-2]["skipped"] is True
    # flushes
    a.evict_deferred(hk[:, :, 3:4], hv[:, :, 3:4])
    b.evict_from_hot(hk[:, :, 3:4], hv[:, :, 3:4])
    ka, va = a.read_tokens()
    kb, vb = b.read_tokens()
    assert a._pending is None and torch.equal(ka, kb) and torch.equal(va, vb)
    a.evict_deferred(hk[:, :, 4:5], hv[:, :, 4:5])
    b.evict_from_hot(hk[:, :, 4:5], hv[:, :, 4:5])
    assert a.memory_bytes() == b.memory_bytes() and a._pending is None
    a.evict_deferred(hk[:, :, 5:6], hv[:, :, 5:6])
    a.reset()
    assert a._pending is None and a.cold_length == 0
    assert a.retrieve_top_kv(q, w.scaling, cfg) == (None, None)
