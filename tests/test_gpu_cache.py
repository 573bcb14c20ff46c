"""The reference's cache tests (tests/test_cache.py), on the HIP store.

The reference runs these on CPU tensors; here the same geometry (fp32,
head_dim 4, pages of 2 tokens) runs on the GPU store, and the cases go on
where the reference's stop: the truncated cache keeps decoding, a reset
store is refilled and retrieves what the oracle retrieves, and the memory
report of a populated host tier counts what the reference's formulas count
(kiv/cold_store.py:399-414, kiv/tiered_cache.py:259-286) plus what this
path reserves.
"""

from __future__ import annotations

import pytest
import torch
from transformers import PretrainedConfig

from kiv_amd import ColdKVStore, KIVConfig, ModelTopology
from kiv_amd.synthetic import Workload, generate
from kiv_amd.tiered_cache import TieredKVCache
from oracle.torch_ref import OracleColdStore
from tests.test_gpu_retrieval import attention_check, build, check_retrieval

pytestmark = pytest.mark.gpu


def _topology(**kw):
    """tests/test_cache.py:12-27 of the reference: Hq 2, Hkv 1, head_dim 4."""
    args = dict(global_layer_indices=(0,), independent_kv_layers=(0,), kv_sharing_map={}, num_query_heads=2,
                num_kv_heads=1, head_dim=4, num_hidden_layers=1)
    args.update(kw)
    return ModelTopology.manual(**args)


def test_retrieve_top_kv_preserves_batch_dimension(cuda):
    """tests/test_cache.py:30-44, with its shapes and dtype, on the GPU; the
    one selected token per batch row is the oracle's, K/V bit-exact."""
    g = torch.Generator().manual_seed(0)
    config = KIVConfig(page_size=2, top_p=1, top_pages=1, prefetch_stream=False)
    store = ColdKVStore(config, _topology(), cuda)
    key, value, query = torch.randn(2, 1, 2, 4, generator=g), torch.randn(2, 1, 2, 4, generator=g), \
        torch.randn(2, 2, 1, 4, generator=g)
    store.evict_from_hot(key.to(cuda), value.to(cuda))
    cold_key, cold_value = store.retrieve_top_kv(query.to(cuda), 1.0, config)
    assert cold_key.shape == (2, 1, 1, 4) and cold_value.shape == (2, 1, 1, 4)
    hot_key = torch.randn(2, 1, 1, 4, generator=g).to(cuda)
    assert torch.cat([cold_key, hot_key], dim=2).shape == (2, 1, 2, 4)
    oracle = OracleColdStore(2, 2)
    oracle.evict(key, value)
    ok, ov, _ = oracle.retrieve(query, 1.0, 1, 1)
    assert torch.equal(cold_key.cpu(), ok) and torch.equal(cold_value.cpu(), ov)


def test_head_dim_4_retrieve_and_attend(cuda):
    """Rows of one 16-byte chunk (fp32, head_dim 4) through the whole decode
    step: bands and oracle for the selection, the attention bar."""
    w = Workload("d4_f32", 4, 2, 4, torch.float32, hot=40, cold=3000 + 5, top_pages=6, top_p=50, segment=64,
                 page_size=16)
    data = generate(w, seed=81)
    store, oracle, cfg = build(w, data, cuda, chunks=(1000, 3))
    q, hk, hv = data["q"].to(cuda), data["hot_k"].to(cuda), data["hot_v"].to(cuda)
    out = store.retrieve_attend(q, w.scaling, cfg, hk, hv, None)
    k_out, v_out, _ = check_retrieval(store, oracle, cfg, w, data, data["q"])
    attention_check(q, k_out, v_out, hk, hv, w.scaling, out=out)


def test_truncate_to_rejects_truncation_into_cold(cuda):
    """tests/test_cache.py:106-132 on the GPU store, then decoding goes on
    from the truncated cache."""
    config = KIVConfig(hot_budget=4, page_size=2, prefetch_stream=False)
    cache = TieredKVCache(PretrainedConfig(num_hidden_layers=1), config, _topology(), cuda)
    g = torch.Generator().manual_seed(1)
    key, value = torch.randn(1, 1, 10, 4, generator=g).to(cuda), torch.randn(1, 1, 10, 4, generator=g).to(cuda)
    cache.update(key, value, 0)
    cache.mark_prefill_complete()
    store = cache.cold_stores[0]
    assert store.cold_length == 6
    assert cache.truncate_to(3) is False
    assert cache.layers[0].keys.shape[2] == 4  # untouched on rejection
    assert cache.truncate_to(6) is True
    assert cache.layers[0].keys.shape[2] == 0 and cache.get_seq_length(0) == 6 and cache._decode_step == 0
    # The next decode token: one hot row, and the cold tier still answers.
    k1, v1 = torch.randn(1, 1, 1, 4, generator=g).to(cuda), torch.randn(1, 1, 1, 4, generator=g).to(cuda)
    keys, _ = cache.update(k1, v1, 0)
    assert keys.shape[2] == 1 and torch.equal(keys, k1) and cache.get_seq_length(0) == 7
    q = torch.randn(1, 2, 1, 4, generator=g)
    ck, cv = store.retrieve_top_kv(q.to(cuda), 0.5, config, step=cache._decode_step)
    oracle = OracleColdStore(2, 2)
    oracle.evict(key[:, :, :6].cpu(), value[:, :, :6].cpu())
    ok, ov, _ = oracle.retrieve(q, 0.5, config.top_p, config.top_pages)
    assert ck.shape == ok.shape == (1, 1, 6, 4)
    assert torch.equal(ck.cpu(), ok) and torch.equal(cv.cpu(), ov)


def test_truncate_within_hot_with_a_populated_cold_tier(cuda):
    w = Workload("trunc", 8, 2, 64, torch.bfloat16, hot=64, cold=5000 + 9, top_pages=4, top_p=64, segment=256)
    data = generate(w, seed=82)
    config = KIVConfig(hot_budget=w.hot, top_p=w.top_p, top_pages=w.top_pages, page_size=w.page_size)
    topo = ModelTopology.manual(global_layer_indices=(0,), num_query_heads=8, num_kv_heads=2, head_dim=64,
                                num_hidden_layers=1)
    cache = TieredKVCache(PretrainedConfig(num_hidden_layers=1), config, topo, cuda)
    keys = torch.cat([data["cold_k"], data["hot_k"]], dim=2).to(cuda)
    vals = torch.cat([data["cold_v"], data["hot_v"]], dim=2).to(cuda)
    cache.update(keys, vals, 0)
    cache.mark_prefill_complete()
    store = cache.cold_stores[0]
    assert store.cold_length == w.cold and cache.layers[0].keys.shape[2] == w.hot
    store.retrieve_top_kv(data["q"].to(cuda), w.scaling, config, step=3)
    assert store._cached_step == 3
    total = w.cold + w.hot
    assert cache.truncate_to(total + 1) is False and cache.truncate_to(w.cold - 1) is False
    assert cache.truncate_to(total - 20) is True
    assert cache.layers[0].keys.shape[2] == w.hot - 20 and cache.get_seq_length(0) == total - 20
    assert torch.equal(cache.layers[0].keys, keys[:, :, w.cold:total - 20])
    assert torch.equal(cache.layers[0].values, vals[:, :, w.cold:total - 20])
    assert store._cached_step == -1 and store._cached_candidate_k is None and cache._decode_step == 0
    oracle = OracleColdStore(w.page_size, w.groups)
    oracle.evict(data["cold_k"], data["cold_v"])
    check_retrieval(store, oracle, config, w, data, data["q"])


def test_store_reset_then_refill(cuda):
    """ColdKVStore.reset (kiv/cold_store.py:374-389): an emptied store
    returns (None, None); refilled with other rows it retrieves what the
    oracle retrieves from those rows only (no stale summaries, union or
    partial rows), and reports their sizes."""
    w = Workload("reset_a", 8, 2, 64, torch.bfloat16, hot=16, cold=4000 + 7, top_pages=4, top_p=64, segment=256)
    data = generate(w, seed=83)
    store, oracle, cfg = build(w, data, cuda, chunks=(999, 1))
    store.retrieve_top_kv(data["q"].to(cuda), w.scaling, cfg, step=2)
    store.reset()
    assert store.cold_length == 0 and store.num_pages == 0 and store._cached_step == -1
    assert store.retrieve_top_kv(data["q"].to(cuda), w.scaling, cfg) == (None, None)
    mem = store.memory_bytes()
    assert mem["k_index_cpu"] == mem["v_store_cpu"] == mem["page_summaries_gpu"] == mem["partial_gpu"] == 0
    w2 = w.with_cold(2500 + 3)
    data2 = generate(w2, seed=84)
    oracle2 = OracleColdStore(w2.page_size, w2.groups)
    for t in range(0, w2.cold, 700):
        store.evict_from_hot(data2["cold_k"][:, :, t:t + 700].to(cuda), data2["cold_v"][:, :, t:t + 700].to(cuda))
        oracle2.evict(data2["cold_k"][:, :, t:t + 700], data2["cold_v"][:, :, t:t + 700])
    assert store.cold_length == w2.cold
    k, v = store.read_tokens()
    assert torch.equal(k.cpu(), data2["cold_k"]) and torch.equal(v.cpu(), data2["cold_v"])
    check_retrieval(store, oracle2, cfg, w2, data2, data2["q"])


def test_reset_telemetry(cuda):
    w = Workload("tele_reset", 8, 2, 64, torch.bfloat16, hot=16, cold=3000, top_pages=4, top_p=64, segment=256)
    data = generate(w, seed=85)
    store, _, cfg = build(w, data, cuda)
    for _ in range(3):
        store.retrieve_top_kv(data["q"].to(cuda), w.scaling, cfg)
    assert store.telemetry_snapshot()["aggregates"]["fine_calls"] == 3
    store.reset_telemetry()
    snap = store.telemetry_snapshot()
    assert snap["recent"] == [] and snap["aggregates"] == {"total_calls": 0, "coarse_calls": 0,
                                                           "coarse_real_calls": 0, "coarse_skipped_calls": 0,
                                                           "fine_calls": 0}
    store.retrieve_top_kv(data["q"].to(cuda), w.scaling, cfg)
    snap = store.telemetry_snapshot()
    assert len(snap["recent"]) == 2 and snap["aggregates"]["fine_calls"] == 1
    assert snap["aggregates"]["avg_fine_top_score"] == snap["recent"][-1]["top_score"]


@pytest.mark.parametrize("tier", ["host", "hbm", "split"])
def test_memory_bytes_and_report(cuda, tier):
    """The reference's keys count the bytes in use, by its formulas (K/V rows
    of finished pages, dtype summaries, the partial page's rows, the hot
    windows); the totals cover what this path holds, reservations included."""
    B, hkv, D, ps, cold, hot = 2, 2, 128, 128, 3 * 128 + 50, 96
    w = Workload("mem", 8, hkv, D, torch.bfloat16, hot=hot, cold=cold, top_pages=2, top_p=64, segment=128)
    data = generate(w, seed=86, batch=B)
    config = KIVConfig(hot_budget=hot, top_p=64, top_pages=2, page_size=ps, cold_tier=tier)
    topo = ModelTopology.manual(global_layer_indices=(0,), num_query_heads=8, num_kv_heads=hkv, head_dim=D,
                                num_hidden_layers=1)
    cache = TieredKVCache(PretrainedConfig(num_hidden_layers=1), config, topo, cuda)
    cache.update(torch.cat([data["cold_k"], data["hot_k"]], 2).to(cuda),
                 torch.cat([data["cold_v"], data["hot_v"]], 2).to(cuda), 0)
    cache.mark_prefill_complete()
    store = cache.cold_stores[0]
    store.retrieve_top_kv(data["q"].to(cuda), w.scaling, config)
    N, p, eb = cold // ps, cold % ps, 2
    rows = B * hkv * N * ps * D * eb             # [B, Hkv, N*ps, D] (kiv/cold_store.py:401-402)
    mem = store.memory_bytes()
    assert mem["page_summaries_gpu"] == B * hkv * N * D * eb
    assert mem["partial_gpu"] == 2 * B * hkv * p * D * eb
    placed = {"host": ("k_index_cpu", "v_store_cpu"), "hbm": ("k_cold_gpu", "v_cold_gpu"),
              "split": ("k_cold_gpu", "v_store_cpu")}[tier]
    for key in ("k_index_cpu", "v_store_cpu", "k_cold_gpu", "v_cold_gpu"):
        assert mem[key] == (rows if key in placed else 0), key
    cpu_rows = sum(mem[k] for k in ("k_index_cpu", "v_store_cpu"))
    gpu_used = mem["page_summaries_gpu"] + mem["partial_gpu"] + mem["k_cold_gpu"] + mem["v_cold_gpu"]
    assert mem["reserved_cpu"] >= cpu_rows and mem["reserved_gpu"] >= gpu_used
    rep = cache.memory_report()
    for key in ("hot_vram_bytes", "k_index_cpu_bytes", "v_store_cpu_bytes", "page_summaries_gpu_bytes",
                "total_vram_bytes", "total_cpu_bytes"):
        assert key in rep, key
    assert rep["hot_vram_bytes"] == 2 * B * hkv * hot * D * eb
    assert rep["k_index_cpu_bytes"] == mem["k_index_cpu"] and rep["v_store_cpu_bytes"] == mem["v_store_cpu"]
    assert rep["page_summaries_gpu_bytes"] == mem["page_summaries_gpu"]
    # The reference's totals: bytes in use (kiv/tiered_cache.py:279-286), plus HBM-resident cold rows.
    assert rep["total_vram_bytes"] == rep["hot_vram_bytes"] + gpu_used
    assert rep["total_cpu_bytes"] == cpu_rows
    assert rep["cold_rows_gpu_bytes"] == mem["k_cold_gpu"] + mem["v_cold_gpu"]
    if tier == "host":
        assert rep["total_vram_bytes"] == rep["hot_vram_bytes"] + mem["page_summaries_gpu"] + mem["partial_gpu"]
    # Reservations, reported apart.
    assert rep["hot_buffer_vram_bytes"] >= rep["hot_vram_bytes"]
    assert rep["reserved_total_vram_bytes"] == rep["hot_buffer_vram_bytes"] + mem["reserved_gpu"]
    assert rep["reserved_total_cpu_bytes"] == max(mem["reserved_cpu"], cpu_rows)
    assert rep["retrieval_scratch_vram_bytes"] == mem["reserved_gpu"] - gpu_used


def test_cache_reset_and_reuse(cuda):
    """TieredKVCache.reset (kiv/tiered_cache.py:183-192): the stores are
    emptied and the counters cleared; the hot layers go through
    DynamicCache.reset, which zeroes their rows and keeps their count (as in
    the reference).  The same cache then takes a new sequence: its first
    eviction moves the zeroed rows and the new ones to the cold tier, which
    retrieves what the oracle retrieves from those rows."""
    w = Workload("cache_reset", 8, 2, 64, torch.bfloat16, hot=32, cold=1500, top_pages=4, top_p=64, segment=128)
    data = generate(w, seed=87)
    config = KIVConfig(hot_budget=w.hot, top_p=w.top_p, top_pages=w.top_pages, page_size=w.page_size)
    topo = ModelTopology.manual(global_layer_indices=(0,), num_query_heads=8, num_kv_heads=2, head_dim=64,
                                num_hidden_layers=1)
    cache = TieredKVCache(PretrainedConfig(num_hidden_layers=1), config, topo, cuda)
    all_k = torch.cat([data["cold_k"], data["hot_k"]], 2)
    all_v = torch.cat([data["cold_v"], data["hot_v"]], 2)
    cache.update(all_k.to(cuda), all_v.to(cuda), 0)
    cache.mark_prefill_complete()
    assert cache.cold_stores[0].cold_length == w.cold
    cache.reset()
    store = cache.cold_stores[0]
    assert store.cold_length == 0 and cache._decode_step == 0 and not cache._prefill_complete
    assert cache._total_tokens == {}
    layer = cache.layers[0]
    assert layer.keys.shape[2] == w.hot and not layer.keys.any() and not layer.values.any()
    assert cache.get_seq_length(0) == w.hot
    n = 700
    cache.update(all_k[:, :, :n + w.hot].to(cuda), all_v[:, :, :n + w.hot].to(cuda), 0)
    cache.mark_prefill_complete()
    zeros = torch.zeros(1, 2, w.hot, 64, dtype=w.dtype)
    cold_k = torch.cat([zeros, all_k[:, :, :n]], 2)
    cold_v = torch.cat([zeros, all_v[:, :, :n]], 2)
    assert store.cold_length == n + w.hot and cache.get_seq_length(0) == n + 2 * w.hot
    k, v = store.read_tokens()
    assert torch.equal(k.cpu(), cold_k) and torch.equal(v.cpu(), cold_v)
    oracle = OracleColdStore(w.page_size, w.groups)
    oracle.evict(cold_k, cold_v)
    part = dict(data, cold_k=cold_k, cold_v=cold_v)
    check_retrieval(store, oracle, config, w.with_cold(n + w.hot), part, data["q"])
