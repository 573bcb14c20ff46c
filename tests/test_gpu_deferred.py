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


def _tiny_qwen2(cuda, dtype):
    from transformers import Qwen2Config, Qwen2ForCausalLM

    cfg = Qwen2Config(vocab_size=512, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=2, head_dim=64, max_position_embeddings=4096,
                      tie_word_embeddings=False)
    cfg._attn_implementation = "eager"
    torch.manual_seed(0)
    return Qwen2ForCausalLM(cfg).to(dtype).to(cuda).eval()


@pytest.mark.parametrize("dtype,per_step", [(torch.bfloat16, 1), (torch.float32, 1), (torch.bfloat16, 2)])
def test_hot_rows_written_by_the_retrieval_match_the_cache_copy(cuda, dtype, per_step, monkeypatch):
    """Under the middleware a decode update leaves the new hot rows to the
    layer's retrieval: its first launch writes them (the coarse scan's extra
    blocks, or a copy launch while the store has no finished page), or the
    wrapper writes them on paths without it (two query positions per step).
    fp32 takes the call's two-launch form, whose retrieval writes them.  Against the
    same model with the cache's own copies: identical logits and telemetry at
    every step, from a cold tier of 5 tokens (no finished page) to several
    pages."""
    print(f"deferred hot rows case dtype={dtype} per_step={per_step}", flush=True)
    from kiv_amd import KIVMiddleware
    from kiv_amd import middleware as mwmod

    seen = {"retrieval": 0, "wrapper": 0}
    real_retrieve, real_write = ColdKVStore._retrieve, mwmod._write_rows

    def retrieve_spy(self, *args, **kwargs):
        rows = args[5] if len(args) > 5 else kwargs.get("hot_rows")
        seen["retrieval"] += rows is not None
        return real_retrieve(self, *args, **kwargs)

    def write_spy(rows):
        seen["wrapper"] += rows is not None
        return real_write(rows)

    monkeypatch.setattr(ColdKVStore, "_retrieve", retrieve_spy)
    monkeypatch.setattr(mwmod, "_write_rows", write_spy)
    model = _tiny_qwen2(cuda, dtype)
    mw = KIVMiddleware(model, KIVConfig(hot_budget=64, top_p=16, page_size=16, top_pages=2))
    mw.install()
    try:
        ids = torch.randint(0, 512, (1, 69), generator=torch.Generator().manual_seed(8)).to(cuda)
        runs = []
        for defer in (True, False):
            cache = mw.create_cache(cuda)
            cache._defer_hot_append = defer
            logits, tel = [], []
            with torch.no_grad():
                out = mw.chunked_prefill(ids, cache, chunk_size=32)
                assert cache.get_cold_store(0).cold_length == 5
                tok = out.argmax(-1, keepdim=True).repeat(1, per_step)
                for _ in range(40):
                    lg = model(input_ids=tok, past_key_values=cache, use_cache=True).logits[:, -per_step:]
                    logits.append(lg)
                    tok = lg.argmax(-1)
            assert all(layer._pending_rows is None for layer in cache.layers if hasattr(layer, "_pending_rows"))
            for i in sorted(cache.cold_stores):
                tel.append(cache.cold_stores[i].telemetry_snapshot()["recent"])
            runs.append((logits, tel, cache))
        (la, ta, ca), (lb, tb, cb) = runs
        # Every decode step of both layers deferred its rows in the first run:
        # the retrieval took them (one position), or the wrapper wrote them.
        if per_step == 1:
            assert seen["retrieval"] == 80 and seen["wrapper"] == 0
        else:
            assert seen["retrieval"] == 0 and seen["wrapper"] == 80
        assert ca.get_cold_store(0).num_pages >= 2
        for x, y in zip(la, lb):
            assert torch.equal(x, y)
        assert ta == tb
        for i in ca.cold_stores:
            assert torch.equal(ca.layers[i].keys, cb.layers[i].keys)
            assert torch.equal(ca.layers[i].values, cb.layers[i].values)
    finally:
        mw.uninstall()
