"""Host-side API behaviour (CPU): the reference's own test intents, run
against kiv_amd (tests/test_model_topology.py, tests/test_middleware.py and
the hot-window parts of tests/test_cache.py in the reference), plus
detection and install/uninstall on a tiny random-init Qwen2 model.

Anything that evicts to the cold tier needs the HIP kernels and lives in
the GPU tests; here it must fail loudly instead of falling back to CPU.
"""

from __future__ import annotations

from types import SimpleNamespace

import pytest
import torch
from transformers import PretrainedConfig

from kiv_amd import ColdKVStore, KIVConfig, ModelTopology
from kiv_amd.mask_utils import extend_mask_for_cold
from kiv_amd.middleware import KIVMiddleware, _prefill_logits_kwargs
from kiv_amd.tiered_cache import TieredKVCache


def _make(**overrides):
    d = dict(model_family="test", num_hidden_layers=4, global_layer_indices=(0, 1, 2),
             independent_kv_layers=(0, 1, 2), kv_sharing_map={}, num_query_heads=2, num_kv_heads=1, head_dim=4)
    d.update(overrides)
    return ModelTopology(**d)


def _topology(global_layer_indices=(0,), independent_kv_layers=(0,), kv_sharing_map=None, num_hidden_layers=1):
    return ModelTopology.manual(global_layer_indices=global_layer_indices,
                                independent_kv_layers=independent_kv_layers,
                                kv_sharing_map=kv_sharing_map or {}, num_query_heads=2, num_kv_heads=1,
                                head_dim=4, num_hidden_layers=num_hidden_layers)


# ------------------------------------------------------------------ topology
def test_valid_topology_constructs():
    t = _make(global_layer_indices=(0, 1, 2, 3), independent_kv_layers=(0, 2), kv_sharing_map={1: 0, 3: 2})
    assert t.kv_sharing_map == {1: 0, 3: 2}


def test_independent_kv_layers_not_subset_rejected():
    with pytest.raises(ValueError, match="independent_kv_layers"):
        _make(global_layer_indices=(0, 1), independent_kv_layers=(0, 1, 5))


def test_sharing_key_outside_globals_rejected():
    with pytest.raises(ValueError, match="kv_sharing_map keys"):
        _make(global_layer_indices=(0, 2), independent_kv_layers=(0, 2), kv_sharing_map={1: 0})


def test_sharing_source_outside_independents_rejected():
    with pytest.raises(ValueError, match="kv_sharing_map values"):
        _make(global_layer_indices=(0, 1, 2), independent_kv_layers=(0,), kv_sharing_map={2: 1})


def test_manual_defaults_to_globals_for_independents():
    t = ModelTopology.manual(global_layer_indices=(0, 1), num_query_heads=2, num_kv_heads=1, head_dim=4,
                             num_hidden_layers=2)
    assert t.independent_kv_layers == (0, 1)


# -------------------------------------------------------------------- config
def test_config_defaults_and_validation():
    c = KIVConfig()
    assert (c.hot_budget, c.top_p, c.page_size, c.top_pages, c.prefetch_stream) == (2048, 256, 128, 32, True)
    assert KIVConfig(4096, 512, 64, 16, False).top_pages == 16
    with pytest.raises(ValueError):
        KIVConfig(cold_tier="disk")
    with pytest.raises(ValueError):
        KIVConfig(score_rounding="fp8")
    assert c.fine_pruning is False and KIVConfig(fine_pruning=True).fine_pruning is True


# ---------------------------------------------------------------------- mask
def test_extend_mask_for_cold():
    m2 = torch.tensor([[True, False]])
    out = extend_mask_for_cold(m2, 3)
    assert out.tolist() == [[True, True, True, True, False]]
    m4 = torch.full((2, 1, 1, 4), float("-inf"))
    out4 = extend_mask_for_cold(m4, 2)
    assert out4.shape == (2, 1, 1, 6) and torch.all(out4[..., :2] == 0) and torch.all(torch.isinf(out4[..., 2:]))
    m3 = torch.zeros(2, 3, 5)
    assert extend_mask_for_cold(m3, 1).shape == (2, 3, 6)


# --------------------------------------------------------------------- cache
def test_shared_layer_seq_length_resolves_to_source_layer():
    topo = _topology(global_layer_indices=(0, 1), independent_kv_layers=(0,), kv_sharing_map={1: 0},
                     num_hidden_layers=2)
    cache = TieredKVCache(PretrainedConfig(num_hidden_layers=2), KIVConfig(prefetch_stream=False), topo,
                          torch.device("cpu"))
    cache._total_tokens[0] = 123
    assert cache.get_seq_length(0) == 123
    assert cache.get_seq_length(1) == 123
    assert cache.get_cold_store(1) is cache.cold_stores[0]


def test_truncate_to_hot_only_succeeds():
    cache = TieredKVCache(PretrainedConfig(num_hidden_layers=1), KIVConfig(prefetch_stream=False), _topology(),
                          torch.device("cpu"))
    key, value = torch.randn(1, 1, 10, 4), torch.randn(1, 1, 10, 4)
    cache.update(key, value, 0)
    assert cache.truncate_to(6) is True
    layer = cache.layers[0]
    assert layer.keys.shape[2] == 6 and layer.values.shape[2] == 6
    assert cache._total_tokens[0] == 6
    torch.testing.assert_close(layer.keys, key[:, :, :6])
    torch.testing.assert_close(layer.values, value[:, :, :6])


def test_truncate_to_rejects_lengths_beyond_current_total():
    cache = TieredKVCache(PretrainedConfig(num_hidden_layers=1), KIVConfig(prefetch_stream=False), _topology(),
                          torch.device("cpu"))
    cache.update(torch.randn(1, 1, 4, 4), torch.randn(1, 1, 4, 4), 0)
    assert cache.truncate_to(10) is False
    assert cache.layers[0].keys.shape[2] == 4


def test_no_eviction_before_prefill_and_mask_sizes():
    cfg = KIVConfig(hot_budget=4, page_size=2)
    cache = TieredKVCache(PretrainedConfig(num_hidden_layers=1), cfg, _topology(), torch.device("cpu"))
    cache.update(torch.randn(1, 1, 10, 4), torch.randn(1, 1, 10, 4), 0)
    assert cache.layers[0].keys.shape[2] == 10 and cache.cold_stores[0].cold_length == 0
    assert cache.get_seq_length(0) == 10
    assert cache.get_mask_sizes(1, 0) == (11, 0)
    mem = cache.memory_report()
    assert mem["hot_vram_bytes"] == 2 * 10 * 4 * 4 and mem["total_cpu_bytes"] == 0


def test_cold_tier_has_no_cpu_fallback():
    """Eviction on a CPU tensor raises: the cold tier only exists as HIP kernels."""
    cache = TieredKVCache(PretrainedConfig(num_hidden_layers=1), KIVConfig(hot_budget=4, page_size=2),
                          _topology(), torch.device("cpu"))
    cache.update(torch.randn(1, 1, 10, 4), torch.randn(1, 1, 10, 4), 0)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        cache.mark_prefill_complete()
    store = ColdKVStore(KIVConfig(), _topology(), torch.device("cpu"))
    assert store.retrieve_top_kv(torch.zeros(1, 2, 1, 4), 1.0, KIVConfig()) == (None, None)


# ---------------------------------------------------------------- middleware
class _FakeCache:
    def __init__(self):
        self._suppress_cold = False
        self._prefill_complete = False
        self.evict_calls = []
        self.marked = False
        self.evicted_excess = False

    def _evict_to_cap(self, cap):
        self.evict_calls.append(cap)

    def _evict_excess_all_layers(self):
        self.evicted_excess = True

    def mark_prefill_complete(self):
        self.marked = True


class _ModelWithLogitsToKeep(torch.nn.Module):
    def __init__(self):
        super().__init__()
        self.config = SimpleNamespace()
        self.calls = []

    def forward(self, input_ids, past_key_values=None, use_cache=False, logits_to_keep=0):
        self.calls.append(logits_to_keep)
        return SimpleNamespace(logits=torch.zeros(input_ids.shape[0], logits_to_keep or input_ids.shape[1], 3))


class _ModelWithoutLogitsToKeep(torch.nn.Module):
    def __init__(self):
        super().__init__()
        self.config = SimpleNamespace()
        self.calls = 0

    def forward(self, input_ids, past_key_values=None, use_cache=False):
        self.calls += 1
        return SimpleNamespace(logits=torch.zeros(input_ids.shape[0], input_ids.shape[1], 3))


class _RaisingModel(torch.nn.Module):
    def __init__(self):
        super().__init__()
        self.config = SimpleNamespace()

    def forward(self, input_ids, past_key_values=None, use_cache=False):
        raise RuntimeError("boom")


def _installed(model):
    mw = KIVMiddleware(model)
    mw._installed = True
    mw._original_impl = "eager"
    mw._kiv_key = "kiv_eager"
    return mw


def test_prefill_logits_kwargs_detection():
    assert _prefill_logits_kwargs(_ModelWithLogitsToKeep()) == {"logits_to_keep": 1}
    assert _prefill_logits_kwargs(_ModelWithoutLogitsToKeep()) == {}


def test_chunked_prefill_uses_logits_to_keep_when_supported():
    model = _ModelWithLogitsToKeep()
    cache = _FakeCache()
    logits = _installed(model).chunked_prefill(torch.ones(1, 5, dtype=torch.long), cache, chunk_size=2)
    assert model.calls == [1, 1, 1] and logits.shape == (1, 3) and cache.marked


def test_chunked_prefill_falls_back_for_unsupported_models():
    model = _ModelWithoutLogitsToKeep()
    cache = _FakeCache()
    logits = _installed(model).chunked_prefill(torch.ones(1, 5, dtype=torch.long), cache, chunk_size=2)
    assert model.calls == 3 and logits.shape == (1, 3) and cache.marked


def test_chunked_prefill_with_cap_evicts_between_chunks():
    model = _ModelWithLogitsToKeep()
    cache = _FakeCache()
    _installed(model).chunked_prefill(torch.ones(1, 5, dtype=torch.long), cache, chunk_size=2, prefill_hot_cap=3)
    assert cache.evict_calls == [3, 3, 3] and cache._prefill_complete and cache.evicted_excess
    assert not cache.marked and cache._suppress_cold is False


def test_chunked_prefill_empty_cache_is_opt_in(monkeypatch):
    calls = []
    monkeypatch.setattr(torch.cuda, "empty_cache", lambda: calls.append(True))
    _installed(_ModelWithLogitsToKeep()).chunked_prefill(torch.ones(1, 10, dtype=torch.long), _FakeCache(),
                                                        chunk_size=1)
    assert calls == []
    _installed(_ModelWithLogitsToKeep()).chunked_prefill(torch.ones(1, 5, dtype=torch.long), _FakeCache(),
                                                        chunk_size=1, empty_cache_interval=2)
    assert calls == [True, True]


def test_chunked_prefill_restores_wrapper_on_error():
    model = _RaisingModel()
    mw = _installed(model)
    cache = _FakeCache()
    with pytest.raises(RuntimeError, match="boom"):
        mw.chunked_prefill(torch.ones(1, 5, dtype=torch.long), cache, chunk_size=2, prefill_hot_cap=4)
    # The wrapper stays registered; its no-retrieval mode and the cache flag are reset.
    assert not hasattr(model.config, "_attn_implementation")
    assert mw._prefilling is False and cache._suppress_cold is False


def test_chunked_prefill_requires_install():
    with pytest.raises(RuntimeError, match="install"):
        KIVMiddleware(_ModelWithLogitsToKeep()).chunked_prefill(torch.ones(1, 2, dtype=torch.long), _FakeCache())
    with pytest.raises(RuntimeError, match="install"):
        KIVMiddleware(_ModelWithLogitsToKeep()).create_cache()


# ------------------------------------------------- detection on a real model
def _tiny_qwen2(attn="eager"):
    from transformers import Qwen2Config, Qwen2ForCausalLM

    cfg = Qwen2Config(vocab_size=97, hidden_size=64, intermediate_size=128, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=512)
    cfg._attn_implementation = attn
    torch.manual_seed(0)
    return Qwen2ForCausalLM(cfg).eval()


def test_detect_topology_qwen2():
    from kiv_amd import detect_topology

    t = detect_topology(_tiny_qwen2())
    assert t.model_family == "qwen2" and t.global_layer_indices == (0, 1)
    assert (t.num_query_heads, t.num_kv_heads, t.head_dim) == (4, 2, 16)
    assert t.kv_sharing_map == {}


def test_detect_topology_layer_types_and_sharing():
    from kiv_amd.hf_topology import detect_topology

    layers = [SimpleNamespace(self_attn=SimpleNamespace()) for _ in range(6)]
    cfg = SimpleNamespace(model_type="gemma3n_text", num_hidden_layers=6, num_attention_heads=8,
                          num_key_value_heads=2, head_dim=32, hidden_size=256,
                          layer_types=["sliding_attention", "full_attention"] * 3, num_kv_shared_layers=2)
    model = SimpleNamespace(config=cfg, model=SimpleNamespace(layers=layers))
    t = detect_topology(model)
    assert t.global_layer_indices == (1, 3, 5)
    assert t.independent_kv_layers == (1, 3) and t.kv_sharing_map == {5: 3}
    assert t.model_family == "gemma3n"


def test_install_registers_and_uninstall_restores():
    from transformers.masking_utils import ALL_MASK_ATTENTION_FUNCTIONS
    from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS

    for impl in ("eager", "sdpa"):
        model = _tiny_qwen2(impl)
        mw = KIVMiddleware(model, KIVConfig(hot_budget=8))
        mw.install()
        key = f"kiv_{impl}"
        assert model.config._attn_implementation == key and key in ALL_ATTENTION_FUNCTIONS
        if impl in ALL_MASK_ATTENTION_FUNCTIONS:
            assert key in ALL_MASK_ATTENTION_FUNCTIONS._global_mapping
        cache = mw.create_cache(torch.device("cpu"))
        assert model.model.layers[1].self_attn._kiv_cache is cache
        # Prefill-length forward with no cold tokens goes through the original attention.
        with torch.no_grad():
            out = model(input_ids=torch.arange(12)[None] % 97, past_key_values=cache, use_cache=True)
        assert out.logits.shape == (1, 12, 97)
        mw.uninstall()
        assert model.config._attn_implementation == impl and key not in ALL_ATTENTION_FUNCTIONS
        assert not hasattr(model.model.layers[0].self_attn, "_kiv_cache")


def test_hot_layer_appends_in_place_and_evicts_by_moving_the_start():
    """The buffered hot window (kiv_amd.tiered_cache._HotLayer) behaves as
    DynamicLayer.update + slice eviction would, copying only new rows."""
    from kiv_amd.tiered_cache import _HotLayer

    g = torch.Generator().manual_seed(0)
    rows = lambda n: torch.randn(1, 2, n, 8, generator=g)
    layer = _HotLayer()
    k0, v0 = rows(5), rows(5)
    keys, values = layer.update(k0, v0)
    ref_k, ref_v = k0.clone(), v0.clone()
    assert torch.equal(keys, ref_k) and torch.equal(values, ref_v)
    base = layer._kb.data_ptr()
    for step in range(300):  # crosses the buffer's slack: one move to a new buffer
        k1, v1 = rows(1), rows(1)
        keys, values = layer.update(k1, v1)
        ref_k, ref_v = torch.cat([ref_k, k1], 2), torch.cat([ref_v, v1], 2)
        layer.drop_front(1)
        ref_k, ref_v = ref_k[:, :, 1:], ref_v[:, :, 1:]
        assert torch.equal(layer.keys, ref_k) and torch.equal(layer.values, ref_v)
        assert keys.stride(3) == 1 and layer.get_seq_length() == 5
    assert layer._kb.data_ptr() != base
    # A replacement from outside (crop, truncation) is adopted at the next update.
    layer.crop(-2)
    ref_k, ref_v = ref_k[:, :, :-2], ref_v[:, :, :-2]
    k2, v2 = rows(4), rows(4)
    layer.update(k2, v2)
    assert torch.equal(layer.keys, torch.cat([ref_k, k2], 2)) and torch.equal(layer.values, torch.cat([ref_v, v2], 2))


def test_hot_layer_defers_only_rows_the_retrieval_can_copy():
    """A deferred update leaves rows for the retrieval's copy only when it
    can take them (the window's dtype, unit stride over head_dim, 16-byte
    aligned starts and strides); anything else is written at once, so a
    reader of the returned view sees it."""
    from kiv_amd.tiered_cache import _HotLayer

    g = torch.Generator().manual_seed(1)
    layer = _HotLayer()
    layer.update(torch.randn(1, 2, 4, 8, generator=g), torch.randn(1, 2, 4, 8, generator=g))
    ok_k, ok_v = torch.randn(1, 2, 1, 8, generator=g), torch.randn(1, 2, 1, 8, generator=g)
    layer.defer_append = True
    layer.update(ok_k, ok_v)
    assert layer._pending_rows is not None      # left to the retrieval
    layer.flush()
    assert torch.equal(layer.keys[:, :, -1:], ok_k) and torch.equal(layer.values[:, :, -1:], ok_v)
    wide = torch.randn(1, 2, 1, 9, generator=g)
    cases = {
        "head_dim stride 2": (torch.randn(1, 2, 1, 16, generator=g)[..., ::2], ok_v),
        "start off 16 bytes": (wide[..., 1:], ok_v),
        "row stride not a 16-byte multiple": (torch.randn(1, 2, 9, 1, generator=g).transpose(2, 3)[..., :8], ok_v),
        "other dtype": (ok_k.double(), ok_v),
    }
    for name, (k, v) in cases.items():
        layer.defer_append = True
        layer.update(k, v)
        assert layer._pending_rows is None, name   # written at once
        assert torch.equal(layer.keys[:, :, -1:], k.to(layer.keys.dtype)), name
        assert torch.equal(layer.values[:, :, -1:], v), name


def test_tiered_cache_uses_buffered_hot_layers_for_owned_layers():
    from transformers import Qwen2Config

    from kiv_amd.tiered_cache import _HotLayer

    cfg = Qwen2Config(hidden_size=64, num_attention_heads=4, num_key_value_heads=2, num_hidden_layers=3,
                      intermediate_size=128, vocab_size=100)
    topo = ModelTopology.manual(global_layer_indices=(0, 2), num_query_heads=4, num_kv_heads=2, head_dim=16,
                                num_hidden_layers=3)
    cache = TieredKVCache(cfg, KIVConfig(), topo, device="cpu")
    assert isinstance(cache.layers[0], _HotLayer) and isinstance(cache.layers[2], _HotLayer)
    assert not isinstance(cache.layers[1], _HotLayer)


def test_missing_mask_rule_follows_the_original_attention():
    """What a None mask means for a query of many positions: SDPA's is_causal
    (taken only when the query and key counts agree, where its top-left
    alignment and the cache's bottom-right one coincide), nothing for eager."""
    from types import SimpleNamespace

    from kiv_amd.middleware import _none_mask_rule

    causal_module, plain_module = SimpleNamespace(is_causal=True), SimpleNamespace(is_causal=False)
    assert _none_mask_rule("sdpa", causal_module, 64, 64) == "causal"
    assert _none_mask_rule("sdpa", causal_module, 64, 96) is None
    assert _none_mask_rule("sdpa", plain_module, 64, 96) == "none"
    assert _none_mask_rule("eager", causal_module, 64, 96) == "none"
    assert _none_mask_rule("flash_attention_2", causal_module, 64, 64) is None


def test_detect_topology_gemma4_per_layer_geometry():
    """Gemma4 keeps its full-attention layers' head_dim and kv heads in
    per_layer_config: detection reads them there, and the kv-shared
    full-attention layer maps to the last owning one, as in the topology
    the reference's golden run used (tests/golden/manifest.json)."""
    import json
    import os

    from transformers import Gemma4TextConfig
    from transformers.models.gemma4.modeling_gemma4 import Gemma4ForCausalLM

    from kiv_amd import detect_topology

    here = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
    with open(os.path.join(here, "manifest.json")) as f:
        meta = json.load(f)["tiny_gemma4_shared"]
    model = Gemma4ForCausalLM(Gemma4TextConfig(**meta["config"]))
    t = detect_topology(model)
    top = meta["topology"]
    assert t.global_layer_indices == tuple(top["global_layer_indices"])
    assert t.independent_kv_layers == tuple(top["independent_kv_layers"])
    assert t.kv_sharing_map == {int(k): v for k, v in top["kv_sharing_map"].items()}
    assert (t.num_query_heads, t.num_kv_heads, t.head_dim) == (top["num_query_heads"], top["num_kv_heads"],
                                                                top["head_dim"])
