"""Installs the tiered cache into a HuggingFace model.

Drop-in for the reference's ``KIVMiddleware`` (kiv/middleware.py:43-356):
``install`` registers a wrapper under ``ALL_ATTENTION_FUNCTIONS["kiv_<impl>"]``
(mirroring the mask function), ``create_cache`` / ``activate_cache`` bind a
:class:`TieredKVCache` to the global attention modules and
``chunked_prefill`` runs long prompts chunk by chunk without retrieval.  At
decode the wrapper retrieves the top-P cold K/V with the HIP kernels and,
for single-position queries, runs one merged softmax over [retrieved ; hot]
(``ColdKVStore.retrieve_attend``) instead of concatenating and
calling the original attention.  Queries of many positions (prefill chunks,
and long queries with a cold tier) run on the matrix-core attention
(:func:`kiv_amd.attention.prefill_attention`).  Shapes the kernels do not
cover take the reference's route: concatenate, widen the mask, call the
original attention function.
"""

from __future__ import annotations

import importlib
import inspect
import logging
from typing import Any

import torch
from transformers.masking_utils import ALL_MASK_ATTENTION_FUNCTIONS
from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS

from .attention import fused_supported, prefill_attention, prefill_supported
from .config import KIVConfig
from .hf_topology import _find_text_model, detect_topology
from .mask_utils import extend_mask_for_cold
from .model_topology import ModelTopology
from .tiered_cache import TieredKVCache

logger = logging.getLogger(__name__)

_extend_mask_for_cold = extend_mask_for_cold


def _prefill_logits_kwargs(model: Any, logits_to_keep: int = 1) -> dict[str, int]:
    """``{"logits_to_keep": n}`` when the model's forward accepts it, else ``{}``
    (kiv/middleware.py:22-37)."""
    try:
        params = inspect.signature(model.forward).parameters
    except (TypeError, ValueError, AttributeError):
        return {}
    return {"logits_to_keep": logits_to_keep} if "logits_to_keep" in params else {}


def _plain_softmax(module, kwargs) -> bool:
    """The HIP attention kernels reproduce plain softmax attention only: no
    dropout, soft-capping or attention sinks."""
    if kwargs.get("dropout", 0.0) and getattr(module, "training", False):
        return False
    return kwargs.get("softcap") is None and kwargs.get("s_aux") is None and kwargs.get("sinks") is None


def _merged_kernel_applies(module, query, key, mask, kwargs) -> bool:
    return _plain_softmax(module, kwargs) and fused_supported(query, key, mask)


def _none_mask_rule(impl: str | None, module, q_len: int, kv_len: int) -> str | None:
    """What a missing mask means to the original attention for a query of
    q_len positions over kv_len keys: "causal" (SDPA's is_causal, which HF
    sets when the mask is None; top-left aligned, so only q_len == kv_len is
    taken here), "none" (eager adds no mask), or None (not handled)."""
    if impl == "eager":
        return "none"
    if impl == "sdpa":
        if not getattr(module, "is_causal", True):
            return "none"
        return "causal" if q_len == kv_len else None
    return None


def _write_rows(rows) -> None:
    """Write hot rows a decode update left unwritten (src_k, src_v, dst_k, dst_v)."""
    if rows is not None:
        rows[2].copy_(rows[0])
        rows[3].copy_(rows[1])


class KIVMiddleware:

    def __init__(self, model: Any, config: KIVConfig | None = None, topology: ModelTopology | None = None) -> None:
        self.model = model
        self.config = config or KIVConfig()
        self._topology_override = topology
        self.topology: ModelTopology | None = None
        self._text_model: Any = None
        self._installed = False
        self._original_impl: str | None = None
        self._kiv_key: str | None = None
        self._prefilling = False  # chunked_prefill: the wrapper attends without retrieval

    # -------------------------------------------------------------- install
    def install(self) -> None:
        """Detect the topology, tag global layers, register the wrapper
        (kiv/middleware.py:60-106)."""
        if self._installed:
            logger.warning("KIV middleware already installed.")
            return
        self.topology = self._topology_override or detect_topology(self.model)
        self._text_model = _find_text_model(self.model)
        for i in self.topology.global_layer_indices:
            self._text_model.layers[i].self_attn._kiv_layer_idx = i
        self._original_impl = self._resolve_attn_impl()
        original = self._get_attn_fn(self._original_impl)
        self._kiv_key = f"kiv_{self._original_impl}"
        ALL_ATTENTION_FUNCTIONS[self._kiv_key] = self._make_kiv_attention(original)
        # The mask preprocessing looks the implementation up in _global_mapping.
        if self._original_impl in ALL_MASK_ATTENTION_FUNCTIONS:
            ALL_MASK_ATTENTION_FUNCTIONS._global_mapping[self._kiv_key] = (
                ALL_MASK_ATTENTION_FUNCTIONS[self._original_impl])
        self._set_attn_impl(self._kiv_key)
        self._installed = True
        logger.info("KIV installed: %d global layers (%d independent, %d shared), attn=%s, hot=%d, top_p=%d",
                    len(self.topology.global_layer_indices), len(self.topology.independent_kv_layers),
                    len(self.topology.kv_sharing_map), self._original_impl, self.config.hot_budget,
                    self.config.top_p)

    def uninstall(self) -> None:
        """Restore the original attention and drop the registrations
        (kiv/middleware.py:108-134)."""
        if not self._installed:
            return
        prev = getattr(self, "_active_cache", None)
        if prev is not None:
            prev.flush_hot()
            prev._defer_hot_append = False
            self._active_cache = None
        if self._original_impl is not None:
            self._set_attn_impl(self._original_impl)
        if self._kiv_key is not None:
            if self._kiv_key in ALL_ATTENTION_FUNCTIONS:
                del ALL_ATTENTION_FUNCTIONS[self._kiv_key]
            ALL_MASK_ATTENTION_FUNCTIONS._global_mapping.pop(self._kiv_key, None)
        if self._text_model is not None and self.topology is not None:
            for i in self.topology.global_layer_indices:
                attn = self._text_model.layers[i].self_attn
                for attr in ("_kiv_layer_idx", "_kiv_cache"):
                    if hasattr(attn, attr):
                        delattr(attn, attr)
        self._installed = False
        self._original_impl = None
        self._kiv_key = None

    # ---------------------------------------------------------------- caches
    def create_cache(self, device: torch.device | None = None) -> TieredKVCache:
        """New :class:`TieredKVCache`, bound as the active cache."""
        if self.topology is None:
            raise RuntimeError("Call install() before create_cache().")
        if device is None:
            device = next(self.model.parameters()).device
        cache = TieredKVCache(config=self.model.config, kiv_config=self.config, topology=self.topology,
                              device=device)
        self.activate_cache(cache)
        return cache

    def activate_cache(self, cache: TieredKVCache | None) -> None:
        """Point the wrapper of every global layer at ``cache`` (or unbind).

        The active cache's decode updates leave each owned layer's new hot
        rows to that layer's retrieval, which writes them in its first
        launch (the wrapper below always takes them); a cache that stops
        being active writes any such rows and stops deferring."""
        if self.topology is None or self._text_model is None:
            return
        prev = getattr(self, "_active_cache", None)
        if prev is not None and prev is not cache:
            prev.flush_hot()
            prev._defer_hot_append = False
        for i in self.topology.global_layer_indices:
            attn = self._text_model.layers[i].self_attn
            if cache is None:
                if hasattr(attn, "_kiv_cache"):
                    delattr(attn, "_kiv_cache")
            else:
                attn._kiv_cache = cache
        if cache is not None:
            cache._defer_hot_append = True
        self._active_cache = cache

    # --------------------------------------------------------------- prefill
    def chunked_prefill(self, input_ids: torch.Tensor, cache: TieredKVCache, chunk_size: int = 4096,
                        prefill_hot_cap: int | None = None, empty_cache_interval: int | None = None) -> torch.Tensor:
        """Prefill ``input_ids`` [B, T] in chunks; returns last-token logits [B, vocab].

        Same control flow as kiv/middleware.py:174-260: plain attention over
        the hot window for every chunk (no retrieval during prefill); with
        ``prefill_hot_cap`` the hot windows are trimmed to the cap after each
        chunk; the wrapper is restored even when a forward raises; finally
        the hot windows are trimmed to ``hot_budget``.  Where the reference
        switches to the original attention function, the wrapper stays
        installed in a no-retrieval mode and runs the chunk's attention on
        the matrix-core kernel (kiv_prefill_attention), falling back to the
        original function for shapes the kernel does not cover.
        """
        if not self._installed:
            raise RuntimeError("Call install() before chunked_prefill().")
        total = input_ids.shape[1]
        logits = None
        extra = _prefill_logits_kwargs(self.model, logits_to_keep=1)
        if prefill_hot_cap is not None:
            cache._suppress_cold = True
        self._prefilling = True
        try:
            for n, start in enumerate(range(0, total, chunk_size)):
                end = min(start + chunk_size, total)
                with torch.no_grad():
                    out = self.model(input_ids=input_ids[:, start:end], past_key_values=cache, use_cache=True,
                                     **extra)
                if end == total:
                    logits = out.logits[:, -1, :]
                del out
                if prefill_hot_cap is not None:
                    cache._evict_to_cap(prefill_hot_cap)
                if empty_cache_interval and empty_cache_interval > 0 and (n + 1) % empty_cache_interval == 0:
                    torch.cuda.empty_cache()
        finally:
            cache._suppress_cold = False
            self._prefilling = False
        if prefill_hot_cap is None:
            cache.mark_prefill_complete()
        else:
            cache._prefill_complete = True
            cache._evict_excess_all_layers()
        return logits

    # --------------------------------------------------------------- helpers
    def _resolve_attn_impl(self) -> str:
        cfg = self.model.config
        cfg = getattr(cfg, "text_config", cfg)
        return getattr(cfg, "_attn_implementation", "eager")

    def _get_attn_fn(self, impl: str) -> Any:
        if impl in ALL_ATTENTION_FUNCTIONS:
            return ALL_ATTENTION_FUNCTIONS[impl]
        attn = self._text_model.layers[self.topology.global_layer_indices[0]].self_attn
        fn = getattr(importlib.import_module(type(attn).__module__), "eager_attention_forward", None)
        if fn is None:
            raise ValueError(f"Cannot find attention function for implementation '{impl}'")
        return fn

    def _set_attn_impl(self, impl: str) -> None:
        cfg = self.model.config
        if hasattr(cfg, "text_config"):
            cfg.text_config._attn_implementation = impl
        cfg._attn_implementation = impl

    def _make_kiv_attention(self, original_fn: Any) -> Any:
        """The registered attention function (kiv/middleware.py:295-356)."""
        kiv_config = self.config
        sample = self._text_model.layers[self.topology.global_layer_indices[0]].self_attn
        fallback_scaling = getattr(sample, "scaling", None)
        if fallback_scaling is None:
            fallback_scaling = self.topology.head_dim ** -0.5

        middleware = self
        impl = self._original_impl

        def dense_attention(module, query, key, value, attention_mask, kwargs):
            """Attention over the given keys only: the matrix-core kernel for
            queries of many positions, the original function otherwise."""
            T = key.shape[2]
            if attention_mask is not None and attention_mask.shape[-1] != T:
                # Eager attention uses the mask's first T columns; other
                # implementations take the mask as it is.
                if impl != "eager" or attention_mask.shape[-1] < T:
                    return original_fn(module, query, key, value, attention_mask, **kwargs)
                attention_mask = attention_mask[..., :T]
            if (query.shape[2] > 1 and kwargs.get("sliding_window") is None and _plain_softmax(module, kwargs)
                    and prefill_supported(query, key, attention_mask)):
                rule = None if attention_mask is not None else _none_mask_rule(impl, module, query.shape[2], T)
                if attention_mask is not None or rule is not None:
                    scaling = kwargs.get("scaling")
                    if scaling is None:
                        scaling = getattr(module, "scaling", None) or fallback_scaling
                    out = prefill_attention(query, None, None, key, value, attention_mask, scaling,
                                            causal=rule == "causal")
                    return out, None
            return original_fn(module, query, key, value, attention_mask, **kwargs)

        def kiv_attention(module, query, key, value, attention_mask, **kwargs):
            cache = getattr(module, "_kiv_cache", None)
            layer_idx = getattr(module, "_kiv_layer_idx", None)
            # Hot rows this layer's update left unwritten: the fused call
            # below writes them in its first launch; every other path writes
            # them here first.
            pend = cache.take_hot_rows(layer_idx) if cache is not None and layer_idx is not None else None
            if (middleware._prefilling or cache is None or layer_idx is None
                    or getattr(cache, "_suppress_cold", False)):
                _write_rows(pend)
                return dense_attention(module, query, key, value, attention_mask, kwargs)
            store = cache.get_cold_store(layer_idx)
            if store is None or store.cold_length == 0:
                _write_rows(pend)
                return dense_attention(module, query, key, value, attention_mask, kwargs)
            scaling = kwargs.get("scaling")
            if scaling is None:
                scaling = fallback_scaling
            step = getattr(cache, "_decode_step", -1)
            hot_len = key.shape[2]
            # The mask was built before this step's eviction: keep its last hot_len columns.
            if attention_mask is not None and attention_mask.shape[-1] > hot_len:
                attention_mask = attention_mask[..., -hot_len:]
            if _merged_kernel_applies(module, query, key, attention_mask, kwargs):
                # Retrieval and the merged attention in one call (hot-window
                # splits overlap the retrieval's gather).
                try:
                    out = store.retrieve_attend(query, scaling, kiv_config, key, value, attention_mask, step=step,
                                                hot_rows=pend)
                except BaseException:
                    _write_rows(pend)
                    raise
                return out.to(query.dtype), None
            _write_rows(pend)
            cold_k, cold_v = store.retrieve_top_kv(query, scaling, kiv_config, step=step)
            if cold_k is None:
                return dense_attention(module, query, key, value, attention_mask, kwargs)
            if (attention_mask is not None and query.shape[2] > 1 and _plain_softmax(module, kwargs)
                    and prefill_supported(query, key, attention_mask)):
                # A query of many positions: one matrix-core pass over
                # [retrieved ; hot], the mask applying to the hot columns.
                out = prefill_attention(query, cold_k, cold_v, key, value, attention_mask, scaling)
                return out, None
            key = torch.cat([cold_k, key], dim=2)
            value = torch.cat([cold_v, value], dim=2)
            if attention_mask is not None:
                attention_mask = extend_mask_for_cold(attention_mask, cold_k.shape[2])
            return original_fn(module, query, key, value, attention_mask, **kwargs)

        return kiv_attention
