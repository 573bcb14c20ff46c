"""Derive a :class:`ModelTopology` from a loaded HuggingFace model.

Detection rules follow the reference's ``detect_topology``
(kiv/hf_topology.py:166-225):
  * text model: ``model.model.language_model`` / ``.text_model`` / ``model.model``
    (kiv/hf_topology.py:21-37);
  * global layers from ``layer_types == "full_attention"``, else every layer
    (kiv/hf_topology.py:40-73);
  * KV sharing from ``num_kv_shared_layers`` or per-module
    ``is_kv_shared_layer`` / ``kv_shared_layer_index`` (kiv/hf_topology.py:76-122);
  * head geometry preferring the global-layer fields (kiv/hf_topology.py:125-143).
"""

from __future__ import annotations

import logging
from typing import Any

from .model_topology import ModelTopology

logger = logging.getLogger(__name__)

_FAMILY = {
    "gemma4_text": "gemma4", "gemma4": "gemma4",
    "gemma3_text": "gemma3", "gemma3": "gemma3",
    "gemma3n_text": "gemma3n", "gemma3n": "gemma3n",
    "gemma2": "gemma2", "gemma": "gemma",
    "llama": "llama", "mistral": "mistral",
    "cohere2": "cohere2", "cohere": "cohere",
    "phi3": "phi3", "phi": "phi", "qwen2": "qwen2",
}


def _text_config(model: Any) -> Any:
    cfg = model.config
    return cfg.text_config if hasattr(cfg, "text_config") else cfg


def _find_text_model(model: Any) -> Any:
    inner = getattr(model, "model", None)
    if inner is not None:
        for name in ("language_model", "text_model"):
            cand = getattr(inner, name, None)
            if cand is not None and hasattr(cand, "layers"):
                return cand
        if hasattr(inner, "layers"):
            return inner
    raise AttributeError(
        "Cannot find text model layers. "
        "Supported: model.model.language_model, model.model.text_model, model.model"
    )


def _global_layers(cfg: Any) -> tuple[int, ...]:
    n = cfg.num_hidden_layers
    kinds = getattr(cfg, "layer_types", None)
    if kinds is not None:
        full = tuple(i for i, kind in enumerate(kinds) if kind == "full_attention")
        if full:
            return full
        logger.warning("layer_types has no 'full_attention' entry; all %d layers are global.", n)
    return tuple(range(n))


def _kv_sharing(cfg: Any, model: Any, globals_: tuple[int, ...]):
    shared = getattr(cfg, "num_kv_shared_layers", 0) or 0
    if shared > 0:
        first_shared = cfg.num_hidden_layers - shared
        owners = tuple(i for i in globals_ if i < first_shared)
        if not owners:
            return globals_, {}
        return owners, {i: owners[-1] for i in globals_ if i >= first_shared}
    try:
        layers = _find_text_model(model).layers
        owners, sharing = [], {}
        for i in globals_:
            attn = layers[i].self_attn
            src = getattr(attn, "kv_shared_layer_index", None)
            if getattr(attn, "is_kv_shared_layer", False) and src is not None:
                sharing[i] = src
            else:
                owners.append(i)
        if sharing:
            return tuple(owners), sharing
    except (AttributeError, IndexError):
        pass
    return globals_, {}


def _first_attr(cfg: Any, names: tuple[str, ...]):
    for name in names:
        try:
            val = getattr(cfg, name, None)
        except Exception:  # a per-layer attribute of a heterogeneous config
            val = None
        if val is not None:
            return val
    return None


def _head_geometry(cfg: Any, global_layers: tuple[int, ...] = ()) -> tuple[int, int, int]:
    """(Hq, Hkv, D) of the global layers (kiv/hf_topology.py:130-150).

    Configs whose attention geometry varies per layer (Gemma4 in
    transformers 5.x keeps ``head_dim`` and the kv head count of its
    full-attention layers in ``per_layer_config``) are read at the first
    global layer."""
    hq = cfg.num_attention_heads
    layer_cfg = None
    per_layer = getattr(cfg, "per_layer_config", None)
    if per_layer is not None and global_layers:
        try:
            layer_cfg = per_layer[global_layers[0]]
        except (KeyError, IndexError, TypeError):
            layer_cfg = None
    hkv = _first_attr(cfg, ("num_global_key_value_heads",))
    if hkv is None and layer_cfg is not None:
        hkv = _first_attr(layer_cfg, ("num_key_value_heads",))
    hkv = hkv or _first_attr(cfg, ("num_key_value_heads",)) or hq
    d = _first_attr(cfg, ("global_head_dim",))
    if d is None and layer_cfg is not None:
        d = _first_attr(layer_cfg, ("head_dim",))
    d = d or _first_attr(cfg, ("head_dim",)) or cfg.hidden_size // hq
    return hq, hkv, d


def detect_topology(model: Any) -> ModelTopology:
    """Inspect ``model`` and describe the layers the tiered cache manages."""
    cfg = _text_config(model)
    model_type = getattr(cfg, "model_type", "unknown")
    family = _FAMILY.get(model_type)
    if family is None:
        logger.warning(
            "Unknown model_type '%s'; treating all layers as global with no KV sharing.",
            model_type,
        )
        family = model_type
    globals_ = _global_layers(cfg)
    owners, sharing = _kv_sharing(cfg, model, globals_)
    hq, hkv, d = _head_geometry(cfg, globals_)
    topo = ModelTopology(
        model_family=family,
        num_hidden_layers=cfg.num_hidden_layers,
        global_layer_indices=globals_,
        independent_kv_layers=owners,
        kv_sharing_map=sharing,
        num_query_heads=hq,
        num_kv_heads=hkv,
        head_dim=d,
    )
    logger.info(
        "KIV topology for %s: %d global layers (%d independent, %d shared), Hq=%d Hkv=%d D=%d",
        family, len(globals_), len(owners), len(sharing), hq, hkv, d,
    )
    return topo
