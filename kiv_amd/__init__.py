"""kiv_amd -- the tiered KV cache decode path as hand-written gfx950 HIP kernels.

Same import surface as the reference package ``kiv`` (kiv/__init__.py:5-35):
``KIVConfig``, ``ColdKVStore`` and ``ModelTopology`` eagerly; ``detect_topology``,
``TieredKVCache`` and ``KIVMiddleware`` on first access (they import
transformers).
"""

__version__ = "0.1.0"

from .config import KIVConfig
from .cold_store import ColdKVStore
from .model_topology import ModelTopology

__all__ = [
    "KIVConfig",
    "ColdKVStore",
    "ModelTopology",
    "detect_topology",
    "TieredKVCache",
    "KIVMiddleware",
]

_LAZY = {
    "detect_topology": (".hf_topology", "detect_topology"),
    "TieredKVCache": (".tiered_cache", "TieredKVCache"),
    "KIVMiddleware": (".middleware", "KIVMiddleware"),
}


def __getattr__(name: str):
    if name in _LAZY:
        import importlib

        mod, attr = _LAZY[name]
        value = getattr(importlib.import_module(mod, __name__), attr)
        globals()[name] = value
        return value
    raise AttributeError(f"module 'kiv_amd' has no attribute {name!r}")
