"""Hot window + cold tier cache for HuggingFace models.

Drop-in for the reference's ``TieredKVCache`` (kiv/tiered_cache.py:17-286):
still a ``transformers.DynamicCache`` so HF layers and callers that read
``layers[i].keys`` keep working.  Global layers that own KV keep at most
``hot_budget`` recent tokens after prefill; older rows go to the layer's
:class:`ColdKVStore`.  Positions (``get_seq_length``) and mask sizes count
hot + cold tokens.

The hot window of an owned layer lives in a preallocated buffer with slack
(:class:`_HotLayer`): a decode step writes its one new row in place and an
eviction moves the window's start, where DynamicLayer's ``torch.cat`` and
the reference's slice-and-``.contiguous()`` eviction each copy the whole
window (kiv/tiered_cache.py:55-72).  ``layers[i].keys`` is then a view of
the buffer ([B, H, T, D], unit stride over D).
"""

from __future__ import annotations

import logging

import torch
from transformers import DynamicCache
from transformers.cache_utils import DynamicLayer

from . import persist
from .cold_store import ColdKVStore
from .config import KIVConfig
from .model_topology import ModelTopology

logger = logging.getLogger(__name__)


class _HotLayer(DynamicLayer):
    """A DynamicLayer whose rows [start, end) live in [B, H, cap, D] buffers.

    ``update`` copies only the new rows (at ``end``); ``drop_front`` evicts by
    advancing ``start``.  When an append would run past ``cap``, the window
    moves to a fresh buffer with ``slack`` free rows (one copy per ``slack``
    appended rows in decode).  Any other code that replaces ``keys`` /
    ``values`` (crop, batch selection, truncation) is picked up at the next
    update, which copies the replacement into a new buffer.

    With ``defer_append`` set (by the cache, for one decode update under the
    middleware), update leaves the new rows unwritten: the layer's attention
    takes them (``take_pending``) and the retrieval's first launch writes
    them, or writes them itself (``flush``).
    """

    slack = 256

    def __init__(self) -> None:
        super().__init__()
        self._kb = self._vb = None
        self._start = self._end = 0
        self._view = None
        self._pending_rows = None  # (src_k, src_v, first row, n) not written yet
        self.defer_append = False

    def flush(self) -> None:
        """Write rows an update left unwritten."""
        p = self._pending_rows
        if p is not None:
            self._pending_rows = None
            k, v, e, n = p
            self._kb[:, :, e:e + n].copy_(k)
            self._vb[:, :, e:e + n].copy_(v)

    def take_pending(self):
        """(src_k, src_v, dst_k, dst_v) of the rows the last update left
        unwritten, or None; the caller writes them before anything reads
        the window."""
        p = self._pending_rows
        if p is None:
            return None
        self._pending_rows = None
        k, v, e, n = p
        return k, v, self._kb[:, :, e:e + n], self._vb[:, :, e:e + n]

    def _window(self) -> None:
        self.keys = self._kb[:, :, self._start:self._end]
        self.values = self._vb[:, :, self._start:self._end]
        self._view = self.keys

    def _move(self, k: torch.Tensor, v: torch.Tensor, extra: int) -> None:
        """New buffers holding k / v at the front, with room for ``extra`` more rows."""
        B, H, T, D = k.shape
        cap = T + extra + self.slack
        kb = torch.empty(B, H, cap, D, dtype=k.dtype, device=k.device)
        vb = torch.empty(B, H, cap, v.shape[3], dtype=v.dtype, device=v.device)
        if T:
            kb[:, :, :T].copy_(k)
            vb[:, :, :T].copy_(v)
        self._kb, self._vb, self._start, self._end = kb, vb, 0, T

    def update(self, key_states: torch.Tensor, value_states: torch.Tensor, *args, **kwargs):
        self.flush()
        defer, self.defer_append = self.defer_append, False
        if not self.is_initialized:
            self.lazy_initialization(key_states, value_states)
        n = key_states.shape[-2]
        if self._kb is None or self.keys is not self._view:
            # First rows, or keys replaced from outside.
            k, v = self.keys, self.values
            if k.numel() == 0:
                k = key_states[:, :, :0]
                v = value_states[:, :, :0]
            self._move(k, v, n)
        elif (self._end + n > self._kb.shape[2] or key_states.shape[:2] != self._kb.shape[:2]
              or key_states.dtype != self._kb.dtype):
            self._move(self.keys, self.values, n)
        if defer and self._deferrable(key_states, value_states):
            self._pending_rows = (key_states, value_states, self._end, n)
        else:
            self._kb[:, :, self._end:self._end + n].copy_(key_states)
            self._vb[:, :, self._end:self._end + n].copy_(value_states)
        self._end += n
        self._window()
        return self.keys, self.values

    def _deferrable(self, k: torch.Tensor, v: torch.Tensor) -> bool:
        """Rows the retrieval's copy can take: the buffers' dtype, unit stride
        over head_dim, 16-byte aligned starts and strides (what kiv_retrieve
        accepts for hot-window rows); anything else is written at once."""
        if k.dtype != self._kb.dtype or v.dtype != self._vb.dtype:
            return False
        vec = 16 // k.element_size()
        for t in (k, v):
            if t.stride(-1) != 1 or t.data_ptr() % 16 or any(st % vec for st in t.stride()[:-1]):
                return False
        return True

    def drop_front(self, n: int) -> None:
        """Forget the oldest ``n`` rows (already copied to the cold tier)."""
        if self._kb is None or self.keys is not self._view:
            self.keys = self.keys[:, :, n:]
            self.values = self.values[:, :, n:]
            return
        self._start += n
        self._window()


class TieredKVCache(DynamicCache):

    def __init__(self, config, kiv_config: KIVConfig, topology: ModelTopology,
                 device: torch.device | None = None) -> None:
        super().__init__(config=config)
        self.kiv_config = kiv_config
        self.topology = topology
        device = torch.device("cuda") if device is None else torch.device(device)
        self.cold_stores: dict[int, ColdKVStore] = {
            i: ColdKVStore(kiv_config, topology, device) for i in topology.independent_kv_layers
        }
        # Owned full-attention layers keep their hot window in a buffer.
        for i in topology.independent_kv_layers:
            if i < len(self.layers) and type(self.layers[i]) is DynamicLayer:
                self.layers[i] = _HotLayer()
        self._prefill_complete = False   # eviction starts after prefill
        self._suppress_cold = False      # wrapper skips retrieval while set
        self._total_tokens: dict[int, int] = {}
        self._decode_step = 0            # shared-layer candidate reuse key
        # Set by the middleware while this cache is its active one: decode
        # updates of owned layers leave the new hot rows to the layer's
        # retrieval (see _HotLayer.defer_append).
        self._defer_hot_append = False

    # -------------------------------------------------------------- helpers
    def _kv_source_layer_idx(self, layer_idx: int) -> int:
        return self.topology.kv_sharing_map.get(layer_idx, layer_idx)

    def _owned_layers(self):
        """(index, layer) of independent layers that hold tensors."""
        for i in self.topology.independent_kv_layers:
            if i < len(self.layers) and self.layers[i].is_initialized:
                yield i, self.layers[i]

    def _evict_layer(self, layer_idx: int, num_evict: int, deferred: bool = False) -> None:
        """Move the oldest ``num_evict`` hot rows of a layer to its cold store
        (kiv/tiered_cache.py:55-72).  ``deferred``: the decode step's rows,
        written by the layer's retrieval that follows (their hot-window rows
        are never written again)."""
        layer = self.layers[layer_idx]
        store = self.cold_stores[layer_idx]
        evict = store.evict_deferred if deferred else store.evict_from_hot
        evict(layer.keys[:, :, :num_evict], layer.values[:, :, :num_evict])
        if isinstance(layer, _HotLayer):
            layer.drop_front(num_evict)
        else:
            layer.keys = layer.keys[:, :, num_evict:].contiguous()
            layer.values = layer.values[:, :, num_evict:].contiguous()
        self._total_tokens[layer_idx] = self.cold_stores[layer_idx].cold_length + layer.keys.shape[2]

    def _evict_to_cap(self, cap: int) -> None:
        """Bounded prefill: trim every owned hot window to ``cap`` tokens."""
        for i, layer in self._owned_layers():
            excess = layer.keys.shape[2] - cap
            if excess > 0:
                self._evict_layer(i, excess)

    def _evict_excess_all_layers(self) -> None:
        """Trim every owned hot window to ``hot_budget`` tokens."""
        budget = self.kiv_config.hot_budget
        for i, layer in self._owned_layers():
            excess = layer.keys.shape[2] - budget
            if excess > 0:
                self._evict_layer(i, excess)
                logger.debug("layer %d: evicted %d tokens (cold=%d)", i, excess,
                             self.cold_stores[i].cold_length)

    def mark_prefill_complete(self) -> None:
        self._prefill_complete = True
        self._evict_excess_all_layers()

    # ----------------------------------------------------------------- HF API
    def update(self, key_states: torch.Tensor, value_states: torch.Tensor, layer_idx: int, *args, **kwargs):
        """Append, then (after prefill) evict past ``hot_budget`` (kiv/tiered_cache.py:107-142).

        The token appended in this call stays hot; the evicted ones are
        already cold candidates for the same layer call.
        """
        if (self._defer_hot_append and self._prefill_complete and layer_idx in self.cold_stores
                and layer_idx < len(self.layers) and isinstance(self.layers[layer_idx], _HotLayer)
                and key_states.shape[-2] <= self.kiv_config.hot_budget):
            # The new rows outlive this step's eviction (it takes the oldest
            # hot_len - hot_budget rows), so their write can wait for the
            # layer's retrieval.
            self.layers[layer_idx].defer_append = True
        keys, values = super().update(key_states, value_states, layer_idx, *args, **kwargs)
        owned = self.topology.independent_kv_layers
        if layer_idx in owned:
            if self._prefill_complete and layer_idx == owned[0]:
                self._decode_step += 1
            self._total_tokens[layer_idx] = self.cold_stores[layer_idx].cold_length + keys.shape[2]
        if self._prefill_complete and layer_idx in self.cold_stores:
            layer = self.layers[layer_idx]
            excess = layer.keys.shape[2] - self.kiv_config.hot_budget
            if excess > 0:
                self._evict_layer(layer_idx, excess, deferred=True)
                keys, values = layer.keys, layer.values
        return keys, values

    def get_cold_store(self, layer_idx: int) -> ColdKVStore | None:
        """The store of ``layer_idx`` or of the layer it shares KV with."""
        if layer_idx in self.cold_stores:
            return self.cold_stores[layer_idx]
        src = self.topology.kv_sharing_map.get(layer_idx)
        return None if src is None else self.cold_stores.get(src)

    def get_mask_sizes(self, query_length: int, layer_idx: int) -> tuple[int, int]:
        """(hot + query length, cold length) once cold tokens exist
        (kiv/tiered_cache.py:156-168); parent behaviour otherwise."""
        store = self.get_cold_store(layer_idx)
        src = self._kv_source_layer_idx(layer_idx)
        if store is not None and src < len(self.layers) and store.cold_length > 0:
            layer = self.layers[src]
            hot = layer.get_seq_length() if layer.is_initialized else 0
            return hot + query_length, store.cold_length
        return super().get_mask_sizes(query_length, layer_idx)

    def get_seq_length(self, layer_idx: int = 0) -> int:
        """Hot + cold tokens, so position ids keep counting evicted tokens."""
        if layer_idx in self._total_tokens:
            return self._total_tokens[layer_idx]
        src = self._kv_source_layer_idx(layer_idx)
        if src in self._total_tokens:
            return self._total_tokens[src]
        return super().get_seq_length(src)

    def reset(self) -> None:
        self.flush_hot()
        super().reset()
        for store in self.cold_stores.values():
            store.reset()
        self._total_tokens.clear()
        self._prefill_complete = False
        self._suppress_cold = False
        self._decode_step = 0

    def truncate_to(self, new_len: int) -> bool:
        """Cut every owned layer back to ``new_len`` tokens, within the hot window only.

        Same rules as kiv/tiered_cache.py:194-257: False (cache untouched)
        when ``new_len`` exceeds the current total or falls inside the cold
        tier; otherwise hot K/V are sliced, the candidate caches cleared and
        the decode-step counter restarted.
        """
        self.flush_hot()
        owned = list(self._owned_layers())
        for i, layer in owned:
            cold = self.cold_stores[i].cold_length
            if new_len > cold + layer.keys.shape[2] or new_len < cold:
                return False
        for i, layer in owned:
            keep = new_len - self.cold_stores[i].cold_length
            if keep < layer.keys.shape[2]:
                layer.keys = layer.keys[:, :, :keep].contiguous()
                layer.values = layer.values[:, :, :keep].contiguous()
            self._total_tokens[i] = new_len
        for store in self.cold_stores.values():
            store._invalidate_candidates()
        self._decode_step = 0
        return True

    # ------------------------------------------------------------ persistence
    def take_hot_rows(self, layer_idx: int):
        """The hot rows layer ``layer_idx``'s last update left unwritten, as
        (src_k, src_v, dst_k, dst_v), or None; the caller writes them."""
        if layer_idx < len(self.layers) and isinstance(self.layers[layer_idx], _HotLayer):
            return self.layers[layer_idx].take_pending()
        return None

    def flush_hot(self) -> None:
        """Write every hot row a decode update left to its layer's retrieval."""
        for layer in self.layers:
            if isinstance(layer, _HotLayer):
                layer.flush()

    def save(self, path) -> None:
        """Write the whole cache to ``path``: every layer's hot K/V, every
        cold tier's rows, the token counts and the decode-step counter (the
        format in kiv_amd/persist.py).  No counterpart in the reference,
        whose cache lives in process memory only.  Layers other than plain
        full-attention layers (a sliding window's running state) are not
        stored: saving such a cache raises NotImplementedError."""
        self.flush_hot()
        entries = []
        for i, layer in enumerate(self.layers):
            if not layer.is_initialized or layer.keys is None or layer.keys.numel() == 0:
                entries.append({"index": i, "kind": "empty"})
                continue
            if type(layer) not in (DynamicLayer, _HotLayer):
                raise NotImplementedError(f"TieredKVCache.save: layer {i} is a {type(layer).__name__}; only "
                                          "full-attention layers (DynamicLayer) are stored")
            entries.append({"index": i, "kind": "kv", "dtype": persist.dtype_name(layer.keys.dtype),
                            "k_shape": list(layer.keys.shape), "v_shape": list(layer.values.shape)})
        header = {"format": "kiv-cache", "version": persist.VERSION, "num_layers": len(self.layers),
                  "prefill_complete": self._prefill_complete, "decode_step": self._decode_step,
                  "total_tokens": {str(i): n for i, n in self._total_tokens.items()},
                  "cold_layers": sorted(self.cold_stores), "layers": entries}
        with open(path, "wb") as f:
            persist.write_header(f, persist.CACHE_MAGIC, header)
            for e in entries:
                if e["kind"] == "kv":
                    layer = self.layers[e["index"]]
                    persist.write_tensor(f, layer.keys)
                    persist.write_tensor(f, layer.values)
            for i in sorted(self.cold_stores):
                self.cold_stores[i].save(f)

    def load(self, path) -> None:
        """Restore a cache written by :meth:`save` into this empty cache (one
        made for the same model and KIVConfig, e.g. by create_cache()).  Hot
        windows are appended as the model would append them; cold tiers are
        re-evicted in order, which rebuilds their pages and summaries bit
        for bit.  Telemetry starts empty."""
        if any(l.is_initialized and l.keys is not None and l.keys.numel() for l in self.layers) or \
                any(st.cold_length for st in self.cold_stores.values()):
            raise RuntimeError("TieredKVCache.load: the cache is not empty; reset() it first")
        device = next(iter(self.cold_stores.values())).device if self.cold_stores else torch.device("cuda")
        with open(path, "rb") as f:
            h = persist.read_header(f, persist.CACHE_MAGIC)
            if h["num_layers"] != len(self.layers) or sorted(h["cold_layers"]) != sorted(self.cold_stores):
                raise ValueError("TieredKVCache.load: the file was written for another layer layout "
                                 f"({h['num_layers']} layers, cold tiers {h['cold_layers']}; this cache: "
                                 f"{len(self.layers)} layers, cold tiers {sorted(self.cold_stores)})")
            for e in h["layers"]:
                if e["kind"] != "kv":
                    continue
                dtype = persist.dtype_of(e["dtype"])
                k = persist.read_tensor(f, tuple(e["k_shape"]), dtype, device)
                v = persist.read_tensor(f, tuple(e["v_shape"]), dtype, device)
                self.layers[e["index"]].update(k, v)
            for i in sorted(self.cold_stores):
                self.cold_stores[i].load(f, device)
        self._total_tokens = {int(i): n for i, n in h["total_tokens"].items()}
        self._prefill_complete = bool(h["prefill_complete"])
        self._decode_step = int(h["decode_step"])

    def memory_report(self) -> dict:
        """Bytes per tier: the keys of kiv/tiered_cache.py:259-286 with its
        formulas (bytes in use), plus what this path holds beyond them.

        ``total_vram_bytes`` = hot + page summaries + partial pages (+ cold
        rows kept in HBM by the hbm and split tiers, which the reference does
        not have) and ``total_cpu_bytes`` = K + V rows in host memory, as the
        reference counts them.  ``cold_rows_gpu_bytes`` is the HBM-resident
        cold rows.  ``hot_buffer_vram_bytes`` is the hot windows' buffers
        (each keeps room for 256 more rows), ``retrieval_scratch_vram_bytes``
        the stores' device memory beyond their summaries, partial pages and
        cold rows (mostly the K staging copy), and
        ``reserved_total_vram_bytes`` / ``reserved_total_cpu_bytes``
        everything held in device / pinned host memory, reservations
        included, for a caller that budgets by the real footprint."""
        hot = hot_buf = 0
        for _, l in self._owned_layers():
            used = l.keys.nelement() * l.keys.element_size() + l.values.nelement() * l.values.element_size()
            hot += used
            if isinstance(l, _HotLayer) and l._kb is not None and l.keys is l._view:
                hot_buf += l._kb.nelement() * l._kb.element_size() + l._vb.nelement() * l._vb.element_size()
            else:
                hot_buf += used
        tot = {"k_index_cpu": 0, "v_store_cpu": 0, "page_summaries_gpu": 0, "partial_gpu": 0,
               "k_cold_gpu": 0, "v_cold_gpu": 0, "reserved_gpu": 0, "reserved_cpu": 0}
        for store in self.cold_stores.values():
            for key, val in store.memory_bytes().items():
                tot[key] += val
        rows_gpu = tot["k_cold_gpu"] + tot["v_cold_gpu"]
        used_gpu = tot["page_summaries_gpu"] + tot["partial_gpu"] + rows_gpu
        cpu_rows = tot["k_index_cpu"] + tot["v_store_cpu"]
        return {
            "hot_vram_bytes": hot,
            "k_index_cpu_bytes": tot["k_index_cpu"],
            "v_store_cpu_bytes": tot["v_store_cpu"],
            "page_summaries_gpu_bytes": tot["page_summaries_gpu"],
            "total_vram_bytes": hot + used_gpu,
            "total_cpu_bytes": cpu_rows,
            "cold_rows_gpu_bytes": rows_gpu,
            "hot_buffer_vram_bytes": hot_buf,
            "retrieval_scratch_vram_bytes": max(0, tot["reserved_gpu"] - used_gpu),
            "reserved_total_vram_bytes": hot_buf + max(tot["reserved_gpu"], used_gpu),
            "reserved_total_cpu_bytes": max(tot["reserved_cpu"], cpu_rows),
        }
