"""Cold tier of one independent KV layer, backed by the gfx950 HIP kernels.

Drop-in for the reference's ``ColdKVStore`` (kiv/cold_store.py:35-414): same
constructor, ``evict_from_hot`` / ``retrieve_top_kv`` / ``cold_length`` /
``num_pages`` / ``reset`` / ``telemetry_snapshot`` / ``reset_telemetry`` /
``memory_bytes`` and the ``_cached_candidate_*`` / ``_cached_step``
attributes other code clears.  The state lives in a native store
(include/kiv_hip.h): page summaries and the partial page in HBM, finished
pages' K/V rows in pinned mapped host memory (or HBM, ``cold_tier="hbm"``;
or K in HBM and V in host memory, ``cold_tier="split"``).

Every device call is enqueued on torch's current stream; retrieval does not
synchronise the host except when the output width depends on the union size
(only possible when ``top_p > top_pages * page_size``).  There is no CPU
implementation: a store on a non-GPU device raises on its first eviction.
"""

from __future__ import annotations

import ctypes as C
import math
from collections import deque

import torch

from . import _native as nat
from . import attention, persist
from .config import KIVConfig
from .model_topology import ModelTopology


class _CandidateSet:
    """Marker that the last coarse union may be reused (shape[0] = batch)."""

    __slots__ = ("shape",)

    def __init__(self, batch: int) -> None:
        self.shape = (batch,)


class ColdKVStore:
    """Evicted tokens of one layer, paged, with coarse-to-fine retrieval."""

    def __init__(self, kiv_config: KIVConfig, topology: ModelTopology, device: torch.device) -> None:
        self.kiv_config = kiv_config
        self.device = torch.device(device)
        self._num_query_heads = topology.num_query_heads
        self._num_kv_heads = topology.num_kv_heads
        self._num_kv_groups = topology.num_query_heads // topology.num_kv_heads
        self._head_dim = topology.head_dim
        self._page_size = kiv_config.page_size
        self._handle: int | None = None
        self._batch: int | None = None
        self._dtype: torch.dtype | None = None
        self._num_finalized = 0
        self._partial_len = 0
        # Shared-layer reuse of the last coarse union (kiv/cold_store.py:81-85).
        self._cached_candidate_k = None
        self._cached_candidate_v = None
        self._cached_candidate_idx = None
        self._cached_step = -1
        self._telemetry = _RetrievalTelemetry()
        self._umax_key: tuple | None = None  # (Q, top_pages, pages) of the cached union bound
        self._umax = 1
        self._fused_kv: tuple[torch.Tensor, torch.Tensor] | None = None
        # Argument blocks of the C calls, reused call after call.
        self._rargs = nat.RetrieveArgs()
        self._rargs_ref = C.byref(self._rargs)
        self._aargs = nat.AttentionArgs()
        self._aargs_ref = C.byref(self._aargs)
        self._dev_index = -1
        self._last_coarse_slot = None  # telemetry slot of the last coarse pass (its union size)
        # Rows evicted with evict_deferred and not yet written: (k, v, T).
        self._pending: tuple[torch.Tensor, torch.Tensor, int] | None = None

    # ------------------------------------------------------------ lifetime
    def __del__(self) -> None:
        self._destroy()

    def _destroy(self) -> None:
        self._pending = None
        h, self._handle = getattr(self, "_handle", None), None
        if h is not None:
            try:
                nat.lib().kiv_store_destroy(h)
            except Exception:
                pass

    def _ensure_handle(self, k: torch.Tensor) -> None:
        if self._handle is not None:
            return
        if k.device.type != "cuda":
            raise RuntimeError(
                "ColdKVStore needs a ROCm GPU tensor: the cold tier runs only as HIP kernels "
                f"(got a tensor on {k.device})"
            )
        cfg = nat.StoreConfig(
            batch=k.shape[0],
            num_q_heads=self._num_query_heads,
            num_kv_heads=self._num_kv_heads,
            head_dim=self._head_dim,
            page_size=self._page_size,
            dtype=nat.dtype_code(k.dtype),
            cold_tier={"host": nat.TIER_HOST, "hbm": nat.TIER_HBM, "split": nat.TIER_SPLIT}[self.kiv_config.cold_tier],
            score_rounding=(nat.ROUND_ACTIVATION if self.kiv_config.score_rounding == "activation"
                            else nat.ROUND_FP32),
            reserve_tokens=int(self.kiv_config.reserve_tokens),
        )
        handle = C.c_void_p()
        nat.check(nat.lib().kiv_store_create(C.byref(cfg), k.device.index or 0, C.byref(handle)),
                  "kiv_store_create")
        self._handle = handle.value
        self._batch = k.shape[0]
        self._dtype = k.dtype
        self.device = k.device
        self._dev_index = k.get_device()

    # ------------------------------------------------------------- sizes
    @property
    def cold_length(self) -> int:
        return self._num_finalized + self._partial_len

    @property
    def num_pages(self) -> int:
        return self._num_finalized // self._page_size

    @property
    def _partial_len_tokens(self) -> int:
        return self._partial_len

    # ----------------------------------------------------------- eviction
    def evict_from_hot(self, k_evicted: torch.Tensor, v_evicted: torch.Tensor) -> None:
        """Append [B, Hkv, T, D] rows; full pages get summaries and move to the arena.

        Same contract as kiv/cold_store.py:142-184.
        """
        self._flush_pending()
        k, v, T = self._check_rows(k_evicted, v_evicted)
        if T == 0:
            return
        nat.check(nat.lib().kiv_evict(self._handle, k.data_ptr(), nat.strides(k, 3), v.data_ptr(),
                                      nat.strides(v, 3), T, nat.stream_ptr(self.device)), "kiv_evict")
        self._count(T)

    def evict_deferred(self, k_evicted: torch.Tensor, v_evicted: torch.Tensor) -> None:
        """evict_from_hot, with the rows written by the next retrieval's first
        kernel instead of a launch of their own (when they stay in the
        partial page); any other use of the store writes them first.

        For the cache's decode steps: the rows must stay unchanged until then
        (the store keeps a reference to them, which keeps their memory alive;
        the hot window only ever writes rows after its end)."""
        self._flush_pending()
        k, v, T = self._check_rows(k_evicted, v_evicted)
        if T == 0:
            return
        if self._partial_len + T >= self._page_size or self._num_finalized == 0:
            nat.check(nat.lib().kiv_evict(self._handle, k.data_ptr(), nat.strides(k, 3), v.data_ptr(),
                                          nat.strides(v, 3), T, nat.stream_ptr(self.device)), "kiv_evict")
        else:
            self._pending = (k, v, T)
        self._count(T)

    def _flush_pending(self) -> None:
        """Write deferred rows now (a launch of their own)."""
        p = self._pending
        if p is None:
            return
        self._pending = None
        k, v, T = p
        nat.check(nat.lib().kiv_evict(self._handle, k.data_ptr(), nat.strides(k, 3), v.data_ptr(),
                                      nat.strides(v, 3), T, nat.stream_ptr(self.device)), "kiv_evict")

    def _count(self, T: int) -> None:
        total = self._partial_len + T
        self._num_finalized += (total // self._page_size) * self._page_size
        self._partial_len = total % self._page_size

    def _check_rows(self, k_evicted: torch.Tensor, v_evicted: torch.Tensor):
        """Validated (k, v, T) of evicted rows (unit stride over D); invalidates
        the shared-layer candidates (kiv/cold_store.py:148-151)."""
        self._invalidate_candidates()
        shape = k_evicted.shape
        if len(shape) != 4 or shape != v_evicted.shape:
            raise ValueError(f"expected matching [B, Hkv, T, D] K/V, got {tuple(shape)} "
                             f"and {tuple(v_evicted.shape)}")
        T = shape[2]
        if T == 0:
            return k_evicted, v_evicted, 0
        if self._handle is None:
            self._ensure_handle(k_evicted)
        if shape[0] != self._batch or shape[1] != self._num_kv_heads or shape[3] != self._head_dim:
            raise ValueError(f"evicted rows {tuple(shape)} do not match the store "
                             f"(B={self._batch}, Hkv={self._num_kv_heads}, D={self._head_dim})")
        if k_evicted.dtype != self._dtype or v_evicted.dtype != self._dtype:
            raise TypeError(f"evicted rows are {k_evicted.dtype}, the store holds {self._dtype}")
        if k_evicted.get_device() != self._dev_index or v_evicted.get_device() != self._dev_index:
            raise ValueError(f"evicted rows on {k_evicted.device}, store on {self.device}")
        k = k_evicted if k_evicted.stride(3) == 1 else k_evicted.contiguous()
        v = v_evicted if v_evicted.stride(3) == 1 else v_evicted.contiguous()
        return k, v, T

    def _invalidate_candidates(self) -> None:
        self._cached_candidate_k = None
        self._cached_candidate_v = None
        self._cached_candidate_idx = None
        self._cached_step = -1

    # ---------------------------------------------------------- retrieval
    def retrieve_top_kv(self, query: torch.Tensor, scaling: float, kiv_config: KIVConfig,
                        step: int = -1):
        """Top-P cold K/V ``[B, Hkv, P', D]`` in descending score order, or (None, None).

        Same contract as kiv/cold_store.py:283-371: coarse page scores against
        the summaries, union of every (batch, head, position)'s top pages,
        fine scores max-reduced over heads and positions, top-P per batch row.
        """
        if self.cold_length == 0:
            return None, None
        k_out, v_out, _ = self._retrieve(query, scaling, kiv_config, step, None)
        return k_out, v_out

    def retrieve_attend(self, query: torch.Tensor, scaling: float, kiv_config: KIVConfig,
                        hot_k: torch.Tensor, hot_v: torch.Tensor, mask: torch.Tensor | None,
                        step: int = -1, hot_rows=None) -> torch.Tensor | None:
        """retrieve_top_kv followed by the merged attention over [retrieved ; hot]
        (kiv_retrieve_attend), or None when the cold tier is empty.

        Returns the attention output ``[B, Q, Hq, D]``; the retrieval's
        telemetry and candidate cache are updated as by retrieve_top_kv.
        ``hot_rows = (src_k, src_v, dst_k, dst_v)``: rows of the hot window
        not written yet (the cache's decode step leaves them to this call):
        the call copies src into dst ([B, Hkv, n, D] views) with its first
        launch, before the attention reads the window.  With None returned
        they are not written.
        """
        if self.cold_length == 0:
            return None
        _, _, out = self._retrieve(query, scaling, kiv_config, step, (hot_k, hot_v, mask), hot_rows)
        return out

    def _retrieve(self, query, scaling, kiv_config, step, attend, hot_rows=None):
        """One retrieval; with ``attend = (hot_k, hot_v, mask)`` also the merged
        attention (fused when the output width is known on the host)."""
        shape = query.shape
        if len(shape) != 4 or shape[1] != self._num_query_heads or shape[3] != self._head_dim:
            raise ValueError(f"query must be [B, {self._num_query_heads}, Q, {self._head_dim}], "
                             f"got {tuple(shape)}")
        B, _, Q, D = shape
        if B != self._batch:
            raise ValueError(f"query batch {B} != store batch {self._batch}")
        if query.get_device() != self._dev_index:
            raise ValueError(f"query on {query.device}, store on {self.device}")
        q = query if query.dtype == self._dtype else query.to(self._dtype)
        if q.stride(3) != 1:
            q = q.contiguous()
        top_p, top_pages = kiv_config.top_p, kiv_config.top_pages
        cold = self._num_finalized + self._partial_len
        P = min(top_p, cold)
        N = self._num_finalized // self._page_size
        reuse = (step >= 0 and step == self._cached_step and self._cached_candidate_k is not None
                 and self._cached_candidate_k.shape[0] == B)
        # Lower bound of the candidate count: the union holds at least
        # min(top_pages, N) pages (exactly N when every page is selected).
        c_low = min(top_pages, N) * self._page_size + self._partial_len
        width = min(P, c_low)
        exact = width == P
        if not exact:
            width = P  # buffer width; the true count follows from U below

        lib = nat.lib()
        key = (Q, top_pages, N)
        if self._umax_key != key:
            umax = C.c_int64(0)
            nat.check(lib.kiv_max_union_pages(self._handle, Q, top_pages, C.byref(umax)), "kiv_max_union_pages")
            self._umax_key, self._umax = key, max(1, umax.value)
        dev = self.device
        fused = attend is not None and exact
        if fused:
            # Consumed by the attention on the same stream: one pair per store.
            kv = self._fused_kv
            if kv is None or kv[0].shape[2] != width:
                shape_kv = (B, self._num_kv_heads, width, D)
                kv = self._fused_kv = (torch.empty(shape_kv, dtype=self._dtype, device=dev),
                                       torch.empty(shape_kv, dtype=self._dtype, device=dev))
            k_out, v_out = kv
        else:
            k_out = torch.empty(B, self._num_kv_heads, width, D, dtype=self._dtype, device=dev)
            v_out = torch.empty_like(k_out)
        coarse_runs = N > 0 and not reuse
        # This call's slot of the telemetry ring (kernels fill every entry
        # they own, so no zero-fill launches here).
        tel = self._telemetry
        slot = tel.take_slot(dev, B, width, self._umax, coarse_runs)
        a = self._rargs
        a.q = q.data_ptr()
        a.q_stride = nat.strides(q, 4)
        a.q_len = Q
        a.scaling = scaling
        a.top_pages = top_pages
        a.out_width = width
        a.reuse_candidates = 1 if reuse else 0
        a.flags = nat.RETRIEVE_PRUNE if getattr(kiv_config, "fine_pruning", False) else 0
        a.k_out = k_out.data_ptr()
        a.v_out = v_out.data_ptr()
        a.idx_out = slot.sel_ptr
        a.pages_out = slot.pages_ptr
        a.union_count_out = slot.count_ptr
        a.stats_out = slot.stats_ptr
        a.stats_accum = tel.accum_ptr
        pend = self._pending
        if pend is not None:
            # The deferred rows go in with this call (their own launch only
            # when they finish a page or no coarse pass runs).
            self._pending = None
            pk, pv, pt = pend
            a.append_k, a.append_v = pk.data_ptr(), pv.data_ptr()
            a.append_k_stride, a.append_v_stride = nat.strides(pk, 3), nat.strides(pv, 3)
            a.append_tokens = pt
        else:
            a.append_tokens = 0
        if hot_rows is not None:
            sk, sv, dk, dv = hot_rows
            a.hot_src_k, a.hot_src_v, a.hot_dst_k, a.hot_dst_v = sk.data_ptr(), sv.data_ptr(), dk.data_ptr(), dv.data_ptr()
            a.hot_src_k_stride, a.hot_src_v_stride = nat.strides(sk, 3), nat.strides(sv, 3)
            a.hot_dst_k_stride, a.hot_dst_v_stride = nat.strides(dk, 3), nat.strides(dv, 3)
            a.hot_tokens = sk.shape[2]
        else:
            a.hot_tokens = 0
        stream = nat.stream_ptr(dev)
        out = None
        try:
            if fused:
                hot_k, hot_v, mask = attend
                out, _keep = attention.fill_args(self._aargs, q, width, hot_k, hot_v, mask, scaling)
                self._aargs.cold_k, self._aargs.cold_v = a.k_out, a.v_out
                nat.check(lib.kiv_retrieve_attend(self._handle, self._rargs_ref, self._aargs_ref, stream),
                          "kiv_retrieve_attend")
            else:
                nat.check(lib.kiv_retrieve(self._handle, self._rargs_ref, stream), "kiv_retrieve")
        except Exception as e:
            # A call refused by its checks evicted nothing: the deferred rows
            # are still this store's to write (counted already).
            if pend is not None and (not isinstance(e, nat.KivError) or e.refused):
                self._pending = pend
            raise

        if coarse_runs:
            self._last_coarse_slot = slot
            tel.record_coarse(slot, num_pages=N, cold_length=cold)
        else:
            tel.record_coarse_skipped(cold_length=cold)
        if not reuse:
            self._cached_candidate_k = self._cached_candidate_v = self._cached_candidate_idx = _CandidateSet(B)
            if step >= 0:
                self._cached_step = step

        if not exact:
            # Only reachable when top_p > top_pages * page_size: the output
            # width depends on the union size, so read U back.
            U = tel.union_size(self._last_coarse_slot) if N > 0 else 0
            actual = min(P, U * self._page_size + self._partial_len)
            k_out, v_out = k_out[:, :, :actual], v_out[:, :, :actual]
        else:
            actual = width
        tel.record_fine(slot, actual_P=actual, requested_P=int(top_p), cold_length=cold)
        if attend is not None and out is None:
            hot_k, hot_v, mask = attend
            out = attention.decode_attention(q, k_out, v_out, hot_k, hot_v, mask, scaling)
        return k_out, v_out, out

    # ------------------------------------------------------ bookkeeping
    def reset(self) -> None:
        """Drop every cold token (kiv/cold_store.py:374-389); allocations are kept."""
        self._pending = None  # deferred rows are cold tokens too: dropped
        if self._handle is not None:
            nat.check(nat.lib().kiv_store_reset(self._handle), "kiv_store_reset")
        self._num_finalized = 0
        self._partial_len = 0
        self._invalidate_candidates()

    # ------------------------------------------------------ persistence
    def save(self, f) -> None:
        """Write the cold tier to the binary file ``f`` (a section of the
        format in kiv_amd/persist.py): the rows of every cold token, in
        order.  No counterpart in the reference, whose cold tier lives in
        process memory only."""
        self._flush_pending()
        T = self.cold_length
        persist.write_header(f, persist.COLD_MAGIC, {
            "format": "kiv-cold", "version": persist.VERSION,
            "dtype": persist.dtype_name(self._dtype or torch.float32), "batch": self._batch or 0,
            "num_kv_heads": self._num_kv_heads, "head_dim": self._head_dim, "page_size": self._page_size,
            "cold_length": T, "chunk_tokens": persist.CHUNK_TOKENS,
        })
        for first in range(0, T, persist.CHUNK_TOKENS):
            k, v = self.read_tokens(first, min(persist.CHUNK_TOKENS, T - first))
            persist.write_tensor(f, k)
            persist.write_tensor(f, v)

    def load(self, f, device: torch.device | None = None) -> None:
        """Refill an empty store from a section written by :meth:`save`.

        The rows are evicted again in order, which rebuilds the pages, the
        summaries and the radii bit for bit.  The file's kv heads, head dim
        and page size must be this store's; its batch and dtype become the
        store's.  ``device`` is where a store without rows yet puts them (the
        store's device by default)."""
        if self.cold_length:
            raise RuntimeError("ColdKVStore.load: the store already holds cold tokens; reset() it first")
        h = persist.read_header(f, persist.COLD_MAGIC)
        for key, mine in (("num_kv_heads", self._num_kv_heads), ("head_dim", self._head_dim),
                          ("page_size", self._page_size)):
            if h[key] != mine:
                raise ValueError(f"ColdKVStore.load: the file's {key} is {h[key]}, this store's is {mine}")
        dtype = persist.dtype_of(h["dtype"])
        if self._dtype is not None and dtype != self._dtype:
            raise ValueError(f"ColdKVStore.load: the file holds {dtype}, this store {self._dtype}")
        dev = torch.device(device) if device is not None else self.device
        B, H, D, T, chunk = h["batch"], h["num_kv_heads"], h["head_dim"], h["cold_length"], h["chunk_tokens"]
        for first in range(0, T, chunk):
            n = min(chunk, T - first)
            k = persist.read_tensor(f, (B, H, n, D), dtype, dev)
            v = persist.read_tensor(f, (B, H, n, D), dtype, dev)
            self.evict_from_hot(k, v)

    def telemetry_snapshot(self) -> dict:
        return self._telemetry.snapshot()

    def reset_telemetry(self) -> None:
        self._telemetry = _RetrievalTelemetry()

    def memory_bytes(self) -> dict[str, int]:
        """Bytes per tier, keys as kiv/cold_store.py:399-414, plus the HBM
        tiers' cold rows and what the store reserves.

        The reference's keys count the bytes in use (K/V rows of finished
        pages, dtype summaries, the partial page's rows).  ``reserved_gpu``
        is everything the store holds in device memory -- grown buffers,
        the HBM tiers' arena chunks and the retrieval scratch, whose K
        staging copy is the largest part (up to 256 MiB per store on the
        host tier) -- and ``reserved_cpu`` the pinned host arena's chunks."""
        out = {"k_index_cpu": 0, "v_store_cpu": 0, "page_summaries_gpu": 0, "partial_gpu": 0,
               "k_cold_gpu": 0, "v_cold_gpu": 0, "reserved_gpu": 0, "reserved_cpu": 0}
        if self._handle is None:
            return out
        self._flush_pending()
        info = nat.StoreInfo()
        nat.check(nat.lib().kiv_store_info(self._handle, C.byref(info)), "kiv_store_info")
        tier = self.kiv_config.cold_tier
        out["k_index_cpu" if tier == "host" else "k_cold_gpu"] = info.k_cold_bytes
        out["v_cold_gpu" if tier == "hbm" else "v_store_cpu"] = info.v_cold_bytes
        out["page_summaries_gpu"] = info.summary_bytes
        out["partial_gpu"] = info.partial_bytes
        out["reserved_gpu"] = info.reserved_device_bytes
        out["reserved_cpu"] = info.reserved_host_bytes
        return out

    # ------------------------------------------------- inspection (tests)
    def fine_scan_stats(self) -> tuple[int, int]:
        """(page slices the last retrieval's fine scan read, union page slices);
        a slice is one kv row of one union page.  Synchronises the device."""
        self._flush_pending()
        scanned, total = C.c_int64(), C.c_int64()
        nat.check(nat.lib().kiv_fine_scan_stats(self._handle, C.byref(scanned), C.byref(total)),
                  "kiv_fine_scan_stats")
        return scanned.value, total.value

    def readahead_bytes(self) -> int:
        """Host bytes the last retrieval's coarse select read ahead into HBM
        for the pruned fine scan (its first speculative page per kv row;
        0: none)."""
        if self._handle is None:
            return 0
        info = nat.StoreInfo()
        nat.check(nat.lib().kiv_store_info(self._handle, C.byref(info)), "kiv_store_info")
        return int(info.readahead_bytes)

    def read_summaries(self, first: int = 0, n: int | None = None) -> tuple[torch.Tensor, torch.Tensor]:
        """(dtype summaries, fp32 means) of pages [first, first+n), each
        [n, B, Hkv, D], copied from HBM (every page by default)."""
        self._flush_pending()
        n = self.num_pages - first if n is None else n
        if first < 0 or n < 0 or first + n > self.num_pages:
            raise ValueError(f"pages [{first}, {first + n}) outside the store's {self.num_pages}")
        shape = (n, self._batch or 1, self._num_kv_heads, self._head_dim)
        s = torch.empty(shape, dtype=self._dtype or torch.float32, device=self.device)
        s32 = torch.empty(shape, dtype=torch.float32, device=self.device)
        if n:
            nat.check(nat.lib().kiv_store_read_summaries(self._handle, first, n, s.data_ptr(), s32.data_ptr(),
                                                         nat.stream_ptr(self.device)), "read_summaries")
        return s, s32

    def read_tokens(self, first: int = 0, n: int | None = None) -> tuple[torch.Tensor, torch.Tensor]:
        """Cold tokens [first, first+n) as [B, Hkv, n, D] K and V on the device."""
        self._flush_pending()
        n = self.cold_length - first if n is None else n
        k = torch.empty(self._batch or 1, self._num_kv_heads, n, self._head_dim,
                        dtype=self._dtype or torch.float32, device=self.device)
        v = torch.empty_like(k)
        if n:
            nat.check(nat.lib().kiv_store_read_tokens(self._handle, first, n, k.data_ptr(), v.data_ptr(),
                                                      nat.stream_ptr(self.device)), "read_tokens")
        return k, v


class _Slot:
    """Device addresses of one retrieval call's entries in the telemetry rings."""

    __slots__ = ("index", "rings", "batch", "width", "stats_ptr", "sel_ptr", "pages_ptr", "count_ptr")


class _RetrievalTelemetry:
    """Per-call coarse/fine records in a 256-entry ring, read lazily.

    Same schema as kiv/cold_store.py:417-581.  Kernels write each call's
    statistics, union pages and selected ids into slots of preallocated
    device rings (one slot per retrieval call, 256 slots, so a slot outlives
    the records that refer to it) and add the scores to a device
    accumulator: recording allocates nothing and costs no host
    synchronisation; :meth:`snapshot` converts everything at once.
    """

    _MAX_BUFFER = 256

    def __init__(self) -> None:
        self.total_calls = 0
        self.coarse_calls = 0
        self.coarse_real_calls = 0
        self.coarse_cold_length_sum = 0
        self.fine_calls = 0
        self.selected_count_sum = 0
        self._accum: torch.Tensor | None = None
        self.accum_ptr = 0
        self._ring: deque = deque(maxlen=self._MAX_BUFFER)
        self._calls = 0  # retrieval calls, the slot counter
        # Rings, one row per slot: stats [256, 4] f32, union sizes [256] i32,
        # union pages [256, cap] i32, selected ids [256, cap] i64.  A ring
        # that must grow is replaced; records keep the one they refer to.
        self._rings: dict[str, torch.Tensor] = {}

    def _ring_for(self, name: str, device, cols: int, dtype) -> torch.Tensor:
        r = self._rings.get(name)
        if r is None or r.shape[1] < cols:
            r = torch.empty(self._MAX_BUFFER, cols, dtype=dtype, device=device)
            self._rings[name] = r
        return r

    def take_slot(self, device: torch.device, batch: int, width: int, max_pages: int, coarse: bool) -> _Slot:
        """This call's slot: device addresses of its stats[4], selected ids
        [batch, width], union pages [max_pages] and union size (the last two
        0 when no coarse pass runs)."""
        if self._accum is None:
            self._accum = torch.zeros(4, dtype=torch.float64, device=device)
            self.accum_ptr = self._accum.data_ptr()
        stats = self._ring_for("stats", device, 4, torch.float32)
        count = self._ring_for("count", device, 1, torch.int32)
        sel = self._ring_for("sel", device, max(batch * width, 256), torch.int64)
        i = self._calls % self._MAX_BUFFER
        self._calls += 1
        s = _Slot()
        s.index, s.batch, s.width = i, batch, width
        s.stats_ptr = stats.data_ptr() + i * 16
        s.sel_ptr = sel.data_ptr() + i * sel.shape[1] * 8
        if coarse:
            pages = self._ring_for("pages", device, max(max_pages, 64), torch.int32)
            s.pages_ptr = pages.data_ptr() + i * pages.shape[1] * 4
            s.count_ptr = count.data_ptr() + i * 4
            s.rings = (stats, sel, pages, count)
        else:
            s.pages_ptr = s.count_ptr = 0
            s.rings = (stats, sel, None, None)
        return s

    def union_size(self, slot: _Slot) -> int:
        """U of the slot's coarse pass (synchronises)."""
        return int(slot.rings[3][slot.index, 0].item())

    def record_coarse(self, slot: _Slot, *, num_pages, cold_length) -> None:
        self.coarse_calls += 1
        self.coarse_real_calls += 1
        self.coarse_cold_length_sum += cold_length
        self._ring.append({"kind": "coarse", "cold_length": cold_length, "num_pages": num_pages,
                           "_slot": slot, "skipped": False})

    def record_coarse_skipped(self, *, cold_length: int) -> None:
        self.coarse_calls += 1
        self.coarse_cold_length_sum += cold_length
        self._ring.append({"kind": "coarse", "cold_length": cold_length, "num_pages": 0,
                           "num_pages_selected": 0, "top_score": 0.0, "mean_score": 0.0, "score_ratio": 0.0,
                           "pages_selected": [], "skipped": True})

    def record_fine(self, slot: _Slot, *, actual_P, requested_P, cold_length) -> None:
        self.fine_calls += 1
        self.total_calls += 1
        self.selected_count_sum += actual_P
        self._ring.append({"kind": "fine", "cold_length": cold_length, "actual_P": actual_P,
                           "requested_P": requested_P, "_slot": slot})

    @staticmethod
    def _ratio(top: float, mean: float) -> float:
        return (top / abs(mean)) if mean else math.inf

    def _materialise(self, rec: dict) -> dict:
        slot = rec.get("_slot")
        if slot is None:
            return dict(rec)
        stats_ring, sel_ring, pages_ring, count_ring = slot.rings
        stats = stats_ring[slot.index].tolist()
        out = {k: v for k, v in rec.items() if not k.startswith("_")}
        if rec["kind"] == "coarse":
            n = int(count_ring[slot.index, 0].item())
            pages = pages_ring[slot.index, :n].tolist()
            top, mean = stats[0], stats[1]
            out.update(num_pages_selected=len(pages), top_score=top, mean_score=mean,
                       score_ratio=self._ratio(top, mean), pages_selected=pages)
            out = {k: out[k] for k in ("kind", "cold_length", "num_pages", "num_pages_selected",
                                       "top_score", "mean_score", "score_ratio", "pages_selected",
                                       "skipped")}
        else:
            top, mean = stats[2], stats[3]
            ids = sel_ring[slot.index, :slot.batch * slot.width].view(slot.batch, slot.width)
            out.update(top_score=top, mean_score=mean, score_ratio=self._ratio(top, mean),
                       selected_token_indices=ids[:, :rec["actual_P"]].reshape(-1).tolist())
            out = {k: out[k] for k in ("kind", "cold_length", "actual_P", "requested_P", "top_score",
                                       "mean_score", "score_ratio", "selected_token_indices")}
        return out

    def snapshot(self) -> dict:
        sums = self._accum.tolist() if self._accum is not None else [0.0] * 4
        agg = {
            "total_calls": self.total_calls,
            "coarse_calls": self.coarse_calls,
            "coarse_real_calls": self.coarse_real_calls,
            "coarse_skipped_calls": self.coarse_calls - self.coarse_real_calls,
            "fine_calls": self.fine_calls,
        }
        if self.coarse_real_calls:
            agg["avg_coarse_top_score"] = sums[0] / self.coarse_real_calls
            agg["avg_coarse_mean_score"] = sums[1] / self.coarse_real_calls
        if self.coarse_calls:
            agg["avg_cold_length"] = self.coarse_cold_length_sum / self.coarse_calls
        if self.fine_calls:
            agg["avg_fine_top_score"] = sums[2] / self.fine_calls
            agg["avg_fine_mean_score"] = sums[3] / self.fine_calls
            agg["avg_selected_P"] = self.selected_count_sum / self.fine_calls
        return {"aggregates": agg, "recent": [self._materialise(r) for r in self._ring]}
