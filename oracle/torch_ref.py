"""The reference's tiered-cache op sequence on CPU torch tensors.

Test infrastructure only (see oracle/__init__.py).  This is the CPU baseline
("port") and the dtype-faithful checker: each step uses the torch op the
reference uses, in the activation dtype, so rounding matches the reference
running on CPU.  Ties inside ``topk`` follow torch's CPU kernel, which the
reference leaves unspecified; parity tests compare index *sets* only where
the selection boundary is separated (oracle.exact.top_k_set gaps).
"""

from __future__ import annotations

from dataclasses import dataclass, field

import torch


def expand_kv(x: torch.Tensor, groups: int) -> torch.Tensor:
    """GQA expansion, materialised as in kiv/cold_store.py:23-32."""
    if groups == 1:
        return x
    B, H, T, D = x.shape
    return x[:, :, None].expand(B, H, groups, T, D).reshape(B, H * groups, T, D)


@dataclass
class RetrieveTrace:
    """Intermediates of one retrieval, for parity tests."""

    coarse_scores: torch.Tensor | None = None   # [B, Hq, Q, N] dtype
    pages: torch.Tensor | None = None           # union, ascending
    candidate_ids: torch.Tensor | None = None   # [C]
    agg_scores: torch.Tensor | None = None      # [B, C] dtype
    top_local: torch.Tensor | None = None       # [B, P'] candidate positions
    selected_ids: torch.Tensor | None = None    # [B, P'] global ids
    extra: dict = field(default_factory=dict)


class OracleTelemetry:
    """The retrieval telemetry ring of kiv/cold_store.py:417-581: a coarse and
    a fine record per retrieval (a placeholder coarse record when the coarse
    pass is skipped), running sums over real passes, and the snapshot with
    its aggregates.  Scores are the dtype tensors' own ``max``/``mean``
    (``float(t.max())``, ``float(t.mean())`` as at :468-469 and :524-525)."""

    MAX_BUFFER = 256

    def __init__(self) -> None:
        self.total_calls = 0
        self.coarse_calls = 0
        self.coarse_real_calls = 0
        self.coarse_top_sum = 0.0
        self.coarse_mean_sum = 0.0
        self.coarse_cold_sum = 0
        self.fine_calls = 0
        self.fine_top_sum = 0.0
        self.fine_mean_sum = 0.0
        self.selected_sum = 0
        self.ring: list[dict] = []

    def _push(self, rec: dict) -> None:
        # kiv/cold_store.py:549-552
        self.ring.append(rec)
        self.ring = self.ring[-self.MAX_BUFFER:]

    @staticmethod
    def _ratio(top: float, mean: float) -> float:
        return top / abs(mean) if mean else float("inf")

    def coarse(self, coarse_scores, top_page_idx, num_pages: int, cold_length: int) -> None:
        # kiv/cold_store.py:456-488
        top, mean = float(coarse_scores.max()), float(coarse_scores.mean())
        pages = top_page_idx.reshape(-1).unique().tolist()
        self.coarse_calls += 1
        self.coarse_real_calls += 1
        self.coarse_top_sum += top
        self.coarse_mean_sum += mean
        self.coarse_cold_sum += cold_length
        self._push({"kind": "coarse", "cold_length": cold_length, "num_pages": num_pages,
                    "num_pages_selected": len(pages), "top_score": top, "mean_score": mean,
                    "score_ratio": self._ratio(top, mean), "pages_selected": pages, "skipped": False})

    def coarse_skipped(self, cold_length: int) -> None:
        # kiv/cold_store.py:490-512
        self.coarse_calls += 1
        self.coarse_cold_sum += cold_length
        self._push({"kind": "coarse", "cold_length": cold_length, "num_pages": 0, "num_pages_selected": 0,
                    "top_score": 0.0, "mean_score": 0.0, "score_ratio": 0.0, "pages_selected": [],
                    "skipped": True})

    def fine(self, agg_scores, selected_ids, actual_P: int, requested_P: int, cold_length: int) -> None:
        # kiv/cold_store.py:514-547
        top, mean = float(agg_scores.max()), float(agg_scores.mean())
        self.fine_calls += 1
        self.total_calls += 1
        self.fine_top_sum += top
        self.fine_mean_sum += mean
        self.selected_sum += actual_P
        self._push({"kind": "fine", "cold_length": cold_length, "actual_P": actual_P, "requested_P": requested_P,
                    "top_score": top, "mean_score": mean, "score_ratio": self._ratio(top, mean),
                    "selected_token_indices": selected_ids.reshape(-1).tolist()})

    def snapshot(self) -> dict:
        # kiv/cold_store.py:554-581
        agg = {"total_calls": self.total_calls, "coarse_calls": self.coarse_calls,
               "coarse_real_calls": self.coarse_real_calls,
               "coarse_skipped_calls": self.coarse_calls - self.coarse_real_calls, "fine_calls": self.fine_calls}
        if self.coarse_real_calls:
            agg["avg_coarse_top_score"] = self.coarse_top_sum / self.coarse_real_calls
            agg["avg_coarse_mean_score"] = self.coarse_mean_sum / self.coarse_real_calls
        if self.coarse_calls:
            agg["avg_cold_length"] = self.coarse_cold_sum / self.coarse_calls
        if self.fine_calls:
            agg["avg_fine_top_score"] = self.fine_top_sum / self.fine_calls
            agg["avg_fine_mean_score"] = self.fine_mean_sum / self.fine_calls
            agg["avg_selected_P"] = self.selected_sum / self.fine_calls
        return {"aggregates": agg, "recent": list(self.ring)}


class OracleColdStore:
    """ColdKVStore semantics (kiv/cold_store.py:35-414) on CPU, with its
    telemetry and its shared-layer candidate cache."""

    def __init__(self, page_size: int, num_kv_groups: int) -> None:
        self.page_size = page_size
        self.groups = num_kv_groups
        self.k_pages: list[torch.Tensor] = []
        self.v_pages: list[torch.Tensor] = []
        self.summaries: list[torch.Tensor] = []
        self.partial_k: torch.Tensor | None = None
        self.partial_v: torch.Tensor | None = None
        self._flat: tuple | None = None  # concatenated summaries / K / V, as after
                                         # kiv/cold_store.py:122-136 (_materialize)
        self.telemetry = OracleTelemetry()
        # kiv/cold_store.py:81-85: candidates of the last coarse pass, for a
        # shared layer's call in the same decode step.
        self.cached: tuple | None = None   # (K, V, ids, pages)
        self.cached_step = -1

    def reset(self) -> None:
        """kiv/cold_store.py:374-389 (the telemetry is kept, as there)."""
        self.k_pages, self.v_pages, self.summaries = [], [], []
        self.partial_k = self.partial_v = None
        self._flat = None
        self.cached, self.cached_step = None, -1

    # kiv/cold_store.py:111-120
    @property
    def num_pages(self) -> int:
        return len(self.summaries)

    @property
    def partial_len(self) -> int:
        return 0 if self.partial_k is None else self.partial_k.shape[2]

    @property
    def cold_length(self) -> int:
        return self.num_pages * self.page_size + self.partial_len

    # kiv/cold_store.py:142-184
    def evict(self, k: torch.Tensor, v: torch.Tensor) -> None:
        """Append rows; every full page gets ``mean(dim=2)`` of its K rows (in
        the dtype) and is stored.  Pages are cut from views of the combined
        rows rather than by re-slicing the partial once per page, which
        keeps bulk evictions linear; the stored values are the same.
        Eviction drops the cached candidates (kiv/cold_store.py:148-151)."""
        self._flat = None
        self.cached, self.cached_step = None, -1
        if self.partial_len:
            k = torch.cat([self.partial_k, k], dim=2)
            v = torch.cat([self.partial_v, v], dim=2)
        ps = self.page_size
        n = k.shape[2] // ps
        for i in range(n):
            pk, pv = k[:, :, i * ps:(i + 1) * ps], v[:, :, i * ps:(i + 1) * ps]
            self.summaries.append(pk.mean(dim=2, keepdim=True))
            self.k_pages.append(pk.clone())
            self.v_pages.append(pv.clone())
        rest = k.shape[2] - n * ps
        self.partial_k = k[:, :, n * ps:].contiguous() if rest else None
        self.partial_v = v[:, :, n * ps:].contiguous() if rest else None

    def flat(self):
        """(summaries [B,Hkv,N,D], K [B,Hkv,N*ps,D], V) of the finished pages."""
        if self._flat is None:
            self._flat = (torch.cat(self.summaries, dim=2), torch.cat(self.k_pages, dim=2),
                          torch.cat(self.v_pages, dim=2))
        return self._flat

    def all_k(self) -> torch.Tensor:
        parts = self.k_pages + ([self.partial_k] if self.partial_len else [])
        return torch.cat(parts, dim=2)

    def all_v(self) -> torch.Tensor:
        parts = self.v_pages + ([self.partial_v] if self.partial_len else [])
        return torch.cat(parts, dim=2)

    # kiv/cold_store.py:186-280
    def candidates(self, query: torch.Tensor, scaling: float, top_pages: int, trace: RetrieveTrace):
        ks, vs, ids = [], [], []
        ps = self.page_size
        if self.num_pages:
            summ, kall, vall = self.flat()
            coarse = torch.matmul(query, expand_kv(summ, self.groups).transpose(-2, -1)) * scaling
            _, top_idx = coarse.topk(min(top_pages, self.num_pages), dim=-1)
            pages = top_idx.reshape(-1).unique(sorted=True)
            trace.extra["top_idx"] = top_idx
            tok = (pages[:, None] * ps + torch.arange(ps)[None, :]).reshape(-1)
            ks.append(kall[:, :, tok])
            vs.append(vall[:, :, tok])
            ids.append(tok)
            trace.coarse_scores, trace.pages = coarse, pages
            self.telemetry.coarse(coarse, top_idx, self.num_pages, self.cold_length)
        if self.partial_len:
            n_fin = self.num_pages * ps
            ks.append(self.partial_k)
            vs.append(self.partial_v)
            ids.append(torch.arange(n_fin, n_fin + self.partial_len))
        if not self.num_pages:
            self.telemetry.coarse_skipped(self.cold_length)   # kiv/cold_store.py:277-278
        return torch.cat(ks, dim=2), torch.cat(vs, dim=2), torch.cat(ids)

    # kiv/cold_store.py:283-371
    def retrieve(self, query: torch.Tensor, scaling: float, top_p: int, top_pages: int, step: int = -1):
        """(K [B,Hkv,P',D], V, trace) or (None, None, trace) when cold is empty.

        A call with ``step >= 0`` equal to the step of the cached candidates
        (and the same batch) reuses them, skipping the coarse pass, and
        scores them with this query (kiv/cold_store.py:303-317);
        ``trace.extra["reused"]`` says which happened."""
        trace = RetrieveTrace()
        if self.cold_length == 0:
            return None, None, trace
        P = min(top_p, self.cold_length)
        if (step >= 0 and step == self.cached_step and self.cached is not None
                and self.cached[0].shape[0] == query.shape[0]):
            ck, cv, cid, trace.pages = self.cached
            self.telemetry.coarse_skipped(self.cold_length)
            trace.extra["reused"] = True
        else:
            ck, cv, cid = self.candidates(query, scaling, top_pages, trace)
            self.cached = (ck, cv, cid, trace.pages)
            if step >= 0:
                self.cached_step = step
            trace.extra["reused"] = False
        k_out, v_out = self._fine(query, ck, cv, cid, scaling, P, trace)
        self.telemetry.fine(trace.agg_scores, trace.selected_ids, int(trace.top_local.shape[-1]), int(top_p),
                            self.cold_length)
        return k_out, v_out, trace

    def _fine(self, query, ck, cv, cid, scaling: float, P: int, trace: RetrieveTrace):
        """kiv/cold_store.py:332-362: fine scores in the dtype, max over heads
        and positions, top-P descending, gather."""
        fine = torch.matmul(query, expand_kv(ck, self.groups).transpose(-2, -1)) * scaling
        agg = fine.amax(dim=(1, 2))
        _, top_local = agg.topk(min(P, agg.shape[-1]), dim=-1)
        idx = top_local[:, None, :, None].expand(-1, ck.shape[1], -1, ck.shape[3])
        trace.candidate_ids, trace.agg_scores, trace.top_local = cid, agg, top_local
        trace.selected_ids = cid[top_local]
        return torch.gather(ck, 2, idx), torch.gather(cv, 2, idx)

    def retrieve_given_union(self, query: torch.Tensor, scaling: float, top_p: int, pages) -> RetrieveTrace:
        """The fine stage of kiv/cold_store.py:283-371 over the candidates of a
        given page union (ascending page ids; the partial page's tokens last,
        as at :227-262), with no telemetry: the reference's top-P conditioned
        on a union, so that a parity test can check the fine selection apart
        from the coarse one."""
        trace = RetrieveTrace()
        ps = self.page_size
        pages = torch.as_tensor(pages, dtype=torch.int64).reshape(-1)
        ks, vs, ids = [], [], []
        if pages.numel():
            _, kall, vall = self.flat()
            tok = (pages[:, None] * ps + torch.arange(ps)[None, :]).reshape(-1)
            ks.append(kall[:, :, tok])
            vs.append(vall[:, :, tok])
            ids.append(tok)
        if self.partial_len:
            n_fin = self.num_pages * ps
            ks.append(self.partial_k)
            vs.append(self.partial_v)
            ids.append(torch.arange(n_fin, n_fin + self.partial_len))
        trace.pages = pages
        P = min(top_p, self.cold_length)
        self._fine(query, torch.cat(ks, dim=2), torch.cat(vs, dim=2), torch.cat(ids), scaling, P, trace)
        return trace


def eager_attention(query, key, value, mask, scaling):
    """Transformers' eager attention (models/qwen2/modeling_qwen2.py:150-172):
    dtype matmul * scaling (+ mask), fp32 softmax cast back, weights @ V.
    Returns [B, Q, Hq, D]."""
    groups = query.shape[1] // key.shape[1]
    w = torch.matmul(query, expand_kv(key, groups).transpose(2, 3)) * scaling
    if mask is not None:
        w = w + mask
    w = torch.softmax(w, dim=-1, dtype=torch.float32).to(query.dtype)
    return torch.matmul(w, expand_kv(value, groups)).transpose(1, 2).contiguous()


def extend_mask(mask: torch.Tensor, num_cold: int) -> torch.Tensor:
    """kiv/mask_utils.py:8-38: prepend always-attend columns."""
    fill = True if mask.dtype == torch.bool else 0.0
    return torch.cat([mask.new_full((*mask.shape[:-1], num_cold), fill), mask], dim=-1)


def kiv_decode_attention(query, hot_k, hot_v, cold_k, cold_v, mask, scaling):
    """The wrapper's decode step (kiv/middleware.py:330-354) with eager attention:
    crop the mask to the hot window, put retrieved keys first, extend the mask."""
    if cold_k is not None:
        hot_len = hot_k.shape[2]
        if mask is not None and mask.shape[-1] > hot_len:
            mask = mask[..., -hot_len:]
        hot_k = torch.cat([cold_k, hot_k], dim=2)
        hot_v = torch.cat([cold_v, hot_v], dim=2)
        if mask is not None:
            mask = extend_mask(mask, cold_k.shape[2])
    return eager_attention(query, hot_k, hot_v, mask, scaling)


def decode_step(store: OracleColdStore, query, hot_k, hot_v, mask, scaling, top_p, top_pages):
    """Retrieve then attend: the CPU baseline of one layer's decode step."""
    ck, cv, trace = store.retrieve(query, scaling, top_p, top_pages)
    return kiv_decode_attention(query, hot_k, hot_v, ck, cv, mask, scaling), trace
