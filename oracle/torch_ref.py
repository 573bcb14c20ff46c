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


class OracleColdStore:
    """ColdKVStore semantics (kiv/cold_store.py:35-414) on CPU, no telemetry."""

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
        keeps bulk evictions linear; the stored values are the same."""
        self._flat = None
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
            tok = (pages[:, None] * ps + torch.arange(ps)[None, :]).reshape(-1)
            ks.append(kall[:, :, tok])
            vs.append(vall[:, :, tok])
            ids.append(tok)
            trace.coarse_scores, trace.pages = coarse, pages
        if self.partial_len:
            n_fin = self.num_pages * ps
            ks.append(self.partial_k)
            vs.append(self.partial_v)
            ids.append(torch.arange(n_fin, n_fin + self.partial_len))
        return torch.cat(ks, dim=2), torch.cat(vs, dim=2), torch.cat(ids)

    # kiv/cold_store.py:283-371
    def retrieve(self, query: torch.Tensor, scaling: float, top_p: int, top_pages: int):
        """(K [B,Hkv,P',D], V, trace) or (None, None, trace) when cold is empty."""
        trace = RetrieveTrace()
        if self.cold_length == 0:
            return None, None, trace
        P = min(top_p, self.cold_length)
        ck, cv, cid = self.candidates(query, scaling, top_pages, trace)
        fine = torch.matmul(query, expand_kv(ck, self.groups).transpose(-2, -1)) * scaling
        agg = fine.amax(dim=(1, 2))
        _, top_local = agg.topk(min(P, agg.shape[-1]), dim=-1)
        idx = top_local[:, None, :, None].expand(-1, ck.shape[1], -1, ck.shape[3])
        trace.candidate_ids, trace.agg_scores, trace.top_local = cid, agg, top_local
        trace.selected_ids = cid[top_local]
        return torch.gather(ck, 2, idx), torch.gather(cv, 2, idx), trace


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
