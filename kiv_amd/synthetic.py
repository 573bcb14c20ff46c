"""Seeded synthetic decode workloads for the tiered cache.

Generator (all draws fp32 from one seeded ``torch.Generator``, then cast):
  * centroids c[h, j] ~ N(0, I_D) per KV head h and segment j;
  * K[h, t] = c[h, t // seg] + 0.3 * N(0, I_D) over cold then hot positions;
  * V iid N(0, 1);
  * query row i (q head i, KV head i // G) = c[i // G, j*[i mod n_targets]]
    + 0.1 * N(0, I_D), targets j* uniform over the cold segments;
  * scaling = D ** -0.5, batch 1, one query position.
Draw order: centroids, targets, K noise, V, query noise.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, replace

import torch


@dataclass(frozen=True)
class Workload:
    name: str
    num_q_heads: int
    num_kv_heads: int
    head_dim: int
    dtype: torch.dtype
    hot: int
    cold: int
    top_pages: int
    top_p: int
    segment: int
    n_targets: int = 1
    page_size: int = 128

    @property
    def groups(self) -> int:
        return self.num_q_heads // self.num_kv_heads

    @property
    def scaling(self) -> float:
        return self.head_dim ** -0.5

    def with_cold(self, cold: int) -> "Workload":
        return replace(self, cold=cold)


WORKLOADS = {
    # TinyLlama-1.1B attention shape, 32,768 cold tokens.
    "tinyllama_32k": Workload("tinyllama_32k", 32, 4, 64, torch.float16, 2048, 32768, 32, 256, 1024),
    # Qwen2.5-7B attention shape, 262,144 cold tokens.
    "qwen7b_256k": Workload("qwen7b_256k", 28, 4, 128, torch.bfloat16, 2048, 262144, 32, 256, 1024),
    # Phi-3.5-mini MHA shape, 131,072 cold tokens, 4 target segments.
    "phi35_128k": Workload("phi35_128k", 32, 32, 96, torch.float16, 2048, 131072, 64, 512, 512, n_targets=4),
    # MQA shape, 1,048,576 cold tokens.
    "mqa_1m": Workload("mqa_1m", 8, 1, 256, torch.bfloat16, 4096, 1048576, 64, 1024, 2048),
    # Qwen2.5-1.5B attention shape, one layer of the whole-model run's cold tier.
    "qwen15b_layer_1m": Workload("qwen15b_layer_1m", 12, 2, 128, torch.bfloat16, 2048, 1046528, 32, 256, 1024),
    # Qwen2.5-7B attention shape, 1,048,576 cold tokens (the headline workload).
    "qwen7b_1m": Workload("qwen7b_1m", 28, 4, 128, torch.bfloat16, 2048, 1048576, 32, 256, 1024),
}


def _split(x: torch.Tensor, cold: int):
    return x[:, :cold], x[:, cold:]


def generate(w: Workload, seed: int = 0, device: str | torch.device = "cpu", batch: int = 1) -> dict:
    """Whole workload in one draw: q [B,Hq,1,D], cold/hot K,V [B,Hkv,T,D]."""
    g = torch.Generator(device=device).manual_seed(seed)
    total = w.cold + w.hot
    nseg = math.ceil(total / w.segment)
    cold_seg = max(1, math.ceil(w.cold / w.segment))
    f32 = dict(dtype=torch.float32, device=device, generator=g)
    out = {"q": [], "cold_k": [], "cold_v": [], "hot_k": [], "hot_v": [], "targets": []}
    for _ in range(batch):
        cent = torch.randn(w.num_kv_heads, nseg, w.head_dim, **f32)
        targets = torch.randint(0, cold_seg, (w.n_targets,), generator=g, device=device)
        seg_of = torch.arange(total, device=device) // w.segment
        k = cent[:, seg_of] + 0.3 * torch.randn(w.num_kv_heads, total, w.head_dim, **f32)
        v = torch.randn(w.num_kv_heads, total, w.head_dim, **f32)
        heads = torch.arange(w.num_q_heads, device=device)
        q = cent[heads // w.groups, targets[heads % w.n_targets]]
        q = q + 0.1 * torch.randn(w.num_q_heads, w.head_dim, **f32)
        ck, hk = _split(k, w.cold)
        cv, hv = _split(v, w.cold)
        out["q"].append(q[:, None])
        out["cold_k"].append(ck)
        out["cold_v"].append(cv)
        out["hot_k"].append(hk)
        out["hot_v"].append(hv)
        out["targets"].append(targets)
    res = {key: torch.stack(val).to(w.dtype) if key != "targets" else torch.stack(val)
           for key, val in out.items()}
    res["scaling"] = w.scaling
    return res


def generate_streaming(w: Workload, seed: int, device: str | torch.device, chunk: int = 65536):
    """Large workloads without holding the cold tier in memory twice.

    Yields ("cold", k_chunk, v_chunk) pieces in position order, then one
    ("hot", k, v) and finally ("query", q, targets).  Same distribution as
    :func:`generate` (different draws: the noise is drawn per chunk).
    """
    g = torch.Generator(device=device).manual_seed(seed)
    total = w.cold + w.hot
    nseg = math.ceil(total / w.segment)
    cold_seg = max(1, math.ceil(w.cold / w.segment))
    f32 = dict(dtype=torch.float32, device=device, generator=g)
    cent = torch.randn(w.num_kv_heads, nseg, w.head_dim, **f32)
    targets = torch.randint(0, cold_seg, (w.n_targets,), generator=g, device=device)

    def rows(t0: int, t1: int):
        seg_of = torch.arange(t0, t1, device=device) // w.segment
        k = cent[:, seg_of] + 0.3 * torch.randn(w.num_kv_heads, t1 - t0, w.head_dim, **f32)
        v = torch.randn(w.num_kv_heads, t1 - t0, w.head_dim, **f32)
        return k.to(w.dtype)[None], v.to(w.dtype)[None]

    for t0 in range(0, w.cold, chunk):
        yield ("cold",) + rows(t0, min(w.cold, t0 + chunk))
    yield ("hot",) + rows(w.cold, total)
    heads = torch.arange(w.num_q_heads, device=device)
    q = cent[heads // w.groups, targets[heads % w.n_targets]]
    q = q + 0.1 * torch.randn(w.num_q_heads, w.head_dim, **f32)
    yield ("query", q.to(w.dtype)[None, :, None], targets)
