"""float64 restatement of the tiered-cache path, plus dtype-rounding emulation.

Test infrastructure only (see oracle/__init__.py).  Every function names the
reference lines it restates.
"""

from __future__ import annotations

import numpy as np


# ------------------------------------------------------------ dtype rounding

def round_to_dtype(x: np.ndarray, dtype: str) -> np.ndarray:
    """Round float64/float32 values to bf16 / fp16 / fp32 (nearest-even), as float64.

    fp32 -> bf16 keeps the top 16 bits of the fp32 pattern after adding
    0x7fff + lsb (round half to even); fp16 uses numpy's IEEE conversion.
    """
    x32 = np.asarray(x, dtype=np.float32)
    if dtype == "float32":
        return x32.astype(np.float64)
    if dtype == "float16":
        return x32.astype(np.float16).astype(np.float64)
    if dtype == "bfloat16":
        u = x32.view(np.uint32).astype(np.uint64)
        r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
        nan = np.isnan(x32)
        out = r.astype(np.uint32).view(np.float32).astype(np.float64)
        out[nan] = np.nan
        return out
    raise ValueError(dtype)


def emulate_scores(dot32: np.ndarray, scaling: float, dtype: str) -> np.ndarray:
    """Score as ``torch.matmul(q, k^T) * scaling`` gives it in the activation dtype.

    kiv/cold_store.py:206-208 and :333-335: the matmul result (fp32
    accumulated) is rounded to the dtype, multiplied by the scale in fp32 and
    rounded again.  ``dot32`` must already be the fp32 dot product.
    """
    s = round_to_dtype(dot32, dtype).astype(np.float32)
    return round_to_dtype(s * np.float32(scaling), dtype)


# ----------------------------------------------------------------- geometry

def expand_kv(x: np.ndarray, groups: int) -> np.ndarray:
    """[B, Hkv, T, D] -> [B, Hkv*groups, T, D]; q head h reads kv head h // groups.

    kiv/cold_store.py:23-32 (_repeat_kv).
    """
    return np.repeat(x, groups, axis=1)


# ----------------------------------------------------------------- summaries

def page_means(k_cold: np.ndarray, page_size: int) -> np.ndarray:
    """Mean of each full page's K rows: [B, Hkv, N, D] in float64.

    kiv/cold_store.py:160-165 (summary = page_k.mean(dim=2)).
    """
    B, H, T, D = k_cold.shape
    n = T // page_size
    pages = k_cold[:, :, : n * page_size].astype(np.float64).reshape(B, H, n, page_size, D)
    return pages.mean(axis=3)


# -------------------------------------------------------------------- scores

def grouped_dots(q: np.ndarray, keys: np.ndarray, groups: int, absolute: bool = False) -> np.ndarray:
    """Exact (float64) q.k of q [B, Hq, Q, D] against keys [B, Hkv, T, D]:
    [B, Hq, Q, T], q head h against kv head h // groups, without
    materialising the expanded keys.  ``absolute``: sum of |q_i k_i|."""
    B, Hq, Q, D = q.shape
    q64 = q.astype(np.float64).reshape(B, Hq // groups, groups, Q, D)
    k64 = keys.astype(np.float64)
    if absolute:
        q64, k64 = np.abs(q64), np.abs(k64)
    return np.matmul(q64, k64[:, :, None].swapaxes(-1, -2)).reshape(B, Hq, Q, keys.shape[2])


def scores64(q: np.ndarray, keys: np.ndarray, scaling: float, groups: int) -> np.ndarray:
    """q [B, Hq, Q, D] against keys [B, Hkv, T, D]: [B, Hq, Q, T] float64 q.k * scaling."""
    return grouped_dots(q, keys, groups) * scaling


def dots32(q: np.ndarray, keys: np.ndarray, groups: int) -> np.ndarray:
    """fp32 dot products (fp64 accumulation rounded once to fp32)."""
    return grouped_dots(q, keys, groups).astype(np.float32)


# ----------------------------------------------------------------- selection

def top_k_set(scores: np.ndarray, k: int) -> tuple[np.ndarray, float]:
    """Indices of the k largest entries of a 1-D array (lower index wins ties)
    and the gap between the k-th and (k+1)-th largest values (inf if k == n)."""
    order = np.lexsort((np.arange(scores.size), -scores))
    sel = np.sort(order[:k])
    if k >= scores.size:
        return sel, float("inf")
    return sel, float(scores[order[k - 1]] - scores[order[k]])


def coarse_union(coarse: np.ndarray, top_pages: int) -> tuple[np.ndarray, float]:
    """Union over (b, h, q) of each row's top pages, sorted, and the smallest
    selection gap among the rows.  kiv/cold_store.py:211-224."""
    B, H, Q, N = coarse.shape
    k = min(top_pages, N)
    pages, gap = set(), float("inf")
    for row in coarse.reshape(-1, N):
        sel, g = top_k_set(row, k)
        pages.update(sel.tolist())
        gap = min(gap, g)
    return np.array(sorted(pages), dtype=np.int64), gap


def candidate_ids(pages: np.ndarray, page_size: int, num_finalized: int, partial_len: int) -> np.ndarray:
    """Finished pages' tokens ascending, then the partial page's tokens.

    kiv/cold_store.py:227-262.
    """
    ids = (pages[:, None] * page_size + np.arange(page_size)[None, :]).reshape(-1)
    return np.concatenate([ids, num_finalized + np.arange(partial_len)]).astype(np.int64)


def fine_aggregate(fine: np.ndarray) -> np.ndarray:
    """max over query heads and positions: [B, Hq, Q, C] -> [B, C].

    kiv/cold_store.py:338 (amax(dim=(1, 2))).
    """
    return fine.max(axis=(1, 2))


# ----------------------------------------------------------------- attention

def attention64(q: np.ndarray, keys: np.ndarray, values: np.ndarray, scaling: float,
                mask: np.ndarray | None = None) -> np.ndarray:
    """Softmax attention in float64; q [B,Hq,Q,D], keys/values [B,Hkv,T,D],
    additive mask broadcastable to [B,Hq,Q,T].  Returns [B, Q, Hq, D].

    Transformers' eager_attention_forward (models/qwen2/modeling_qwen2.py:150-172)
    in exact arithmetic.
    """
    groups = q.shape[1] // keys.shape[1]
    s = scores64(q, keys, scaling, groups)
    if mask is not None:
        s = s + mask
    s = s - s.max(axis=-1, keepdims=True)
    w = np.exp(s)
    w = w / w.sum(axis=-1, keepdims=True)
    out = np.einsum("bhqt,bhtd->bhqd", w, expand_kv(values.astype(np.float64), groups))
    return out.transpose(0, 2, 1, 3)
