"""GPU parity of the matrix-core attention for queries of many positions
(kiv_prefill_attention): prefill chunks and long queries over
[retrieved ; hot].

Reference: transformers' eager attention (scores * scaling + mask, fp32
softmax, probabilities rounded to the dtype, @ V), restated in fp64 by
oracle.exact.attention64.  Bar per output element:

    |out - fp64| <= 2e-3 + half an ulp of the dtype at the fp64 value
                    + u * sum_k p_k |v_k|

The last term is the rounding of the probabilities to the dtype before
they weight V (u = 2^-9 for bf16, 2^-12 for fp16, the unit roundoff; the
reference rounds them as well), computed exactly as the fp64 attention of
|V|.  A dropped rescale, a wrong key or a transposed operand moves outputs
by O(|v|), far outside it.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from kiv_amd.attention import prefill_attention, prefill_supported
from oracle import exact

pytestmark = pytest.mark.gpu

UNIT_ROUNDOFF = {torch.bfloat16: 2.0 ** -9, torch.float16: 2.0 ** -12}
ULP_SCALE = {torch.bfloat16: 2.0 ** 16, torch.float16: 2.0 ** 13}


def f64(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy().astype(np.float64)


def causal_bias(Q: int, T: int) -> np.ndarray:
    """Additive [Q, T] bias: hot column t visible to row i iff t <= i + T - Q."""
    i = np.arange(Q)[:, None]
    t = np.arange(T)[None, :]
    return np.where(t <= i + (T - Q), 0.0, -np.inf)


def check(q, cold_k, cold_v, hot_k, hot_v, scaling, mask=None, causal=False, out=None):
    """prefill_attention (or its given output ``out``) against the fp64 bound."""
    if out is None:
        out = prefill_attention(q, cold_k, cold_v, hot_k, hot_v, mask, scaling, causal=causal)
    torch.cuda.synchronize()
    B, hq, Q, D = q.shape
    T = hot_k.shape[2]
    P = 0 if cold_k is None else cold_k.shape[2]
    keys = torch.cat([cold_k, hot_k], dim=2) if P else hot_k
    vals = torch.cat([cold_v, hot_v], dim=2) if P else hot_v
    if mask is not None:
        mm = torch.where(mask, 0.0, float("-inf")) if mask.dtype == torch.bool else mask.float()
        hot_bias = f64(mm)
        if hot_bias.ndim == 2:
            hot_bias = hot_bias[:, None, None, :]
    elif causal:
        hot_bias = causal_bias(Q, T)[None, None]
    else:
        hot_bias = np.zeros((1, 1, 1, T))
    hot_bias = np.broadcast_to(hot_bias, np.broadcast_shapes(hot_bias.shape, (1, 1, Q, T)))
    bias = np.concatenate([np.zeros(hot_bias.shape[:-1] + (P,)), hot_bias], axis=-1)
    ref = exact.attention64(f64(q), f64(keys), f64(vals), scaling, bias)
    wabs = exact.attention64(f64(q), f64(keys), np.abs(f64(vals)), scaling, bias)
    half_ulp = 0.5 * np.spacing(np.abs(ref).astype(np.float32)) * ULP_SCALE[q.dtype]
    tol = 2e-3 + half_ulp + UNIT_ROUNDOFF[q.dtype] * wabs
    err = np.abs(f64(out) - ref)
    assert out.shape == (B, Q, hq, D)
    assert np.all(np.isfinite(f64(out)))
    assert np.all(err <= tol), f"max-abs error {err.max()} (excess over bound {(err - tol).max()})"
    return out, err.max()


def rand(shape, dtype, gen, scale=1.0):
    return (torch.randn(shape, generator=gen) * scale).to(dtype)


CASES = [
    # name, B, Hq, Hkv, D, Q, retrieved P, hot T, dtype, mask ("causal" | "none" | "bool" | "float" | "bool2d")
    ("first_chunk_causal_gqa", 1, 12, 2, 128, 300, 0, 300, torch.bfloat16, "causal"),
    ("chunk_with_past_causal", 1, 8, 8, 64, 200, 0, 456, torch.float16, "causal"),
    ("retrieved_plus_hot_bool", 2, 8, 2, 128, 130, 100, 400, torch.bfloat16, "bool"),
    ("float_mask_d96", 1, 6, 3, 96, 77, 33, 250, torch.float16, "float"),
    ("no_mask_d256_partial_tiles", 1, 4, 1, 256, 17, 70, 90, torch.bfloat16, "none"),
    ("d32_bool_2d", 2, 4, 2, 32, 64, 0, 190, torch.bfloat16, "bool2d"),
    ("d192_causal", 1, 4, 2, 192, 65, 5, 129, torch.float16, "causal"),
    ("single_row", 1, 8, 2, 128, 1, 64, 64, torch.bfloat16, "causal"),
    # skipped, whole and partial column tiles of a mask tensor in one call
    ("bool_mask_tile_classes", 1, 4, 1, 64, 256, 0, 640, torch.bfloat16, "bool"),
    ("float_mask_tile_classes", 1, 4, 2, 128, 192, 40, 700, torch.bfloat16, "float"),
    # queries too short to fill the GPU: keys split across blocks, then merged
    ("short_query_key_splits", 1, 8, 2, 128, 40, 300, 1500, torch.bfloat16, "bool"),
    ("short_causal_key_splits_d64", 1, 4, 4, 64, 70, 0, 900, torch.float16, "causal"),
    ("d256_key_splits_batch", 2, 4, 1, 256, 20, 64, 500, torch.bfloat16, "none"),
]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_prefill_attention(cuda, case):
    name, B, hq, hkv, D, Q, P, T, dt, mk = case
    print(f"prefill attention case {name}", flush=True)
    gen = torch.Generator().manual_seed(sum(map(ord, name)))
    q = rand((B, hq, Q, D), dt, gen).to(cuda)
    hot_k = rand((B, hkv, T, D), dt, gen).to(cuda)
    hot_v = rand((B, hkv, T, D), dt, gen).to(cuda)
    cold_k = rand((B, hkv, P, D), dt, gen).to(cuda) if P else None
    cold_v = rand((B, hkv, P, D), dt, gen).to(cuda) if P else None
    scaling = D ** -0.5
    mask, causal = None, mk == "causal"
    if mk in ("bool", "float"):
        # causal structure plus a random left padding per batch row
        vis = torch.from_numpy(causal_bias(Q, T) == 0)[None, None].repeat(B, 1, 1, 1)
        for b in range(B):
            vis[b, :, :, : 3 + 11 * b] = False
        mask = vis if mk == "bool" else torch.where(vis, 0.0, torch.finfo(dt).min).to(dt)
        mask = mask.to(cuda)
    elif mk == "bool2d":
        vis = torch.ones(B, T, dtype=torch.bool)
        vis[0, :40] = False
        mask = vis.to(cuda)
    assert prefill_supported(q, hot_k, mask)
    check(q, cold_k, cold_v, hot_k, hot_v, scaling, mask=mask, causal=causal)


def test_prefill_attention_peaked_scores(cuda):
    """Queries aligned with a few keys (softmax close to one-hot): the
    probability rounding term is at its largest here."""
    gen = torch.Generator().manual_seed(7)
    B, hq, hkv, D, Q, T = 1, 8, 2, 128, 96, 512
    dt = torch.bfloat16
    hot_k = rand((B, hkv, T, D), dt, gen).to(cuda)
    hot_v = rand((B, hkv, T, D), dt, gen, scale=3.0).to(cuda)
    idx = torch.randint(0, T - Q, (Q,), generator=gen)
    base = hot_k.float().cpu()[:, :, idx].repeat_interleave(hq // hkv, dim=1)
    q = (base * 4.0 + torch.randn(B, hq, Q, D, generator=gen) * 0.1).to(dt).to(cuda)
    check(q, None, None, hot_k, hot_v, D ** -0.5, causal=True)


def test_prefill_attention_strided_views(cuda):
    """q as the [B, Q, Hq, D] projection transposed (the layout HF passes) and
    hot K/V as a window of a larger buffer."""
    gen = torch.Generator().manual_seed(11)
    B, hq, hkv, D, Q, T = 1, 12, 2, 128, 150, 333
    dt = torch.bfloat16
    q = rand((B, Q, hq, D), dt, gen).to(cuda).transpose(1, 2)
    buf_k = rand((B, hkv, T + 100, D), dt, gen).to(cuda)
    buf_v = rand((B, hkv, T + 100, D), dt, gen).to(cuda)
    hot_k, hot_v = buf_k[:, :, 40:40 + T], buf_v[:, :, 40:40 + T]
    check(q, None, None, hot_k, hot_v, D ** -0.5, causal=True)


def test_prefill_attention_fully_masked_rows_are_zero(cuda):
    gen = torch.Generator().manual_seed(3)
    B, hq, hkv, D, Q, T = 1, 4, 2, 64, 70, 128
    dt = torch.float16
    q = rand((B, hq, Q, D), dt, gen).to(cuda)
    hot_k = rand((B, hkv, T, D), dt, gen).to(cuda)
    hot_v = rand((B, hkv, T, D), dt, gen).to(cuda)
    vis = torch.ones(B, 1, Q, T, dtype=torch.bool)
    vis[:, :, 5] = False
    vis[:, :, 66] = False
    out = prefill_attention(q, None, None, hot_k, hot_v, vis.to(cuda), D ** -0.5)
    torch.cuda.synchronize()
    assert torch.count_nonzero(out[:, [5, 66]]) == 0
    keep = [i for i in range(Q) if i not in (5, 66)]
    sub_vis = vis[:, :, keep].to(cuda)
    ref_out, _ = check(q[:, :, keep].contiguous(), None, None, hot_k, hot_v, D ** -0.5, mask=sub_vis)
    assert torch.equal(out[:, keep], ref_out)


def test_prefill_attention_model_chunk_full_size(cuda):
    """The whole-model run's chunk shape at full size: 4096 query positions
    over 8192 hot keys (hot cap 4096 + chunk 4096), 12 q / 2 kv heads, head
    dim 128, bf16, the model's boolean causal mask.  This is the launch the
    longest-first grid splits over key ranges and merges (3 splits on a
    256-CU GPU).  The fp64 reference runs on the GPU, one head at a time, and
    the bar is the module's."""
    B, hq, hkv, D, Q, T = 1, 12, 2, 128, 4096, 8192
    dt = torch.bfloat16
    gen = torch.Generator(device=cuda).manual_seed(4096)
    q = torch.randn(B, hq, Q, D, generator=gen, device=cuda).to(dt)
    hot_k = torch.randn(B, hkv, T, D, generator=gen, device=cuda).to(dt)
    hot_v = torch.randn(B, hkv, T, D, generator=gen, device=cuda).to(dt)
    vis = torch.from_numpy(causal_bias(Q, T) == 0)[None, None].to(cuda)
    scaling = D ** -0.5
    out = prefill_attention(q, None, None, hot_k, hot_v, vis, scaling)
    torch.cuda.synchronize()
    assert out.shape == (B, Q, hq, D)
    bias = torch.where(vis[0, 0], 0.0, float("-inf")).to(torch.float64)
    worst = 0.0
    for h in range(hq):
        q64 = q[0, h].double()
        k64 = hot_k[0, h // (hq // hkv)].double()
        v64 = hot_v[0, h // (hq // hkv)].double()
        s = q64 @ k64.t().contiguous() * scaling + bias
        prob = torch.softmax(s, dim=-1)
        ref = prob @ v64
        wabs = prob @ v64.abs()
        del s, prob
        half_ulp = 0.5 * torch.from_numpy(
            np.spacing(np.abs(ref.float().cpu().numpy())).astype(np.float64)).to(cuda) * ULP_SCALE[dt]
        tol = 2e-3 + half_ulp + UNIT_ROUNDOFF[dt] * wabs
        err = (out[0, :, h].double() - ref).abs()
        assert torch.isfinite(out[0, :, h].float()).all()
        excess = (err - tol).max().item()
        worst = max(worst, err.max().item())
        assert excess <= 0, f"head {h}: max-abs error {err.max().item()} (excess over bound {excess})"
    print(f"model chunk 4096 x 8192: max-abs error {worst:.3e}", flush=True)


def test_prefill_attention_rejects_bad_arguments(cuda):
    dt = torch.bfloat16
    q = torch.zeros(1, 4, 8, 80, dtype=dt, device=cuda)
    k = torch.zeros(1, 2, 8, 80, dtype=dt, device=cuda)
    assert not prefill_supported(q, k, None)
    with pytest.raises(RuntimeError, match="head_dim 80"):
        prefill_attention(q, None, None, k, k, None, 1.0)
    q = torch.zeros(1, 4, 8, 64, dtype=torch.float32, device=cuda)
    k = torch.zeros(1, 2, 8, 64, dtype=torch.float32, device=cuda)
    with pytest.raises(RuntimeError, match="fp16/bf16"):
        prefill_attention(q, None, None, k, k, None, 1.0)
