"""The matrix-core attention inside a model: chunked prefill and the
reuse-path forward (a follow-up prompt on a cache with a cold tier) of a
random-init bf16 Qwen2 with head_dim 64.

A spy around the kernel checks, for every call the model makes, that it
ran on every global layer of every chunk and that its output on the actual
inputs (mask as the model built it, retrieved keys, causal rule) is within
the bound of tests/test_gpu_prefill.py of fp64 attention over the same
[retrieved ; hot] keys.  The same token sequence also runs with the kernel
disabled, which takes the reference's route (kiv/middleware.py:174-260 and
330-354: the original attention function, after concatenating [retrieved ;
hot] and widening the mask for the reuse path).  The two runs differ by the
attention's rounding, which bf16 hidden states carry from layer to layer
(and which can flip a retrieval choice near a tie in later decode steps),
so their logits are compared coarsely: relative Frobenius difference below
5e-2 (measured: 0.005 to 0.03).
"""

from __future__ import annotations

import pytest
import torch

import kiv_amd.middleware as mwmod
from kiv_amd import KIVConfig, KIVMiddleware
from tests.test_gpu_prefill import check

pytestmark = pytest.mark.gpu


def bf16_qwen2(cuda, attn: str, layers: int = 2):
    from transformers import Qwen2Config, Qwen2ForCausalLM

    cfg = Qwen2Config(vocab_size=512, hidden_size=256, intermediate_size=512, num_hidden_layers=layers,
                      num_attention_heads=4, num_key_value_heads=2, head_dim=64, max_position_embeddings=8192,
                      tie_word_embeddings=False)
    cfg._attn_implementation = attn
    torch.manual_seed(0)
    return Qwen2ForCausalLM(cfg).to(torch.bfloat16).to(cuda).eval()


def run(cuda, attn, kernel: bool, monkeypatch, cap=None, follow=0, decode=0, batch=1):
    """Logits of [prefill last token, decode steps..., follow-up forward] and
    the number of kernel calls."""
    calls = []
    real = mwmod.prefill_attention

    def spy(query, cold_k, cold_v, key, value, mask, scaling, causal=False):
        calls.append(cold_k is not None)  # True when retrieved keys are attended
        out = real(query, cold_k, cold_v, key, value, mask, scaling, causal=causal)
        check(query, cold_k, cold_v, key, value, scaling, mask=mask, causal=causal, out=out)
        return out

    monkeypatch.setattr(mwmod, "prefill_attention", spy)
    if not kernel:
        monkeypatch.setattr(mwmod, "prefill_supported", lambda *a, **k: False)
    model = bf16_qwen2(cuda, attn)
    mw = KIVMiddleware(model, KIVConfig(hot_budget=160, top_p=48, page_size=16, top_pages=4))
    mw.install()
    outs = []
    try:
        cache = mw.create_cache(cuda)
        gen = torch.Generator().manual_seed(5)
        ids = torch.randint(0, 512, (batch, 700), generator=gen).to(cuda)
        with torch.no_grad():
            outs.append(mw.chunked_prefill(ids, cache, chunk_size=256, prefill_hot_cap=cap).float())
            for _ in range(decode):
                tok = outs[-1].argmax(-1, keepdim=True)
                outs.append(model(input_ids=tok, past_key_values=cache, use_cache=True).logits[:, -1].float())
            if follow:
                f = torch.randint(0, 512, (batch, follow), generator=gen).to(cuda)
                outs.append(model(input_ids=f, past_key_values=cache, use_cache=True).logits.float())
        cold = cache.get_cold_store(0).cold_length
    finally:
        mw.uninstall()
        monkeypatch.undo()
    return outs, calls, cold


def rel(a, b):
    return ((a - b).norm() / b.norm()).item()


@pytest.mark.parametrize("attn", ["sdpa", "eager"])
def test_chunked_prefill_runs_on_the_kernel(cuda, attn, monkeypatch):
    print(f"chunked prefill {attn}", flush=True)
    got, calls, _ = run(cuda, attn, True, monkeypatch)
    ref, ref_calls, _ = run(cuda, attn, False, monkeypatch)
    assert len(calls) == 2 * 3 and not any(calls) and ref_calls == []  # 2 layers x 3 chunks
    print("logits relative difference", rel(got[0], ref[0]), flush=True)
    assert rel(got[0], ref[0]) < 5e-2


@pytest.mark.parametrize("batch", [1, 2])
def test_capped_prefill_and_reuse_forward_with_cold_tier(cuda, monkeypatch, batch):
    """prefill_hot_cap evicts between chunks (masks with an offset), then
    decode steps and a 200-token follow-up that retrieves from the cold tier
    and attends [retrieved ; hot] on the kernel; one and two sequences."""
    print(f"capped prefill + reuse forward, batch {batch}", flush=True)
    got, calls, cold = run(cuda, "sdpa", True, monkeypatch, cap=200, follow=200, decode=2, batch=batch)
    ref, _, ref_cold = run(cuda, "sdpa", False, monkeypatch, cap=200, follow=200, decode=2, batch=batch)
    assert cold > 0 and cold == ref_cold
    assert calls.count(False) == 2 * 3 and calls.count(True) == 2  # chunks, then the follow-up per layer
    diffs = [rel(g, r) for g, r in zip(got, ref)]
    print("logits relative differences", diffs, flush=True)
    assert max(diffs) < 5e-2
