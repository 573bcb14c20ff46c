"""The whole-model configuration at its stated shape.

A random-init decoder of the Qwen2.5-1.5B shape (28 layers, hidden 1536, 12
q heads / 2 kv heads, head_dim 128, bf16) prefills 1,048,576 random token
ids through KIVMiddleware.chunked_prefill (chunk 4096, hot cap 4096), then
takes 128 greedy decode steps with live retrieval on every layer (hot 2048,
top_pages 32, top_p 256).  After prefill the cold tier holds exactly 8,176
pages per layer, so the 128th step's eviction finishes page 8,176 on every
layer (the page-end finalize of a decode step, at model scale).

For four layers spread over the depth, the cold tier is read back after the
last step and evicted into the CPU oracle, and the last step's retrieval
(its union and selection, from the telemetry) is checked with the query the
layer used: every page summary against the fp64 means (the new page
included), the new page's rows against the hot-window rows it took, then a
retrieval on the same state within the rounding bands, equal to the oracle
where the bands determine it, differing from it only within 1e-3 of a
selection boundary, with bit-exact K/V rows, and identical to what the
decode step selected.
"""

from __future__ import annotations

import gc

import numpy as np
import pytest
import torch

from kiv_amd import ColdKVStore, KIVConfig, KIVMiddleware
from kiv_amd.synthetic import Workload
from oracle.torch_ref import OracleColdStore
from tests.test_gpu_configs import check_summaries_in_pieces
from tests.test_gpu_retrieval import check_retrieval, separation_line

pytestmark = pytest.mark.gpu

TOKENS, CHUNK, CAP = 1 << 20, 4096, 4096
LAYERS_CHECKED = (0, 9, 18, 27)
STEPS = 128


@pytest.mark.timeout(900)
def test_qwen15b_shape_million_token_prefill_then_128_decode_steps(cuda, monkeypatch):
    from transformers import Qwen2Config, Qwen2ForCausalLM

    cfg = Qwen2Config(vocab_size=151936, hidden_size=1536, intermediate_size=8960, num_hidden_layers=28,
                      num_attention_heads=12, num_key_value_heads=2, max_position_embeddings=TOKENS + 8192,
                      rope_theta=1e6, tie_word_embeddings=True)
    cfg._attn_implementation = "sdpa"
    torch.manual_seed(0)
    with torch.device(cuda):
        model = Qwen2ForCausalLM(cfg)
    model = model.to(torch.bfloat16).eval()
    kcfg = KIVConfig(hot_budget=2048, top_p=256, page_size=128, top_pages=32)
    mw = KIVMiddleware(model, kcfg)
    mw.install()
    try:
        cache = mw.create_cache(cuda)
        ids = torch.randint(0, cfg.vocab_size, (1, TOKENS), generator=torch.Generator().manual_seed(0)).to(cuda)
        print(f"c5: prefill {TOKENS} tokens (chunk {CHUNK}, hot cap {CAP}) ...", flush=True)
        with torch.no_grad():
            logits = mw.chunked_prefill(ids, cache, chunk_size=CHUNK, prefill_hot_cap=CAP)
        torch.cuda.synchronize()
        cold = cache.get_cold_store(0).cold_length
        print(f"c5: prefill done, {cold} cold tokens per layer", flush=True)
        assert cold == TOKENS - kcfg.hot_budget

        # The hot window's oldest 128 rows of the checked layers: the rows the
        # decode steps evict, which fill page 8,176.
        first_out = {}
        for layer in LAYERS_CHECKED:
            hl = cache.layers[layer]
            first_out[layer] = (hl.keys[:, :, :STEPS].cpu(), hl.values[:, :, :STEPS].cpu())

        # Greedy decode; record each store's query (the last step's stays).
        seen = {}
        orig = ColdKVStore._retrieve

        def spy(self, query, scaling, kiv_config, step, attend, *rest, **kw):
            seen[id(self)] = (query.detach().clone(), scaling)
            return orig(self, query, scaling, kiv_config, step, attend, *rest, **kw)

        monkeypatch.setattr(ColdKVStore, "_retrieve", spy)
        tok = logits.argmax(-1, keepdim=True)
        tokens = []
        with torch.no_grad():
            for step in range(STEPS):
                out = model(input_ids=tok, past_key_values=cache, use_cache=True)
                tok = out.logits[:, -1].argmax(-1, keepdim=True)
                tokens.append(int(tok))
                if step in (0, STEPS - 2, STEPS - 1):
                    torch.cuda.synchronize()
                    st = cache.get_cold_store(0)
                    print(f"c5: decode step {step + 1}: cold {st.cold_length} tokens, {st.num_pages} pages, "
                          f"partial {st.cold_length - st.num_pages * 128}", flush=True)
                    assert torch.isfinite(out.logits).all()
        torch.cuda.synchronize()
        monkeypatch.setattr(ColdKVStore, "_retrieve", orig)
        assert len(seen) == cfg.num_hidden_layers
        pages0 = (TOKENS - kcfg.hot_budget) // 128
        for layer in range(cfg.num_hidden_layers):
            st = cache.get_cold_store(layer)
            assert st.cold_length == TOKENS - kcfg.hot_budget + STEPS and st.num_pages == pages0 + 1
        print(f"c5: {STEPS} greedy steps, tokens {tokens[:8]}...{tokens[-4:]}", flush=True)

        for layer in LAYERS_CHECKED:
            store = cache.get_cold_store(layer)
            q, scaling = seen[id(store)]
            snap = store.telemetry_snapshot()
            rec = snap["recent"]
            assert snap["aggregates"]["fine_calls"] == STEPS and len(rec) == 2 * STEPS
            assert all(r["actual_P"] == kcfg.top_p for r in rec if r["kind"] == "fine")
            step_coarse, step_fine = rec[-2], rec[-1]
            assert step_coarse["kind"] == "coarse" and step_fine["kind"] == "fine"
            assert step_coarse["num_pages"] == pages0 + 1
            k_host, v_host = (t.cpu() for t in store.read_tokens())
            # The page the decode steps finished holds the rows they evicted.
            ok, ov = first_out[layer]
            t0 = pages0 * 128
            assert torch.equal(k_host[:, :, t0:t0 + STEPS], ok) and torch.equal(v_host[:, :, t0:t0 + STEPS], ov)
            w = Workload(f"c5_layer{layer}", 12, 2, 128, torch.bfloat16, hot=kcfg.hot_budget,
                         cold=store.cold_length, top_pages=kcfg.top_pages, top_p=kcfg.top_p, segment=1)
            assert abs(scaling - w.scaling) < 1e-7
            check_summaries_in_pieces(store, k_host, w)
            s_new, s32_new = store.read_summaries(pages0, 1)
            m64 = k_host[:, :, t0:t0 + 128].double().mean(dim=2)       # [B, Hkv, D]
            rel = ((s32_new[0].cpu().double() - m64[0]).abs() / m64[0].abs().clamp_min(1e-30)).max()
            assert rel <= 1e-5 and torch.equal(s_new.cpu(), s32_new.cpu().to(s_new.dtype))
            oracle = OracleColdStore(w.page_size, w.groups)
            oracle.evict(k_host, v_host)
            info = {}
            _, _, sel = check_retrieval(store, oracle, kcfg, w, {"cold_k": k_host, "cold_v": v_host}, q.cpu(),
                                        min_det_c=0.0, info=info)
            print(f"c5 layer {layer}, step {STEPS}: union {len(info['union'])} pages, determined coarse "
                  f"{info['det_c']:.2f} fine {info['det_f'][0]:.2f}; oracle union {len(info['oracle_pages'])}; "
                  f"new page {pages0}: rel err of its mean {float(rel):.1e}, "
                  f"{'in' if pages0 in info['union'] else 'not in'} the union", flush=True)
            print("  " + separation_line(info["separation"]), flush=True)
            # The decode step selected the same pages and tokens.
            assert info["union"] == step_coarse["pages_selected"]
            assert sel.reshape(-1).tolist() == step_fine["selected_token_indices"]
            assert np.all(np.diff(info["union"]) > 0)
            del k_host, v_host, oracle
    finally:
        mw.uninstall()
        del model
        gc.collect()
        torch.cuda.empty_cache()
