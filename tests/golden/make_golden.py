"""Writes golden vectors with the reference implementation itself.

    python tests/golden/make_golden.py          (build container only)
    python tests/golden/make_golden.py shared   (adds the shared-layer fixtures only)

The reference (Babyhamsta/KIV, Python) is imported from /root/reference in
this container and never travels: only the vectors below are committed.
They pin what the repository's closed forms and rounding bands leave open:

* retrieval.npz  -- ColdKVStore (kiv/cold_store.py:35-414) on CPU for small
  seeded cases, including exact score ties: union pages, selected token ids
  in the order returned, the returned K/V and the telemetry scores.  Inputs
  are stored as raw 16-bit patterns (bf16 / fp16) so they are bit-exact.
* tiny_qwen2.safetensors + tiny_qwen2.npz -- a random-init 2-layer Qwen2
  driven through KIVMiddleware (kiv/middleware.py:43-356) and TieredKVCache
  (kiv/tiered_cache.py:17-286): chunked_prefill of 96 tokens, then greedy
  decode steps with live retrieval; the weights, input ids, every step's
  logits and the tokens chosen.
* tiny_gemma4_shared.safetensors + .npz -- the same for a random-init 4-layer
  Gemma4 text model whose second full-attention layer shares the first's KV
  (ModelTopology kv_sharing_map), plus the shared store's telemetry.
"""

from __future__ import annotations

import json
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
REFERENCE = "/root/reference"


def bits16(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().copy()


def retrieval_cases():
    from kiv.cold_store import ColdKVStore
    from kiv.config import KIVConfig
    from kiv.model_topology import ModelTopology

    cases = [
        # name, dtype, B, Hq, Hkv, D, Q, page, cold, chunks, top_pages, top_p, kind
        ("gqa_bf16", torch.bfloat16, 1, 8, 2, 64, 1, 16, 600, (100, 7, 493), 4, 40, "clustered"),
        ("mha_f16", torch.float16, 1, 4, 4, 32, 1, 8, 300, (300,), 3, 30, "clustered"),
        ("batch_multiq_bf16", torch.bfloat16, 2, 4, 2, 32, 3, 8, 250, (64, 186), 3, 24, "clustered"),
        ("few_pages_bf16", torch.bfloat16, 1, 4, 1, 32, 1, 16, 40, (40,), 8, 64, "clustered"),
        ("ties_equal_rows_bf16", torch.bfloat16, 1, 2, 1, 16, 1, 8, 64, (64,), 2, 5, "equal"),
        ("ties_repeated_pages_bf16", torch.bfloat16, 1, 4, 1, 16, 1, 8, 96, (50, 46), 3, 12, "repeat"),
    ]
    out, manifest = {}, []
    for i, (name, dtype, B, hq, hkv, D, Q, ps, cold, chunks, tp, P, kind) in enumerate(cases):
        g = torch.Generator().manual_seed(1000 + i)
        seg = 4 * ps
        cent = torch.randn(B, hkv, (cold + seg - 1) // seg, D, generator=g)
        if kind == "equal":
            k = torch.ones(B, hkv, cold, D)
        elif kind == "repeat":
            # every page repeats the first page's rows: page scores and token
            # scores tie across pages
            base = torch.randn(B, hkv, ps, D, generator=g)
            k = base.repeat(1, 1, (cold + ps - 1) // ps, 1)[:, :, :cold]
        else:
            k = cent[:, :, torch.arange(cold) // seg] + 0.3 * torch.randn(B, hkv, cold, D, generator=g)
        v = torch.randn(B, hkv, cold, D, generator=g)
        heads = torch.arange(hq) // (hq // hkv)
        q = cent[:, heads, :1].repeat(1, 1, Q, 1) + 0.1 * torch.randn(B, hq, Q, D, generator=g)
        if kind == "equal":
            q = torch.ones(B, hq, Q, D)
        k, v, q = k.to(dtype), v.to(dtype), q.to(dtype)
        scaling = D ** -0.5
        cfg = KIVConfig(top_p=P, top_pages=tp, page_size=ps, prefetch_stream=False)
        topo = ModelTopology.manual(global_layer_indices=(0,), num_query_heads=hq, num_kv_heads=hkv, head_dim=D,
                                    num_hidden_layers=1)
        store = ColdKVStore(cfg, topo, torch.device("cpu"))
        t = 0
        for c in chunks:
            store.evict_from_hot(k[:, :, t:t + c], v[:, :, t:t + c])
            t += c
        assert t == cold
        k_out, v_out = store.retrieve_top_kv(q, scaling, cfg)
        recent = store.telemetry_snapshot()["recent"]
        coarse, fine = recent[-2], recent[-1]
        pre = f"c{i}_"
        out[pre + "k"], out[pre + "v"], out[pre + "q"] = bits16(k), bits16(v), bits16(q)
        out[pre + "k_out"], out[pre + "v_out"] = bits16(k_out), bits16(v_out)
        out[pre + "pages"] = np.array(coarse.get("pages_selected", []), dtype=np.int64)
        out[pre + "selected"] = np.array(fine["selected_token_indices"], dtype=np.int64)
        manifest.append({
            "index": i, "name": name, "dtype": str(dtype).replace("torch.", ""), "batch": B, "num_q_heads": hq,
            "num_kv_heads": hkv, "head_dim": D, "q_len": Q, "page_size": ps, "cold": cold, "chunks": list(chunks),
            "top_pages": tp, "top_p": P, "scaling": scaling, "kind": kind,
            "coarse_skipped": bool(coarse.get("skipped", False)),
            "coarse_top_score": coarse["top_score"], "coarse_mean_score": coarse["mean_score"],
            "fine_top_score": fine["top_score"], "fine_mean_score": fine["mean_score"],
            "actual_P": fine["actual_P"],
        })
    np.savez_compressed(os.path.join(HERE, "retrieval.npz"), **out)
    return manifest


def tiny_model():
    from safetensors.torch import save_file
    from transformers import Qwen2Config, Qwen2ForCausalLM

    from kiv.config import KIVConfig
    from kiv.middleware import KIVMiddleware

    cfg = Qwen2Config(vocab_size=128, hidden_size=64, intermediate_size=128, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=2, head_dim=16, max_position_embeddings=512,
                      rope_theta=10000.0, tie_word_embeddings=False)
    cfg._attn_implementation = "eager"
    torch.manual_seed(7)
    model = Qwen2ForCausalLM(cfg).eval()
    save_file({k: v.contiguous() for k, v in model.state_dict().items()},
              os.path.join(HERE, "tiny_qwen2.safetensors"))
    kcfg = KIVConfig(hot_budget=24, top_p=12, page_size=8, top_pages=2, prefetch_stream=False)
    mw = KIVMiddleware(model, kcfg)
    mw.install()
    cache = mw.create_cache(torch.device("cpu"))
    ids = torch.randint(0, 128, (1, 96), generator=torch.Generator().manual_seed(8))
    with torch.no_grad():
        logits = mw.chunked_prefill(ids, cache, chunk_size=32)
        steps, toks = [logits[0].float().numpy().copy()], []
        tok = logits.argmax(-1)
        for _ in range(6):
            toks.append(int(tok.item()))
            out = model(input_ids=tok.view(1, 1), past_key_values=cache, use_cache=True)
            lg = out.logits[:, -1]
            steps.append(lg[0].float().numpy().copy())
            tok = lg.argmax(-1)
    np.savez_compressed(os.path.join(HERE, "tiny_qwen2.npz"), input_ids=ids.numpy(), logits=np.stack(steps),
                        tokens=np.array(toks, dtype=np.int64))
    return {"config": cfg.to_dict(), "kiv": {"hot_budget": 24, "top_p": 12, "page_size": 8, "top_pages": 2},
            "prefill": {"tokens": 96, "chunk_size": 32}, "decode_steps": 6, "attn_implementation": "eager",
            "weights_seed": 7, "ids_seed": 8}


GEMMA4_CONFIG = dict(vocab_size=128, hidden_size=64, intermediate_size=128, num_hidden_layers=4,
                     num_attention_heads=4, num_key_value_heads=2, head_dim=16, global_head_dim=32,
                     max_position_embeddings=512, sliding_window=16,
                     layer_types=["sliding_attention", "full_attention", "sliding_attention", "full_attention"],
                     num_kv_shared_layers=2, vocab_size_per_layer_input=128, hidden_size_per_layer_input=8,
                     final_logit_softcapping=None, tie_word_embeddings=False)
GEMMA4_TOPOLOGY = dict(global_layer_indices=(1, 3), independent_kv_layers=(1,), kv_sharing_map={3: 1},
                       num_query_heads=4, num_kv_heads=2, head_dim=32, num_hidden_layers=4)


def tiny_gemma4_shared():
    """A random-init 4-layer Gemma4 text model whose last full-attention layer
    shares the KV of the first (num_kv_shared_layers=2): both global layers
    retrieve from one cold store, the shared layer through the candidate set
    the source layer selected in the same decode step
    (kiv/cold_store.py:303-329, kiv/tiered_cache.py:117-123).  Weights,
    input ids, every step's logits, the tokens chosen and the store's
    telemetry (every coarse and fine record) are written."""
    from safetensors.torch import save_file
    from transformers import Gemma4TextConfig
    from transformers.models.gemma4.modeling_gemma4 import Gemma4ForCausalLM

    from kiv.config import KIVConfig
    from kiv.middleware import KIVMiddleware
    from kiv.model_topology import ModelTopology

    cfg = Gemma4TextConfig(**GEMMA4_CONFIG)
    cfg._attn_implementation = "eager"
    torch.manual_seed(11)
    model = Gemma4ForCausalLM(cfg).eval()
    save_file({k: v.contiguous() for k, v in model.state_dict().items()},
              os.path.join(HERE, "tiny_gemma4_shared.safetensors"))
    kiv = {"hot_budget": 24, "top_p": 12, "page_size": 8, "top_pages": 2}
    kcfg = KIVConfig(prefetch_stream=False, **kiv)
    topo = ModelTopology.manual(**GEMMA4_TOPOLOGY)
    mw = KIVMiddleware(model, kcfg, topology=topo)
    mw.install()
    cache = mw.create_cache(torch.device("cpu"))
    ids = torch.randint(0, 128, (1, 96), generator=torch.Generator().manual_seed(12))
    with torch.no_grad():
        logits = mw.chunked_prefill(ids, cache, chunk_size=32)
        steps, toks = [logits[0].float().numpy().copy()], []
        tok = logits.argmax(-1)
        for _ in range(6):
            toks.append(int(tok.item()))
            out = model(input_ids=tok.view(1, 1), past_key_values=cache, use_cache=True)
            lg = out.logits[:, -1]
            steps.append(lg[0].float().numpy().copy())
            tok = lg.argmax(-1)
    mw.uninstall()
    snap = cache.get_cold_store(1).telemetry_snapshot()
    np.savez_compressed(os.path.join(HERE, "tiny_gemma4_shared.npz"), input_ids=ids.numpy(),
                        logits=np.stack(steps), tokens=np.array(toks, dtype=np.int64))
    return {"config": GEMMA4_CONFIG, "topology": {k: (list(v) if isinstance(v, tuple) else v)
                                                  for k, v in GEMMA4_TOPOLOGY.items()},
            "kiv": kiv, "prefill": {"tokens": 96, "chunk_size": 32}, "decode_steps": 6,
            "attn_implementation": "eager", "weights_seed": 11, "ids_seed": 12,
            "telemetry": snap}


def main():
    sys.path.insert(0, REFERENCE)
    torch.set_num_threads(1)
    path = os.path.join(HERE, "manifest.json")
    if sys.argv[1:] == ["shared"]:
        # Adds the shared-layer fixtures; the others are left as they are.
        with open(path) as f:
            manifest = json.load(f)
        manifest["tiny_gemma4_shared"] = tiny_gemma4_shared()
    else:
        manifest = {"reference": "Babyhamsta/KIV (read-only copy in the build container)",
                    "torch": torch.__version__, "retrieval": retrieval_cases(), "tiny_qwen2": tiny_model(),
                    "tiny_gemma4_shared": tiny_gemma4_shared()}
    with open(path, "w") as f:
        json.dump(manifest, f, indent=1, default=str)
    print("wrote", sorted(os.listdir(HERE)))


if __name__ == "__main__":
    main()
