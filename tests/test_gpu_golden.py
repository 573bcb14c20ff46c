"""The HIP path against vectors the reference itself wrote (tests/golden).

Retrieval: the HIP store on the same inputs must make a selection the
rounding bands allow, equal the reference's wherever the bands determine
it, and return exactly the rows it selected.  Exact ties are left open by
the bands: the reference breaks them through torch.topk, the kernels by the
lowest index, and both are valid.

End to end: the reference ran a random-init 2-layer Qwen2 (weights in
tiny_qwen2.safetensors) through KIVMiddleware.chunked_prefill and greedy
decode steps with live retrieval on CPU in fp32.  The same model through
this package's middleware on the GPU, fed the same tokens, must give the
same logits within 1e-3 and pick the same next token at every step.
"""

from __future__ import annotations

import json
import os

import numpy as np
import pytest
import torch

from kiv_amd import ColdKVStore, KIVConfig, KIVMiddleware, ModelTopology
from oracle import exact
from oracle.bands import check_topk, score_interval
from tests.test_golden import CASES, HERE, tensors

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def data():
    return np.load(os.path.join(HERE, "retrieval.npz"))


@pytest.mark.parametrize("case", CASES, ids=[c["name"] for c in CASES])
def test_hip_retrieval_matches_reference(cuda, case, data):
    t = tensors(case, data)
    cfg = KIVConfig(top_p=case["top_p"], top_pages=case["top_pages"], page_size=case["page_size"])
    topo = ModelTopology.manual(global_layer_indices=(0,), num_query_heads=case["num_q_heads"],
                                num_kv_heads=case["num_kv_heads"], head_dim=case["head_dim"], num_hidden_layers=1)
    store = ColdKVStore(cfg, topo, cuda)
    pos = 0
    for c in case["chunks"]:
        store.evict_from_hot(t["k"][:, :, pos:pos + c].to(cuda), t["v"][:, :, pos:pos + c].to(cuda))
        pos += c
    k_out, v_out = store.retrieve_top_kv(t["q"].to(cuda), case["scaling"], cfg)
    snap = store.telemetry_snapshot()["recent"]
    union = snap[-2]["pages_selected"]
    B, width = case["batch"], k_out.shape[2]
    sel = np.array(snap[-1]["selected_token_indices"], dtype=np.int64).reshape(B, width)
    N, ps = store.num_pages, case["page_size"]
    q = t["q"].float().numpy()
    summ = store.read_summaries()[0].cpu().permute(1, 2, 0, 3).float().numpy()
    lo, hi = score_interval(q, summ, case["scaling"], case["dtype"], "activation")
    det_c = check_topk(set(union), lo.reshape(-1, N), hi.reshape(-1, N), min(case["top_pages"], N))
    if det_c == 1.0:
        assert union == t["pages"].tolist()
    p = store.cold_length - N * ps
    cand = exact.candidate_ids(np.array(union, dtype=np.int64), ps, N * ps, p)
    k_all = t["k"]
    lo, hi = score_interval(q, k_all[:, :, torch.from_numpy(cand)].float().numpy(), case["scaling"], case["dtype"],
                            "activation")
    where = {int(g): i for i, g in enumerate(cand)}
    assert width == min(case["top_p"], store.cold_length, cand.size) == case["actual_P"]
    for b in range(B):
        det_f = check_topk({where[int(g)] for g in sel[b]}, lo.max(axis=(1, 2))[b:b + 1],
                           hi.max(axis=(1, 2))[b:b + 1], width)
        if det_c == 1.0 and det_f == 1.0:
            assert set(sel[b].tolist()) == set(t["selected"][b].tolist())
        idx = torch.from_numpy(sel[b])
        assert torch.equal(k_out[b].cpu(), t["k"][b][:, idx]) and torch.equal(v_out[b].cpu(), t["v"][b][:, idx])


def tiny_qwen2(cuda):
    from safetensors.torch import load_file
    from transformers import Qwen2Config, Qwen2ForCausalLM

    with open(os.path.join(HERE, "manifest.json")) as f:
        meta = json.load(f)["tiny_qwen2"]
    gold = np.load(os.path.join(HERE, "tiny_qwen2.npz"))
    conf = {k: v for k, v in meta["config"].items() if k not in ("architectures", "transformers_version")}
    cfg = Qwen2Config(**conf)
    cfg._attn_implementation = meta["attn_implementation"]
    model = Qwen2ForCausalLM(cfg).eval()
    model.load_state_dict(load_file(os.path.join(HERE, "tiny_qwen2.safetensors")))
    model.to(cuda)
    return model, meta, gold


def test_tiny_qwen2_end_to_end_matches_reference(cuda):
    model, meta, gold = tiny_qwen2(cuda)
    mw = KIVMiddleware(model, KIVConfig(**meta["kiv"]))
    mw.install()
    try:
        cache = mw.create_cache(cuda)
        ids = torch.from_numpy(gold["input_ids"]).to(cuda)
        with torch.no_grad():
            logits = mw.chunked_prefill(ids, cache, chunk_size=meta["prefill"]["chunk_size"])
            steps = [logits[0].float().cpu().numpy()]
            for tok in gold["tokens"].tolist():
                out = model(input_ids=torch.tensor([[tok]], device=cuda), past_key_values=cache, use_cache=True)
                steps.append(out.logits[0, -1].float().cpu().numpy())
        assert cache.get_cold_store(0).cold_length > 0  # the decode steps retrieved from the cold tier
    finally:
        mw.uninstall()
    got = np.stack(steps)
    ref = gold["logits"]
    assert got.shape == ref.shape
    err = np.abs(got - ref).max()
    assert err <= 1e-3, f"max abs logit difference {err}"
    assert np.array_equal(got.argmax(-1)[:-1], gold["tokens"])


def test_tiny_qwen2_multi_token_forward_with_cold_tier(cuda):
    """After prefill and decode, a 400-token forward on the same cache (a
    follow-up prompt, as the reference's reuse-path prefill runs it) takes
    the retrieval with 400 query positions (more than one pass of the scans)
    and the model's own attention over [retrieved ; hot], and must give
    finite logits for every position."""
    model, meta, gold = tiny_qwen2(cuda)
    mw = KIVMiddleware(model, KIVConfig(**meta["kiv"]))
    mw.install()
    try:
        cache = mw.create_cache(cuda)
        ids = torch.from_numpy(gold["input_ids"]).to(cuda)
        with torch.no_grad():
            mw.chunked_prefill(ids, cache, chunk_size=meta["prefill"]["chunk_size"])
            for tok in gold["tokens"].tolist()[:3]:
                model(input_ids=torch.tensor([[tok]], device=cuda), past_key_values=cache, use_cache=True)
            store = cache.get_cold_store(0)
            assert store.cold_length > 0
            before = len(store.telemetry_snapshot()["recent"])
            follow = torch.randint(0, model.config.vocab_size, (1, 400), generator=torch.Generator().manual_seed(3))
            out = model(input_ids=follow.to(cuda), past_key_values=cache, use_cache=True)
        assert out.logits.shape[:2] == (1, 400)
        assert torch.isfinite(out.logits).all()
        assert len(store.telemetry_snapshot()["recent"]) > before  # the forward retrieved from the cold tier
    finally:
        mw.uninstall()
