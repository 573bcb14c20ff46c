"""Telemetry values and shared-layer candidate reuse of the HIP store.

* The reference's own telemetry (tests/golden/manifest.json, written by its
  ColdKVStore): each of the four scores of the HIP record must lie in the
  interval the rounding allows (oracle.bands.max_band / mean_band), and
  equal the reference's value wherever that interval is one dtype value
  (every top score of the golden cases).  With the pruned fine scan, the
  top score and the selection stay those of the full scan.
* A sequence of calls (fresh, shared-layer reuse with other queries and
  another query length, eviction, a new step) against the oracle's
  restatement of the telemetry ring: every record's kind, flags, lengths
  and widths equal, scores in their intervals, selections within the
  bands and equal to the oracle's where determined, and the aggregates.
* Reuse (kiv/cold_store.py:303-317): the second call of a decode step
  scores the first call's union with its own query.  In fp32 the bands
  determine everything, so the HIP selection must equal the oracle's
  exactly, and differ from what the query's own union would give.
* End to end: a random-init 4-layer Gemma4 text model whose last
  full-attention layer shares the first's KV, run by the reference through
  its middleware (tests/golden/make_golden.py): this package's middleware
  must give the same logits within 1e-3, the same greedy tokens, and the
  shared store's telemetry records (fresh and reused calls) of the
  reference.
"""

from __future__ import annotations

import json
import os
from dataclasses import replace

import numpy as np
import pytest
import torch

from kiv_amd import ColdKVStore, KIVConfig, KIVMiddleware, ModelTopology
from kiv_amd.synthetic import Workload, generate
from oracle import exact
from oracle.bands import check_topk, max_band, mean_band, score_interval
from oracle.torch_ref import OracleColdStore
from tests.test_golden import CASES, HERE, build_oracle, telemetry_bands, tensors
from tests.test_gpu_retrieval import DT, build

pytestmark = pytest.mark.gpu

SCORES = ("coarse_top_score", "coarse_mean_score", "fine_top_score", "fine_mean_score")


@pytest.fixture(scope="module")
def data():
    return np.load(os.path.join(HERE, "retrieval.npz"))


def in_band(value: float, band: tuple[float, float], what: str) -> None:
    lo, hi = band
    assert lo <= value <= hi, f"{what}: {value} outside [{lo}, {hi}]"


@pytest.mark.parametrize("case", CASES, ids=[c["name"] for c in CASES])
def test_golden_telemetry_matches_reference(cuda, case, data):
    t = tensors(case, data)
    cfg = KIVConfig(top_p=case["top_p"], top_pages=case["top_pages"], page_size=case["page_size"])
    topo = ModelTopology.manual(global_layer_indices=(0,), num_query_heads=case["num_q_heads"],
                                num_kv_heads=case["num_kv_heads"], head_dim=case["head_dim"], num_hidden_layers=1)
    store = ColdKVStore(cfg, topo, cuda)
    pos = 0
    for c in case["chunks"]:
        store.evict_from_hot(t["k"][:, :, pos:pos + c].to(cuda), t["v"][:, :, pos:pos + c].to(cuda))
        pos += c
    store.retrieve_top_kv(t["q"].to(cuda), case["scaling"], cfg)
    snap = store.telemetry_snapshot()
    coarse, fine = snap["recent"]
    union = coarse["pages_selected"]
    got = {"coarse_top_score": coarse["top_score"], "coarse_mean_score": coarse["mean_score"],
           "fine_top_score": fine["top_score"], "fine_mean_score": fine["mean_score"]}
    bands = telemetry_bands(case, t, build_oracle(case, t), pages=union)
    same_union = union == t["pages"].tolist()
    for name in SCORES:
        in_band(got[name], bands[name], name)
        lo, hi = bands[name]
        if lo == hi and (name.startswith("coarse") or same_union):
            assert got[name] == case[name], name
    assert coarse["skipped"] is False and coarse["num_pages_selected"] == len(union)
    assert fine["actual_P"] == case["actual_P"] and fine["requested_P"] == case["top_p"]
    assert coarse["cold_length"] == fine["cold_length"] == case["cold"]
    agg = snap["aggregates"]
    assert (agg["total_calls"], agg["coarse_calls"], agg["coarse_real_calls"], agg["coarse_skipped_calls"],
            agg["fine_calls"]) == (1, 1, 1, 0, 1)
    assert agg["avg_coarse_top_score"] == got["coarse_top_score"]
    assert agg["avg_coarse_mean_score"] == got["coarse_mean_score"]
    assert agg["avg_fine_top_score"] == got["fine_top_score"]
    assert agg["avg_fine_mean_score"] == got["fine_mean_score"]
    assert agg["avg_cold_length"] == case["cold"] and agg["avg_selected_P"] == case["actual_P"]
    # The pruned fine scan (opt-in) keeps the top score and the selection.
    store.retrieve_top_kv(t["q"].to(cuda), case["scaling"], replace(cfg, fine_pruning=True))
    pruned = store.telemetry_snapshot()["recent"][-1]
    assert pruned["top_score"] == fine["top_score"]
    assert pruned["selected_token_indices"] == fine["selected_token_indices"]


def _query_for_segment(data: dict, w: Workload, seg: int, g: torch.Generator, positions: int = 1) -> torch.Tensor:
    """Query rows near the mean K of a cold segment (so their top pages lie there)."""
    cold = data["cold_k"].float()
    c = cold[:, :, seg * w.segment:(seg + 1) * w.segment].mean(2).repeat_interleave(w.groups, 1)
    q = c[:, :, None].repeat(1, 1, positions, 1) + 0.1 * torch.randn(1, w.num_q_heads, positions, w.head_dim,
                                                                      generator=g)
    return q.to(w.dtype)


def test_telemetry_sequence_matches_oracle(cuda):
    w = Workload("telemetry_seq", 8, 2, 64, torch.bfloat16, hot=64, cold=6000 + 3, top_pages=6, top_p=100,
                 segment=256)
    data = generate(w, seed=51)
    store, oracle, cfg = build(w, data, cuda, chunks=(2000, 7))
    g = torch.Generator().manual_seed(52)
    nseg = w.cold // w.segment
    t0 = int(data["targets"][0, 0])
    q1 = data["q"]
    q2 = _query_for_segment(data, w, (t0 + 5) % nseg, g)
    q3 = _query_for_segment(data, w, (t0 + 11) % nseg, g)
    q4 = _query_for_segment(data, w, (t0 + 3) % nseg, g, positions=3)
    dtype = DT[w.dtype]
    cold_k = data["cold_k"]
    calls = []  # (query, union the fine pass scored, fresh?)
    last_union = None
    plan = [(q1, -1), (q2, 7), (q3, 7), (q4, 7), "evict", (q1, 7), (q3, 8)]
    for item in plan:
        if item == "evict":
            hk, hv = data["hot_k"][:, :, :5], data["hot_v"][:, :, :5]
            store.evict_from_hot(hk.to(cuda), hv.to(cuda))
            oracle.evict(hk, hv)
            cold_k = torch.cat([cold_k, hk], dim=2)
            continue
        q, step = item
        store.retrieve_top_kv(q.to(cuda), w.scaling, cfg, step=step)
        oracle.retrieve(q, w.scaling, cfg.top_p, cfg.top_pages, step=step)
        rec = store.telemetry_snapshot()["recent"][-2]
        fresh = not rec["skipped"]
        if fresh:
            last_union = rec["pages_selected"]
        # bands of this call: coarse over the current summaries, fine over the union scored
        summ = store.read_summaries()[0].cpu().permute(1, 2, 0, 3).float().numpy()
        N, ps = store.num_pages, w.page_size
        lo, hi = score_interval(q.float().numpy(), summ, w.scaling, dtype, "activation")
        cand = exact.candidate_ids(np.array(last_union, dtype=np.int64), ps, N * ps, store.cold_length - N * ps)
        flo, fhi = score_interval(q.float().numpy(), cold_k[:, :, torch.from_numpy(cand)].float().numpy(), w.scaling,
                                  dtype, "activation")
        calls.append(dict(fresh=fresh, rows=(lo.reshape(-1, N), hi.reshape(-1, N)), union=last_union, cand=cand,
                          agg=(flo.max(axis=(1, 2)), fhi.max(axis=(1, 2))),
                          coarse_bands=(max_band(lo, hi), mean_band(lo, hi, dtype, "activation")),
                          fine_bands=None))
        fl, fh = calls[-1]["agg"]
        calls[-1]["fine_bands"] = (max_band(fl, fh), mean_band(fl, fh, dtype, "activation"))
    assert [c["fresh"] for c in calls] == [True, True, False, False, True, True]

    hip, ref = store.telemetry_snapshot(), oracle.telemetry.snapshot()
    assert len(hip["recent"]) == len(ref["recent"]) == 2 * len(calls)
    for i, c in enumerate(calls):
        hc, hf = hip["recent"][2 * i], hip["recent"][2 * i + 1]
        rc, rf = ref["recent"][2 * i], ref["recent"][2 * i + 1]
        for key in ("kind", "cold_length", "num_pages", "skipped"):
            assert hc[key] == rc[key], (i, key)
        for key in ("kind", "cold_length", "actual_P", "requested_P"):
            assert hf[key] == rf[key], (i, key)
        if c["fresh"]:
            k = min(cfg.top_pages, hc["num_pages"])
            det_c = check_topk(set(hc["pages_selected"]), *c["rows"], k)
            check_topk(set(rc["pages_selected"]), *c["rows"], k)
            if det_c == 1.0:
                assert hc["pages_selected"] == rc["pages_selected"], i
            assert hc["num_pages_selected"] == len(hc["pages_selected"])
            for val, band, name in ((hc["top_score"], c["coarse_bands"][0], "coarse top"),
                                    (hc["mean_score"], c["coarse_bands"][1], "coarse mean")):
                in_band(val, band, f"call {i} {name}")
            in_band(rc["top_score"], c["coarse_bands"][0], f"call {i} oracle coarse top")
        else:
            assert hc["pages_selected"] == [] and hc["top_score"] == 0.0 and hc["score_ratio"] == 0.0
        pos = {int(gid): j for j, gid in enumerate(c["cand"])}
        sel = {pos[gid] for gid in hf["selected_token_indices"]}
        det_f = check_topk(sel, c["agg"][0], c["agg"][1], hf["actual_P"])
        if det_f == 1.0 and (not c["fresh"] or hc["pages_selected"] == rc["pages_selected"]):
            assert set(hf["selected_token_indices"]) == set(rf["selected_token_indices"]), i
        in_band(hf["top_score"], c["fine_bands"][0], f"call {i} fine top")
        in_band(hf["mean_score"], c["fine_bands"][1], f"call {i} fine mean")
    ha, ra = hip["aggregates"], ref["aggregates"]
    for key in ("total_calls", "coarse_calls", "coarse_real_calls", "coarse_skipped_calls", "fine_calls",
                "avg_cold_length", "avg_selected_P"):
        assert ha[key] == ra[key], key
    fresh = [c for c in calls if c["fresh"]]
    for key, group, which in (("avg_coarse_top_score", fresh, ("coarse_bands", 0)),
                              ("avg_coarse_mean_score", fresh, ("coarse_bands", 1)),
                              ("avg_fine_top_score", calls, ("fine_bands", 0)),
                              ("avg_fine_mean_score", calls, ("fine_bands", 1))):
        lo = sum(c[which[0]][which[1]][0] for c in group) / len(group)
        hi = sum(c[which[0]][which[1]][1] for c in group) / len(group)
        assert lo - 1e-9 <= ha[key] <= hi + 1e-9, (key, lo, ha[key], hi)
        assert lo - 1e-9 <= ra[key] <= hi + 1e-9, (key, lo, ra[key], hi)


@pytest.mark.parametrize("positions_b", [1, 4])
def test_reuse_scores_first_union_with_second_query(cuda, positions_b):
    """fp32 store: query A's call at step 3 picks the union; query B's call
    at step 3 (one position, or four) must select the oracle's top-P of B
    over A's candidates exactly, which differs from B over its own union."""
    w = Workload("reuse_f32", 8, 2, 64, torch.float32, hot=8, cold=8192 + 29, top_pages=4, top_p=96, segment=256)
    data = generate(w, seed=61)
    store, oracle, cfg = build(w, data, cuda, chunks=(3000, 1))
    g = torch.Generator().manual_seed(62)
    qa = data["q"]
    qb = _query_for_segment(data, w, (int(data["targets"][0, 0]) + 9) % (w.cold // w.segment), g, positions_b)
    ka, va = store.retrieve_top_kv(qa.to(cuda), w.scaling, cfg, step=3)
    kb, vb = store.retrieve_top_kv(qb.to(cuda), w.scaling, cfg, step=3)
    _, _, ta = oracle.retrieve(qa, w.scaling, cfg.top_p, cfg.top_pages, step=3)
    _, _, tb = oracle.retrieve(qb, w.scaling, cfg.top_p, cfg.top_pages, step=3)
    assert tb.extra["reused"]
    rec = store.telemetry_snapshot()["recent"]
    assert rec[-2]["skipped"] is True and rec[-4]["skipped"] is False
    union = rec[-4]["pages_selected"]
    assert union == ta.pages.tolist()
    cand = exact.candidate_ids(np.array(union, dtype=np.int64), w.page_size, store.num_pages * w.page_size,
                               store.cold_length - store.num_pages * w.page_size)
    lo, hi = score_interval(qb.numpy(), data["cold_k"][:, :, torch.from_numpy(cand)].numpy(), w.scaling, "float32",
                            "activation")
    pos = {int(gid): j for j, gid in enumerate(cand)}
    sel = rec[-1]["selected_token_indices"]
    assert check_topk({pos[gid] for gid in sel}, lo.max(axis=(1, 2)), hi.max(axis=(1, 2)), w.top_p) == 1.0
    assert set(sel) == set(tb.selected_ids[0].tolist())
    idx = torch.tensor(sel)
    assert torch.equal(kb[0].cpu(), data["cold_k"][0][:, idx]) and torch.equal(vb[0].cpu(), data["cold_v"][0][:, idx])
    # B over its own union (a fresh step) selects differently: the reuse mattered.
    store.retrieve_top_kv(qb.to(cuda), w.scaling, cfg, step=4)
    own = store.telemetry_snapshot()["recent"][-1]["selected_token_indices"]
    assert set(own) != set(sel)
    agg = store.telemetry_snapshot()["aggregates"]
    assert (agg["coarse_real_calls"], agg["coarse_skipped_calls"]) == (2, 1)


def tiny_gemma4_shared(cuda):
    from safetensors.torch import load_file
    from transformers import Gemma4TextConfig
    from transformers.models.gemma4.modeling_gemma4 import Gemma4ForCausalLM

    with open(os.path.join(HERE, "manifest.json")) as f:
        meta = json.load(f)["tiny_gemma4_shared"]
    gold = np.load(os.path.join(HERE, "tiny_gemma4_shared.npz"))
    cfg = Gemma4TextConfig(**meta["config"])
    cfg._attn_implementation = meta["attn_implementation"]
    model = Gemma4ForCausalLM(cfg).eval()
    model.load_state_dict(load_file(os.path.join(HERE, "tiny_gemma4_shared.safetensors")))
    model.to(cuda)
    top = meta["topology"]
    topo = ModelTopology.manual(global_layer_indices=tuple(top["global_layer_indices"]),
                                independent_kv_layers=tuple(top["independent_kv_layers"]),
                                kv_sharing_map={int(k): int(v) for k, v in top["kv_sharing_map"].items()},
                                num_query_heads=top["num_query_heads"], num_kv_heads=top["num_kv_heads"],
                                head_dim=top["head_dim"], num_hidden_layers=top["num_hidden_layers"])
    return model, topo, meta, gold


def test_gemma4_shared_kv_layer_end_to_end_matches_reference(cuda):
    model, topo, meta, gold = tiny_gemma4_shared(cuda)
    mw = KIVMiddleware(model, KIVConfig(**meta["kiv"]), topology=topo)
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
        snap = cache.get_cold_store(topo.independent_kv_layers[0]).telemetry_snapshot()
    finally:
        mw.uninstall()
    got = np.stack(steps)
    err = np.abs(got - gold["logits"]).max()
    print(f"gemma4 shared-KV model: max abs logit difference {err:.2e}", flush=True)
    assert err <= 1e-3
    assert np.array_equal(got.argmax(-1)[:-1], gold["tokens"])
    ref = meta["telemetry"]
    for key in ("total_calls", "coarse_calls", "coarse_real_calls", "coarse_skipped_calls", "fine_calls",
                "avg_cold_length", "avg_selected_P"):
        assert snap["aggregates"][key] == ref["aggregates"][key], key
    for key in ("avg_coarse_top_score", "avg_coarse_mean_score", "avg_fine_top_score", "avg_fine_mean_score"):
        assert snap["aggregates"][key] == pytest.approx(ref["aggregates"][key], rel=1e-4, abs=1e-5), key
    assert len(snap["recent"]) == len(ref["recent"])
    for mine, theirs in zip(snap["recent"], ref["recent"]):
        for key in ("kind", "cold_length", "skipped", "num_pages", "num_pages_selected", "pages_selected",
                    "actual_P", "requested_P"):
            assert mine.get(key) == theirs.get(key), (key, mine.get(key), theirs.get(key))
        if mine["kind"] == "fine":
            assert set(mine["selected_token_indices"]) == set(theirs["selected_token_indices"])
        for key in ("top_score", "mean_score"):
            assert mine[key] == pytest.approx(theirs[key], rel=1e-4, abs=1e-5), key
