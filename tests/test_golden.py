"""The CPU oracle against vectors the reference itself wrote (tests/golden).

tests/golden/make_golden.py ran the reference's ColdKVStore on CPU for small
seeded cases (kiv/cold_store.py:142-371), including exact score ties.  The
oracle restates the same torch op sequence, so it must reproduce every
output bit for bit: the union of top pages, the selected token ids in the
returned order (ties included: torch.topk on CPU decides them in both), the
returned K/V rows and the telemetry scores.  The selections must also lie
inside the rounding bands of oracle.bands, which is what the HIP path is
held to where scores tie.
"""

from __future__ import annotations

import json
import os

import numpy as np
import pytest
import torch

from oracle import exact
from oracle.bands import check_topk, max_band, mean_band, score_interval
from oracle.torch_ref import OracleColdStore

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
DT = {"bfloat16": torch.bfloat16, "float16": torch.float16}


def load_cases():
    with open(os.path.join(HERE, "manifest.json")) as f:
        return json.load(f)["retrieval"]


CASES = load_cases()


def tensors(case, data):
    """The case's K, V, Q (bit patterns back to the dtype) and its golden outputs."""
    i, dt = case["index"], DT[case["dtype"]]
    t = {name: torch.from_numpy(data[f"c{i}_{name}"]).view(dt) for name in ("k", "v", "q", "k_out", "v_out")}
    t["pages"] = data[f"c{i}_pages"]
    t["selected"] = data[f"c{i}_selected"].reshape(case["batch"], -1)
    return t


def build_oracle(case, t):
    store = OracleColdStore(case["page_size"], case["num_q_heads"] // case["num_kv_heads"])
    pos = 0
    for c in case["chunks"]:
        store.evict(t["k"][:, :, pos:pos + c], t["v"][:, :, pos:pos + c])
        pos += c
    return store


@pytest.fixture(scope="module")
def data():
    return np.load(os.path.join(HERE, "retrieval.npz"))


@pytest.mark.parametrize("case", CASES, ids=[c["name"] for c in CASES])
def test_oracle_reproduces_reference(case, data):
    t = tensors(case, data)
    store = build_oracle(case, t)
    k_out, v_out, trace = store.retrieve(t["q"], case["scaling"], case["top_p"], case["top_pages"])
    assert trace.pages.tolist() == t["pages"].tolist()
    assert np.array_equal(trace.selected_ids.numpy(), t["selected"])
    assert torch.equal(k_out, t["k_out"]) and torch.equal(v_out, t["v_out"])
    # Telemetry records (kiv/cold_store.py:456-547), bit for bit.
    coarse, fine = store.telemetry.ring[-2], store.telemetry.ring[-1]
    assert coarse["top_score"] == case["coarse_top_score"] and coarse["mean_score"] == case["coarse_mean_score"]
    assert fine["top_score"] == case["fine_top_score"] and fine["mean_score"] == case["fine_mean_score"]
    assert coarse["skipped"] == case["coarse_skipped"] and fine["actual_P"] == case["actual_P"]
    assert coarse["pages_selected"] == t["pages"].tolist()
    assert fine["selected_token_indices"] == t["selected"].reshape(-1).tolist()


def telemetry_bands(case, t, store, pages=None):
    """Intervals of the four telemetry scores from the case's inputs:
    {name: (lo, hi)} for coarse/fine top and mean; the fine ones over the
    candidates of ``pages`` (default: the reference's union)."""
    pages = t["pages"] if pages is None else np.asarray(pages, dtype=np.int64)
    q = t["q"].float().numpy()
    N, ps = store.num_pages, case["page_size"]
    lo, hi = score_interval(q, store.flat()[0].float().numpy(), case["scaling"], case["dtype"], "activation")
    out = {"coarse_top_score": max_band(lo, hi), "coarse_mean_score": mean_band(lo, hi, case["dtype"], "activation")}
    cand = exact.candidate_ids(pages, ps, N * ps, store.cold_length - N * ps)
    ck = store.all_k()[:, :, torch.from_numpy(cand)]
    lo, hi = score_interval(q, ck.float().numpy(), case["scaling"], case["dtype"], "activation")
    lo, hi = lo.max(axis=(1, 2)), hi.max(axis=(1, 2))
    out["fine_top_score"] = max_band(lo, hi)
    out["fine_mean_score"] = mean_band(lo, hi, case["dtype"], "activation")
    return out


@pytest.mark.parametrize("case", CASES, ids=[c["name"] for c in CASES])
def test_reference_telemetry_within_bands(case, data):
    """The reference's own telemetry scores lie in the intervals the HIP
    telemetry is held to; where an interval is a single dtype value, that
    value is the reference's."""
    t = tensors(case, data)
    store = build_oracle(case, t)
    for name, (lo, hi) in telemetry_bands(case, t, store).items():
        assert lo <= case[name] <= hi, (name, lo, case[name], hi)
        if "top" in name:
            assert hi - lo <= abs(case[name]) * 2 ** -6 + 1e-6, (name, lo, hi)  # a few dtype steps at most


@pytest.mark.parametrize("case", CASES, ids=[c["name"] for c in CASES])
def test_reference_selection_within_bands(case, data):
    """Every reference choice is one the rounding bands allow; tie cases are
    exactly the ones the bands leave open."""
    t = tensors(case, data)
    store = build_oracle(case, t)
    summ = store.flat()[0]  # [B, Hkv, N, D]
    q = t["q"].float().numpy()
    N = store.num_pages
    lo, hi = score_interval(q, summ.float().numpy(), case["scaling"], case["dtype"], "activation")
    det_c = check_topk(set(t["pages"].tolist()), lo.reshape(-1, N), hi.reshape(-1, N), min(case["top_pages"], N))
    p = store.cold_length - N * case["page_size"]
    cand = exact.candidate_ids(t["pages"], case["page_size"], N * case["page_size"], p)
    ck = store.all_k()[:, :, torch.from_numpy(cand)]
    lo, hi = score_interval(q, ck.float().numpy(), case["scaling"], case["dtype"], "activation")
    pos = {int(g): i for i, g in enumerate(cand)}
    P = min(case["top_p"], store.cold_length, cand.size)
    for b in range(case["batch"]):
        check_topk({pos[int(g)] for g in t["selected"][b]}, lo.max(axis=(1, 2))[b:b + 1],
                   hi.max(axis=(1, 2))[b:b + 1], P)
    if case["kind"] == "clustered":
        assert det_c > 0.5
    elif case["kind"] == "equal":
        assert det_c == 0.0  # every page ties: any choice is allowed
