"""Pins oracle/gaps.py, the distance of a selection difference from the boundary.

* boundary_gaps equals a brute-force search for the smallest change of one
  score that moves its index across the top-k boundary (distinct scores),
  is 0 on exact ties at the boundary and infinite when k >= n;
* the dtype-emulated scores equal torch's matmul-then-scale in the dtype on
  inputs whose dot products are exact, and the float64 ones the closed form;
* planted mistakes: a swap of a well-separated selected index, or a union
  page that no row put near its boundary, is reported; swaps of tied or
  near-boundary indices are not;
* the oracle's top-P conditioned on a union equals its unconditioned
  retrieval when given its own union.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from kiv_amd.synthetic import Workload, generate
from oracle import exact, gaps
from oracle.torch_ref import OracleColdStore


def _topk(s: np.ndarray, k: int) -> set:
    return set(np.argsort(-s, kind="stable")[:k].tolist())


def _brute_gap(s: np.ndarray, k: int, i: int) -> float:
    """Smallest |d| over moves of s_i just past another score that change
    whether i is in the top k (scores distinct)."""
    inside = i in _topk(s, k)
    best = np.inf
    for j in range(s.size):
        if j == i:
            continue
        for eps in (-1e-9, 1e-9):
            t = s.copy()
            t[i] = s[j] + eps
            if (i in _topk(t, k)) != inside:
                best = min(best, abs(s[j] - s[i]))
    return best


@pytest.mark.parametrize("n,k", [(12, 3), (20, 1), (9, 8), (30, 15)])
def test_boundary_gaps_brute_force(n, k):
    rng = np.random.default_rng(n * 100 + k)
    for _ in range(5):
        s = rng.normal(size=n)
        g = gaps.boundary_gaps(s[None, :], k)[0]
        want = np.array([_brute_gap(s, k, i) for i in range(n)])
        np.testing.assert_allclose(g, want, rtol=0, atol=1e-8)


def test_boundary_gaps_ties_and_everything_selected():
    s = np.array([[5.0, 3.0, 3.0, 3.0, 1.0]])
    g = gaps.boundary_gaps(s, 2)[0]
    assert g[0] == 2.0                 # above the tied (k+1)-th by 2
    assert np.all(g[1:4] == 0.0)       # tied at the boundary: any of them may be picked
    assert g[4] == 2.0                 # below the k-th by 2
    assert np.all(np.isinf(gaps.boundary_gaps(s, 5)))
    assert np.all(np.isinf(gaps.boundary_gaps(s, 9)))


@pytest.mark.parametrize("dtype,name", [(torch.bfloat16, "bfloat16"), (torch.float16, "float16")])
def test_scores_both_match_torch_and_closed_form(dtype, name):
    g = torch.Generator().manual_seed(3)
    q = torch.randint(-8, 9, (1, 4, 1, 16), generator=g).to(dtype)
    k = torch.randint(-8, 9, (1, 2, 50, 16), generator=g).to(dtype)
    scaling = 16 ** -0.5
    s64, semu = gaps.scores_both(q.double().numpy(), k.double().numpy(), scaling, name)
    kx = k.repeat_interleave(2, dim=1)
    want = (torch.matmul(q, kx.transpose(-2, -1)) * scaling).double().numpy()
    assert np.array_equal(semu, want)
    closed = np.einsum("bhqd,bhtd->bhqt", q.double().numpy(), kx.double().numpy()) * scaling
    assert np.allclose(s64, closed, rtol=0, atol=1e-12)


def test_topk_differences_planted():
    rng = np.random.default_rng(7)
    s = np.sort(rng.normal(size=40))[::-1].copy()  # distinct, descending
    s[9] = s[10] = s[9]                            # a tie across the boundary of k = 10
    semu = s.copy()
    ref = set(range(10))
    # Swapping the tied boundary pair is within the rule.
    r = gaps.topk_differences(ref - {9} | {10}, ref, s, semu, 10)
    assert r["differ"] == 2 and r["violations"] == []
    # Swapping a well-separated index (the best) for the worst is not.
    r = gaps.topk_differences(ref - {0} | {39}, ref, s, semu, 10)
    assert sorted(r["violations"]) == [0, 39]
    # A gap small in one arithmetic only is excused: emulated tie, float64 apart.
    s2 = s.copy()
    s2[10] = s2[9] - 0.01
    r = gaps.topk_differences(ref - {9} | {10}, ref, s2, semu, 10)
    assert r["violations"] == [] and r["max_gap64"] > 0.009
    r = gaps.topk_differences(ref - {9} | {10}, ref, s2, s2, 10)
    assert sorted(r["violations"]) == [9, 10]


def test_union_differences_planted():
    rng = np.random.default_rng(11)
    rows = rng.normal(size=(3, 30))
    k = 4
    ref_rows = [_topk(r, k) for r in rows]
    ref = set().union(*ref_rows)
    # A page at some row's boundary (the (k+1)-th of row 1, not selected anywhere) is excused
    # when it is made to tie that row's k-th.
    p = int(np.argsort(-rows[1])[k])
    assert p not in ref
    tied = rows.copy()
    tied[1, p] = np.sort(tied[1])[::-1][k - 1]
    r = gaps.union_differences(ref | {p}, ref, tied, tied, k, ref_rows)
    assert r["differ"] == 1 and r["violations"] == []
    # A page far below every row's boundary is a violation.
    far = rows.copy()
    q = int(np.argmin(rows.sum(axis=0)))
    far[:, q] = -100.0
    assert q not in ref
    r = gaps.union_differences(ref | {q}, ref, far, far, k, ref_rows)
    assert r["violations"] == [q]
    # A page the reference selected far above the boundary, missing from the union, is a violation.
    top = int(np.argmax(rows[0]))
    hi = rows.copy()
    hi[0, top] = 100.0
    ref_rows_hi = [_topk(r, k) for r in hi]
    ref_hi = set().union(*ref_rows_hi)
    r = gaps.union_differences(ref_hi - {top}, ref_hi, hi, hi, k, ref_rows_hi)
    assert top in r["violations"]


def test_retrieve_given_its_own_union_is_the_retrieval():
    w = Workload("gu", 8, 2, 32, torch.bfloat16, hot=8, cold=3000 + 17, top_pages=3, top_p=100, segment=256)
    data = generate(w, seed=4)
    store = OracleColdStore(w.page_size, w.groups)
    store.evict(data["cold_k"], data["cold_v"])
    _, _, trace = store.retrieve(data["q"], w.scaling, w.top_p, w.top_pages)
    cond = store.retrieve_given_union(data["q"], w.scaling, w.top_p, trace.pages)
    assert torch.equal(cond.selected_ids, trace.selected_ids)
    assert torch.equal(cond.candidate_ids, trace.candidate_ids)
    # Another union changes the candidates accordingly (first page dropped).
    cond2 = store.retrieve_given_union(data["q"], w.scaling, w.top_p, trace.pages[1:])
    first = int(trace.pages[0])
    assert not np.isin(cond2.selected_ids.numpy() // w.page_size, [first]).any()
    assert "top_idx" in trace.extra and trace.extra["top_idx"].shape[-1] == w.top_pages
    # Per-row selections, re-derived from the reference's scores, form the union.
    rows = trace.extra["top_idx"].reshape(-1, w.top_pages)
    assert sorted(set(rows.reshape(-1).tolist())) == trace.pages.tolist()
    # The gap module sees no disagreement between the oracle and itself.
    s64, semu = gaps.scores_both(data["q"].double().numpy(), torch.cat(store.summaries, 2).double().numpy(),
                                 w.scaling, "bfloat16")
    N = store.num_pages
    ref_rows = [set(r.tolist()) for r in rows]
    r = gaps.union_differences(set(trace.pages.tolist()), set(trace.pages.tolist()), s64.reshape(-1, N),
                               semu.reshape(-1, N), w.top_pages, ref_rows)
    assert r["differ"] == 0
    assert exact.round_to_dtype(np.array([1.0]), "bfloat16")[0] == 1.0
