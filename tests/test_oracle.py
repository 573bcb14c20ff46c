"""Pins the CPU oracle before it is trusted as the checker.

* dtype rounding: numpy emulation == torch's own conversions, bit for bit;
* score rounding (matmul, then * scaling, each rounded to the dtype):
  emulation == torch CPU matmul on inputs whose dot products are exact;
* page summaries: torch restatement vs the fp64 closed form;
* selection: brute force over all tokens when every page is selected,
  and separated top-k sets equal the fp64 ones;
* attention: P = all is lossless (equals full attention over cold + hot up
  to key order), cold = 0 is plain attention, key permutation invariance.
Planted mistakes (a sign error, an off-by-one-page id, rounding once instead of twice) must fail.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from kiv_amd.synthetic import Workload, generate
from oracle import exact
from oracle.torch_ref import OracleColdStore, decode_step, eager_attention, expand_kv, kiv_decode_attention


def f64(t):
    return t.detach().double().numpy()


@pytest.mark.parametrize("dtype,name", [(torch.bfloat16, "bfloat16"), (torch.float16, "float16")])
def test_round_to_dtype_matches_torch(dtype, name):
    g = torch.Generator().manual_seed(0)
    x = torch.cat([
        torch.randn(20000, generator=g) * 10,
        torch.randn(2000, generator=g) * 1e-6,
        torch.tensor([0.0, -0.0, 1.0, -1.0, 65504.0, 1e-8, 3.0e38]),
    ])
    # Halfway cases for bf16: low 16 bits exactly 0x8000.
    u = (torch.randint(0, 2 ** 15, (1000,), generator=g).int() << 16) | 0x8000
    x = torch.cat([x, u.view(torch.float32)])
    x = x[torch.isfinite(x)]
    got = exact.round_to_dtype(x.numpy(), name)
    want = x.to(dtype).double().numpy()
    finite = np.isfinite(want)
    assert np.array_equal(got[finite], want[finite])


@pytest.mark.parametrize("dtype,name", [(torch.bfloat16, "bfloat16"), (torch.float16, "float16")])
def test_emulated_scores_match_torch_matmul(dtype, name):
    """Small-integer inputs make the fp32 dot exact, so only the two
    roundings (after matmul, after * scaling) can differ."""
    g = torch.Generator().manual_seed(1)
    lim = 9 if dtype == torch.bfloat16 else 41  # dot products exceed the dtype's exact-integer range
    q = torch.randint(-lim + 1, lim, (3, 5, 1, 16), generator=g).to(dtype)
    k = torch.randint(-lim + 1, lim, (3, 5, 40, 16), generator=g).to(dtype)
    for scaling in (0.125, 16 ** -0.5, 0.3):
        want = (torch.matmul(q, k.transpose(-2, -1)) * scaling).double().numpy()
        dot = np.einsum("bhqd,bhtd->bhqt", f64(q), f64(k)).astype(np.float32)
        got = exact.emulate_scores(dot, scaling, name)
        assert np.array_equal(got, want), scaling
    # A planted mistake (rounding only once) is caught.
    once = exact.round_to_dtype(dot.astype(np.float64) * 0.3, name)
    assert not np.array_equal(once, (torch.matmul(q, k.transpose(-2, -1)) * 0.3).double().numpy())


def test_page_summaries_closed_form():
    g = torch.Generator().manual_seed(2)
    k = torch.randn(2, 3, 1000, 8, generator=g)
    store = OracleColdStore(page_size=64, num_kv_groups=1)
    for t in range(0, 1000, 37):
        store.evict(k[:, :, t:t + 37], k[:, :, t:t + 37])
    assert store.num_pages == 1000 // 64 and store.partial_len == 1000 % 64
    got = torch.cat(store.summaries, dim=2).double().numpy()
    want = exact.page_means(f64(k), 64)
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-6)
    # Closed form by brute force on page 3.
    assert np.allclose(want[:, :, 3], f64(k)[:, :, 192:256].mean(axis=2))


def _small(cold=1100, hot=40, groups=2, hkv=2, d=16, seed=0, dtype=torch.float32):
    w = Workload("o", hkv * groups, hkv, d, dtype, hot=hot, cold=cold, top_pages=4, top_p=64, segment=128,
                 page_size=32)
    data = generate(w, seed=seed)
    store = OracleColdStore(w.page_size, groups)
    store.evict(data["cold_k"], data["cold_v"])
    return w, data, store


def test_all_pages_selected_is_brute_force():
    w, data, store = _small()
    N = store.num_pages
    ck, cv, trace = store.retrieve(data["q"], w.scaling, top_p=10 ** 6, top_pages=10 ** 6)
    assert trace.pages.tolist() == list(range(N))
    assert sorted(trace.selected_ids[0].tolist()) == list(range(w.cold))
    # Selection order is by brute-force max-over-heads score.
    full = exact.scores64(f64(data["q"]), f64(data["cold_k"]), w.scaling, w.groups).max(axis=(1, 2))[0]
    sel = trace.selected_ids[0].numpy()
    assert np.all(np.diff(full[sel]) <= 1e-5)


def test_separated_top_p_matches_fp64():
    w, data, store = _small(seed=3)
    P = 50
    _, _, trace = store.retrieve(data["q"], w.scaling, top_p=P, top_pages=w.top_pages)
    cand = trace.candidate_ids.numpy()
    fine = exact.scores64(f64(data["q"]), f64(data["cold_k"])[:, :, cand], w.scaling, w.groups)
    agg = exact.fine_aggregate(fine)[0]
    sel, gap = exact.top_k_set(agg, P)
    assert gap > 1e-3
    assert set(cand[sel].tolist()) == set(trace.selected_ids[0].tolist())
    # Coarse union against the fp64 closed form.
    summ = torch.cat(store.summaries, dim=2)
    coarse = exact.scores64(f64(data["q"]), f64(summ), w.scaling, w.groups)
    pages, cgap = exact.coarse_union(coarse, w.top_pages)
    assert cgap > 1e-3 and pages.tolist() == trace.pages.tolist()
    # Planted mistakes: a sign error, and ids mapped one page off.
    wsel, _ = exact.top_k_set(exact.fine_aggregate(-fine)[0], P)
    assert set(cand[wsel].tolist()) != set(trace.selected_ids[0].tolist())
    assert set((cand[sel] + w.page_size).tolist()) != set(trace.selected_ids[0].tolist())


def test_p_all_is_lossless():
    """top_pages >= N and top_p >= cold: retrieval + attention == full attention."""
    w, data, store = _small(seed=4)
    out, _ = decode_step(store, data["q"], data["hot_k"], data["hot_v"], None, w.scaling, 10 ** 6, 10 ** 6)
    keys = torch.cat([data["cold_k"], data["hot_k"]], dim=2)
    vals = torch.cat([data["cold_v"], data["hot_v"]], dim=2)
    full = exact.attention64(f64(data["q"]), f64(keys), f64(vals), w.scaling)
    np.testing.assert_allclose(out.double().numpy(), full, atol=1e-5)


def test_cold_zero_is_plain_attention_and_permutation_invariant():
    w, data, _ = _small(seed=5)
    out = kiv_decode_attention(data["q"], data["hot_k"], data["hot_v"], None, None, None, w.scaling)
    want = exact.attention64(f64(data["q"]), f64(data["hot_k"]), f64(data["hot_v"]), w.scaling)
    np.testing.assert_allclose(out.double().numpy(), want, atol=1e-5)
    perm = torch.randperm(w.hot, generator=torch.Generator().manual_seed(0))
    out2 = eager_attention(data["q"], data["hot_k"][:, :, perm], data["hot_v"][:, :, perm], None, w.scaling)
    np.testing.assert_allclose(out2.double().numpy(), want, atol=1e-5)


def test_empty_store_returns_none():
    store = OracleColdStore(page_size=8, num_kv_groups=1)
    k, v, _ = store.retrieve(torch.zeros(1, 1, 1, 4), 1.0, 4, 2)
    assert k is None and v is None


def test_expand_kv_mapping():
    x = torch.arange(2 * 3 * 1 * 1).reshape(2, 3, 1, 1).float()
    y = expand_kv(x, 4)
    assert y.shape == (2, 12, 1, 1)
    assert torch.equal(y[:, :, 0, 0], x[:, :, 0, 0].repeat_interleave(4, dim=1))
    assert np.array_equal(exact.expand_kv(x.numpy(), 4), y.numpy())


def test_shared_layer_reuse_scores_the_cached_union():
    """kiv/cold_store.py:303-317: a second call in the same decode step
    (step >= 0, same batch) keeps the first call's candidates and scores
    them with its own query.  Query B targets another segment, so its own
    union differs from A's: the reused selection must be the fp64 top-P of
    B over A's candidates (separated scores), and a fresh step recomputes."""
    w = Workload("reuse", 8, 2, 64, torch.float32, hot=8, cold=4096 + 17, top_pages=4, top_p=64, segment=256)
    data = generate(w, seed=8)
    store = OracleColdStore(w.page_size, w.groups)
    store.evict(data["cold_k"], data["cold_v"])
    qa = data["q"]
    g = torch.Generator().manual_seed(9)
    seg_b = (int(data["targets"][0, 0]) + 7) % (w.cold // w.segment)
    cold = data["cold_k"].float()
    qb = (cold[:, :, seg_b * w.segment:(seg_b + 1) * w.segment].mean(2).repeat_interleave(w.groups, 1)[:, :, None]
          + 0.1 * torch.randn(1, w.num_q_heads, 1, w.head_dim, generator=g)).to(w.dtype)
    _, _, ta = store.retrieve(qa, w.scaling, w.top_p, w.top_pages, step=3)
    _, _, tb = store.retrieve(qb, w.scaling, w.top_p, w.top_pages, step=3)
    assert ta.extra["reused"] is False and tb.extra["reused"] is True
    assert torch.equal(tb.pages, ta.pages) and torch.equal(tb.candidate_ids, ta.candidate_ids)
    # B's own union is different: the reuse matters.
    _, _, tb_own = OracleColdStore.retrieve(_copy(store), qb, w.scaling, w.top_p, w.top_pages)
    assert tb_own.pages.tolist() != ta.pages.tolist()
    # The reused selection is B's top-P over A's candidates.
    cand = ta.candidate_ids.numpy()
    fine = exact.scores64(f64(qb), f64(data["cold_k"])[:, :, cand], w.scaling, w.groups)
    want, gap = exact.top_k_set(exact.fine_aggregate(fine)[0], w.top_p)
    assert gap > 1e-3
    assert sorted(tb.selected_ids[0].tolist()) == cand[want].tolist()
    snap = store.telemetry.snapshot()["aggregates"]
    assert (snap["coarse_calls"], snap["coarse_real_calls"], snap["coarse_skipped_calls"], snap["fine_calls"]) == (2, 1, 1, 2)
    # Another step (or an eviction) starts a fresh coarse pass.
    _, _, tc = store.retrieve(qb, w.scaling, w.top_p, w.top_pages, step=4)
    assert tc.extra["reused"] is False and tc.pages.tolist() == tb_own.pages.tolist()
    store.retrieve(qa, w.scaling, w.top_p, w.top_pages, step=5)
    store.evict(data["hot_k"][:, :, :1], data["hot_v"][:, :, :1])
    _, _, td = store.retrieve(qb, w.scaling, w.top_p, w.top_pages, step=5)
    assert td.extra["reused"] is False


def _copy(store: OracleColdStore) -> OracleColdStore:
    """A store with the same rows and no cached candidates or telemetry."""
    c = OracleColdStore(store.page_size, store.groups)
    c.evict(store.all_k(), store.all_v())
    return c
