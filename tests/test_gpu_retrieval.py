"""GPU parity of eviction, coarse/fine retrieval and the merged attention.

Each case builds the same cold tier in the HIP store (through the C-ABI
wrapper ColdKVStore) and in the CPU oracle, then checks:
  * page summaries: fp32 mean within 1e-5 relative of the fp64 mean, and the
    stored dtype summary equal to RNE(fp32 mean);
  * cold rows bit-exact;
  * union pages and top-P ids within the rounding bands of oracle/bands.py,
    and equal to the CPU oracle's (the reference's op sequence) wherever
    every selection boundary is determined;
  * returned K/V bit-exact copies of the selected cold rows, in descending
    score order;
  * merged attention within max-abs 2e-3 of fp64 softmax attention, plus
    the output's own rounding to the dtype (half an ulp).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from kiv_amd import ColdKVStore, KIVConfig, ModelTopology
from kiv_amd.attention import decode_attention
from kiv_amd.synthetic import WORKLOADS, Workload, generate
from oracle import exact
from oracle.torch_ref import OracleColdStore
from oracle.bands import check_topk, row_bands, score_interval

pytestmark = pytest.mark.gpu

DT = {torch.float16: "float16", torch.bfloat16: "bfloat16", torch.float32: "float32"}


def f64(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy().astype(np.float64)


def build(w: Workload, data: dict, device, chunks=(4096,), cold_tier="host", rounding="activation",
          pruning=False):
    cfg = KIVConfig(hot_budget=w.hot, top_p=w.top_p, page_size=w.page_size, top_pages=w.top_pages,
                    cold_tier=cold_tier, score_rounding=rounding, fine_pruning=pruning)
    topo = ModelTopology.manual(global_layer_indices=(0,), num_query_heads=w.num_q_heads,
                                num_kv_heads=w.num_kv_heads, head_dim=w.head_dim, num_hidden_layers=1)
    store = ColdKVStore(cfg, topo, device)
    oracle = OracleColdStore(w.page_size, w.groups)
    ck, cv = data["cold_k"], data["cold_v"]
    dk, dv = ck.to(device), cv.to(device)
    t, i = 0, 0
    while t < w.cold:
        n = min(chunks[i % len(chunks)], w.cold - t)
        store.evict_from_hot(dk[:, :, t:t + n], dv[:, :, t:t + n])
        oracle.evict(ck[:, :, t:t + n], cv[:, :, t:t + n])
        t += n
        i += 1
    return store, oracle, cfg


def check_summaries(store: ColdKVStore, data: dict, w: Workload):
    s, s32 = store.read_summaries()
    N = store.num_pages
    assert s.shape[0] == N
    if N == 0:
        return
    m64 = exact.page_means(f64(data["cold_k"]), w.page_size)       # [B, H, N, D]
    got32 = s32.cpu().numpy().astype(np.float64).transpose(1, 2, 0, 3)  # [B, H, N, D]
    err = np.abs(got32 - m64)
    assert np.all(err <= 1e-5 * np.abs(m64) + 1e-30), f"max rel err {np.max(err / (np.abs(m64) + 1e-30))}"
    # Stored dtype summary is RNE(fp32 mean), bit for bit.
    assert torch.equal(s.cpu(), s32.cpu().to(s.dtype))


def check_rows(store: ColdKVStore, data: dict):
    k, v = store.read_tokens()
    assert torch.equal(k.cpu(), data["cold_k"]) and torch.equal(v.cpu(), data["cold_v"])


def check_retrieval(store, oracle, cfg, w, data, q, rounding="activation", min_det_c=0.5, info=None):
    """Run one retrieval and check it; returns (k_out, v_out, sel ids [B, P']).

    ``min_det_c``: the least fraction of coarse rows whose top pages the
    bands must determine (unclustered model keys leave most rows open).
    ``info``, if given, receives the union, the determined fractions and
    the oracle's selection."""
    dev = store.device
    dtype = DT[w.dtype]
    k_out, v_out = store.retrieve_top_kv(q.to(dev), w.scaling, cfg)
    snap = store.telemetry_snapshot()["recent"]
    fine = snap[-1]
    assert fine["kind"] == "fine"
    B = q.shape[0]
    width = k_out.shape[2]
    sel = np.array(fine["selected_token_indices"], dtype=np.int64).reshape(B, width)
    cold_k, cold_v = data["cold_k"], data["cold_v"]
    q64 = q.cpu()
    N, ps, p = store.num_pages, w.page_size, store.cold_length - store.num_pages * w.page_size
    # Union of per-row top pages.
    if N > 0:
        coarse = snap[-2]
        assert coarse["kind"] == "coarse" and not coarse["skipped"]
        union = coarse["pages_selected"]
        assert union == sorted(set(union))
        summ, _ = store.read_summaries()
        summ = summ.cpu().permute(1, 2, 0, 3)  # [B, H, N, D] dtype as the kernel reads it
        lo_c, hi_c = score_interval(q64.float().numpy(), summ.float().numpy(), w.scaling, dtype, rounding)
        lo_c, hi_c = lo_c.reshape(-1, N), hi_c.reshape(-1, N)
        det_c = check_topk(set(union), lo_c, hi_c, min(cfg.top_pages, N))
        assert det_c >= min_det_c, f"only {det_c:.2f} of coarse rows determined"
    else:
        union, det_c = [], 1.0
    cand = exact.candidate_ids(np.array(union, dtype=np.int64), ps, N * ps, p)
    P = min(cfg.top_p, store.cold_length, cand.size)
    assert width == P
    ck = cold_k[:, :, torch.from_numpy(cand)]
    lo, hi = score_interval(q64.float().numpy(), ck.float().numpy(), w.scaling, dtype, rounding)
    lo_agg, hi_agg = lo.max(axis=(1, 2)), hi.max(axis=(1, 2))  # [B, C]
    pos = {int(g): i for i, g in enumerate(cand)}
    det_f = []
    for b in range(B):
        local = np.array([pos[int(g)] for g in sel[b]])
        assert len(set(local.tolist())) == width
        det_f.append(check_topk(set(local.tolist()), lo_agg[b:b + 1], hi_agg[b:b + 1], P))
        # Descending order: each entry can still be >= the next one.
        assert np.all(hi_agg[b, local[:-1]] >= lo_agg[b, local[1:]])
        # Returned rows are the selected cold rows, bit for bit.
        idx = torch.from_numpy(sel[b])
        assert torch.equal(k_out[b].cpu(), cold_k[b][:, idx]) and torch.equal(v_out[b].cpu(), cold_v[b][:, idx])
    # The CPU oracle (the reference's op sequence in the dtype) obeys the same
    # bands, and where every boundary is determined both pick the same sets.
    _, _, trace = oracle.retrieve(q64, w.scaling, cfg.top_p, cfg.top_pages)
    ns = None
    if rounding == "activation":
        ns = separation_check(oracle, trace, union, sel, q64, cold_k, w, cfg, dtype,
                              (lo_c, hi_c) if N > 0 else None, (lo_agg, hi_agg))
    if info is not None:
        info.update(union=union, det_c=det_c, det_f=det_f, oracle_pages=trace.pages,
                    oracle_selected=trace.selected_ids, trace=trace, separation=ns)
    if rounding == "activation":
        if N > 0:
            check_topk(set(trace.pages.tolist()), lo_c, hi_c, min(cfg.top_pages, N))
            if det_c == 1.0:
                assert trace.pages.tolist() == union
        if N == 0 or trace.pages.tolist() == union:
            for b in range(B):
                osel = set(trace.selected_ids[b].tolist())
                check_topk({pos[g] for g in osel}, lo_agg[b:b + 1], hi_agg[b:b + 1], P)
                if det_f[b] == 1.0:
                    assert osel == set(sel[b].tolist())
    return k_out, v_out, sel


def page_means64(cold_k: torch.Tensor, page_size: int, piece: int = 512) -> np.ndarray:
    """fp64 means of the finished pages of host rows [B, H, T, D]: [B, H, N, D], in pieces."""
    B, H, T, D = cold_k.shape
    N = T // page_size
    out = np.empty((B, H, N, D))
    for p0 in range(0, N, piece):
        p1 = min(N, p0 + piece)
        out[:, :, p0:p1] = exact.page_means(cold_k[:, :, p0 * page_size:p1 * page_size].double().numpy(), page_size)
    return out


def separation_check(oracle, trace, union, sel, q, cold_k, w, cfg, dtype, coarse_bands, fine_bands) -> dict:
    """The parity rule in its own terms: ids may differ from the reference's
    only where the scores are within 1e-3 of the selection boundary.

    Coarse: every page on which the union differs from the oracle's has a
    gap of at most 1e-3 (float64 or dtype-emulated) at a row's boundary
    (oracle/gaps.py).  Fine: the oracle's top-P over this union's
    candidates (its fine stage conditioned on the union, so that a union
    difference does not move the fine boundary) differs from the selection
    only in ids within 1e-3 of the boundary.  Also returns the band widths:
    per fine top-P the certainly-selected (must), possibly-selected (may)
    and selected counts, and for the coarse rows the summed and largest
    |may| - |must|."""
    from oracle import gaps

    out = {}
    B = q.shape[0]
    N, ps = oracle.num_pages, w.page_size
    qn = q.double().numpy()
    if N > 0:
        m64 = page_means64(cold_k, ps)
        s64 = exact.scores64(qn, m64, w.scaling, w.groups).reshape(-1, N)
        summ = torch.cat(oracle.summaries, dim=2).double().numpy()
        semu = exact.emulate_scores(exact.dots32(qn, summ, w.groups), w.scaling, dtype).reshape(-1, N)
        k = min(cfg.top_pages, N)
        ref_rows = [set(r.tolist()) for r in trace.extra["top_idx"].reshape(-1, k)]
        c = gaps.union_differences(set(union), set(trace.pages.tolist()), s64, semu, k, ref_rows)
        widths = [len(may) - len(must) for must, may in
                  (row_bands(lo, hi, k) for lo, hi in zip(*coarse_bands))]
        c.update(band_width_sum=int(sum(widths)), band_width_max=int(max(widths)))
        assert not c["violations"], f"union pages differ beyond 1e-3 of every boundary: {c}"
        out["coarse"] = c
    cond = oracle.retrieve_given_union(q, w.scaling, cfg.top_p, np.array(union, dtype=np.int64))
    cand = cond.candidate_ids
    P = sel.shape[1]
    assert cond.selected_ids.shape[1] == P
    ck = cold_k[:, :, cand].double().numpy()
    s64 = exact.scores64(qn, ck, w.scaling, w.groups).max(axis=(1, 2))
    semu = exact.emulate_scores(exact.dots32(qn, ck, w.groups), w.scaling, dtype).max(axis=(1, 2))
    pos = {int(g): i for i, g in enumerate(cand.tolist())}
    out["fine"] = []
    for b in range(B):
        got = {pos[int(g)] for g in sel[b]}
        ref = {pos[int(g)] for g in cond.selected_ids[b].tolist()}
        f = gaps.topk_differences(got, ref, s64[b], semu[b], P)
        must, may = row_bands(fine_bands[0][b], fine_bands[1][b], P)
        f.update(must=len(must), may=len(may), selected=P, candidates=len(cand))
        assert not f["violations"], f"fine ids differ beyond 1e-3 of the boundary: {f}"
        out["fine"].append(f)
    return out


def separation_line(ns: dict) -> str:
    """One line of separation_check's figures, for the test log."""
    parts = []
    c = ns.get("coarse")
    if c:
        parts.append(f"coarse: union {c['got']} vs oracle {c['ref']}, {c['differ']} differ (max gap f64 "
                     f"{c['max_gap64']:.2e}, emulated {c['max_gap_emu']:.2e}, min of both {c['max_gap_min']:.2e}); "
                     f"row bands |may|-|must| sum {c['band_width_sum']} max {c['band_width_max']}")
    for b, f in enumerate(ns["fine"]):
        parts.append(f"fine[{b}]: |must| {f['must']} |may| {f['may']} selected {f['selected']} of "
                     f"{f['candidates']}; vs oracle on this union {f['differ']} differ (max gap f64 "
                     f"{f['max_gap64']:.2e}, emulated {f['max_gap_emu']:.2e}, min of both {f['max_gap_min']:.2e})")
    return "; ".join(parts)


def attention_check(q, cold_k, cold_v, hot_k, hot_v, scaling, mask=None, tol=2e-3, out=None):
    """decode_attention (or a given output of the same attention) against fp64 softmax attention."""
    if out is None:
        out = decode_attention(q, cold_k, cold_v, hot_k, hot_v, mask, scaling)
    keys = torch.cat([cold_k, hot_k], dim=2) if cold_k is not None else hot_k
    vals = torch.cat([cold_v, hot_v], dim=2) if cold_v is not None else hot_v
    m = None
    if mask is not None:
        mm = mask.float() if mask.dtype != torch.bool else torch.where(mask, 0.0, float("-inf"))
        P = 0 if cold_k is None else cold_k.shape[2]
        m = np.concatenate([np.zeros(mm.shape[:-1] + (P,)), f64(mm)], axis=-1)
    ref = exact.attention64(f64(q), f64(keys), f64(vals), scaling, m)
    # The bar covers the fp32 computation; the output's own rounding to the
    # dtype (the reference rounds its output too) comes on top: half an ulp
    # of the dtype at the reference value.
    half_ulp = 0.5 * np.spacing(np.abs(ref).astype(np.float32)) * {
        torch.bfloat16: 2.0 ** 16, torch.float16: 2.0 ** 13, torch.float32: 1.0}[out.dtype]
    err = np.abs(f64(out) - ref)
    assert np.all(err <= tol + half_ulp), f"attention max-abs error {err.max()} (beyond rounding {(err - half_ulp).max()})"
    return err.max()


SMALL = [
    # name, workload overrides, eviction chunk pattern
    ("tiny_gqa_bf16", dict(num_q_heads=8, num_kv_heads=2, head_dim=64, dtype=torch.bfloat16, cold=3000,
                           hot=300, top_pages=4, top_p=64, segment=256), (1, 7, 128, 300, 1000)),
    ("tiny_mha_f16", dict(num_q_heads=4, num_kv_heads=4, head_dim=96, dtype=torch.float16, cold=2100,
                          hot=100, top_pages=3, top_p=100, segment=128, n_targets=4), (2048, 52)),
    ("tiny_mqa_bf16_d256", dict(num_q_heads=8, num_kv_heads=1, head_dim=256, dtype=torch.bfloat16, cold=5000,
                                hot=64, top_pages=8, top_p=200, segment=512), (4096, 904)),
    ("tiny_f32", dict(num_q_heads=4, num_kv_heads=2, head_dim=32, dtype=torch.float32, cold=1500, hot=50,
                      top_pages=5, top_p=40, segment=100), (333,)),
    ("small_pages", dict(num_q_heads=4, num_kv_heads=1, head_dim=64, dtype=torch.bfloat16, cold=777, hot=30,
                         top_pages=6, top_p=50, segment=64, page_size=16), (5, 11)),
    # head dims off the MFMA scan's multiples of 32: the SGPR-query scan
    ("d80_bf16", dict(num_q_heads=8, num_kv_heads=2, head_dim=80, dtype=torch.bfloat16, cold=2000, hot=64,
                      top_pages=4, top_p=64, segment=256), (2000,)),
    ("d112_f32", dict(num_q_heads=6, num_kv_heads=2, head_dim=112, dtype=torch.float32, cold=1500, hot=40,
                      top_pages=3, top_p=50, segment=200), (700, 800)),
    # head dims whose summary rows the scan reads zero-padded (5, 9, 15, 5 chunks of 16 bytes)
    ("d40_bf16", dict(num_q_heads=8, num_kv_heads=2, head_dim=40, dtype=torch.bfloat16, cold=2000, hot=64,
                      top_pages=4, top_p=64, segment=256), (999, 1001)),
    ("d72_f16", dict(num_q_heads=6, num_kv_heads=3, head_dim=72, dtype=torch.float16, cold=1800, hot=40,
                     top_pages=3, top_p=60, segment=200), (1800,)),
    ("d120_bf16_mha", dict(num_q_heads=4, num_kv_heads=4, head_dim=120, dtype=torch.bfloat16, cold=2100, hot=33,
                           top_pages=3, top_p=100, segment=128, n_targets=4), (2048, 52)),
    ("d20_f32", dict(num_q_heads=4, num_kv_heads=1, head_dim=20, dtype=torch.float32, cold=1500, hot=50,
                     top_pages=5, top_p=40, segment=100), (333,)),
    # more than 8 kv rows: the pruned scan reads the page bound tables, built by the
    # coarse select's extra blocks (MFMA coarse scan) or by their own kernel (VALU scan)
    ("mha16_f16_d64", dict(num_q_heads=16, num_kv_heads=16, head_dim=64, dtype=torch.float16, cold=2100, hot=64,
                           top_pages=3, top_p=100, segment=128, n_targets=4), (2048, 52)),
    ("mha12_bf16_d40", dict(num_q_heads=12, num_kv_heads=12, head_dim=40, dtype=torch.bfloat16, cold=2100, hot=33,
                            top_pages=3, top_p=100, segment=128, n_targets=4), (1000, 1100)),
]


@pytest.mark.parametrize("tier", ["host", "host_pruned", "hbm"])
@pytest.mark.parametrize("name,over,chunks", SMALL, ids=[c[0] for c in SMALL])
def test_small_parity(cuda, name, over, chunks, tier):
    """Each small case on the host tier (VALU fine scan; full and pruned)
    and in HBM (the MFMA fine scan where the head dim allows it)."""
    w = Workload(name=name, **over)
    data = generate(w, seed=1)
    store, oracle, cfg = build(w, data, cuda, chunks, cold_tier=tier.split("_")[0], pruning=tier == "host_pruned")
    assert store.cold_length == w.cold and store.num_pages == w.cold // w.page_size
    check_summaries(store, data, w)
    check_rows(store, data)
    k_out, v_out, _ = check_retrieval(store, oracle, cfg, w, data, data["q"])
    attention_check(data["q"].to(cuda), k_out, v_out, data["hot_k"].to(cuda), data["hot_v"].to(cuda), w.scaling)


def test_head_dim_off_the_chunk_grid_is_refused(cuda):
    """Rows move in 16-byte chunks: a bf16 head dim that is not a multiple of
    8 is refused at the first eviction (KIV_ERR_UNSUPPORTED), cleanly."""
    from kiv_amd import _native as nat

    cfg = KIVConfig(top_p=16, top_pages=2, page_size=16)
    topo = ModelTopology.manual(global_layer_indices=(0,), num_query_heads=4, num_kv_heads=2, head_dim=36,
                                num_hidden_layers=1)
    store = ColdKVStore(cfg, topo, cuda)
    k = torch.zeros(1, 2, 20, 36, dtype=torch.bfloat16, device=cuda)
    with pytest.raises(nat.KivError) as err:
        store.evict_from_hot(k, k)
    assert err.value.code == nat.ERR_UNSUPPORTED and "head_dim 36" in str(err.value)


@pytest.mark.parametrize("key,cold", [("tinyllama_32k", 32768), ("qwen7b_256k", 24576 + 77),
                                      ("phi35_128k", 8192 + 5), ("mqa_1m", 65536)])
def test_workload_parity(cuda, key, cold):
    w = WORKLOADS[key].with_cold(cold)
    data = generate(w, seed=0)
    store, oracle, cfg = build(w, data, cuda, chunks=(4096, 1000, 1))
    check_summaries(store, data, w)
    k_out, v_out, sel = check_retrieval(store, oracle, cfg, w, data, data["q"])
    # The target segment's tokens dominate the selection.
    seg = data["targets"][0].tolist()
    in_target = np.isin(sel[0] // w.segment, seg).mean()
    assert in_target > 0.9
    attention_check(data["q"].to(cuda), k_out, v_out, data["hot_k"].to(cuda), data["hot_v"].to(cuda), w.scaling)


def test_partial_only_and_small_cold(cuda):
    """N == 0 (partial page only) and cold < top_p: everything is returned."""
    w = Workload("partial", 8, 2, 64, torch.bfloat16, hot=16, cold=100, top_pages=4, top_p=256, segment=32)
    data = generate(w, seed=3)
    store, oracle, cfg = build(w, data, cuda, chunks=(1, 3, 40))
    assert store.num_pages == 0 and store.cold_length == 100
    k_out, v_out, sel = check_retrieval(store, oracle, cfg, w, data, data["q"])
    assert sorted(sel[0].tolist()) == list(range(100))
    snap = store.telemetry_snapshot()
    assert snap["recent"][-2]["skipped"] is True
    assert snap["aggregates"]["coarse_skipped_calls"] == 1


def test_fewer_pages_than_top_pages(cuda):
    w = Workload("fewpages", 4, 2, 64, torch.float16, hot=16, cold=3 * 128 + 9, top_pages=32, top_p=500,
                 segment=100)
    data = generate(w, seed=4)
    store, oracle, cfg = build(w, data, cuda, chunks=(200,))
    k_out, v_out, sel = check_retrieval(store, oracle, cfg, w, data, data["q"])
    assert store.telemetry_snapshot()["recent"][-2]["pages_selected"] == [0, 1, 2]
    assert sorted(sel[0].tolist()) == list(range(w.cold))


def test_batch_and_multi_query(cuda):
    """B = 2 and Q = 3: union over every (b, head, position); top-P per batch row."""
    w = Workload("bq", 8, 2, 64, torch.bfloat16, hot=32, cold=4096 + 33, top_pages=3, top_p=96, segment=256)
    data = generate(w, seed=5, batch=2)
    g = torch.Generator().manual_seed(9)
    q = data["q"].float().repeat(1, 1, 3, 1) + 0.05 * torch.randn(2, 8, 3, 64, generator=g)
    q = q.to(w.dtype)
    store, oracle, cfg = build(w, data, cuda, chunks=(1000, 7))
    check_rows(store, data)
    check_retrieval(store, oracle, cfg, w, data, q)


def test_fp32_scores_and_hbm_tier(cuda):
    w = Workload("f32rank", 8, 2, 128, torch.bfloat16, hot=64, cold=6000, top_pages=6, top_p=128, segment=512)
    data = generate(w, seed=6)
    store, oracle, cfg = build(w, data, cuda, chunks=(999,), cold_tier="hbm", rounding="fp32")
    check_rows(store, data)
    check_retrieval(store, oracle, cfg, w, data, data["q"], rounding="fp32")
    mem = store.memory_bytes()
    assert mem["k_index_cpu"] == 0 and mem["k_cold_gpu"] == store.num_pages * 128 * 2 * 128 * 2


@pytest.mark.parametrize("attend", [False, True])
def test_split_tier(cuda, attend):
    """K rows of finished pages in HBM, V rows in pinned host memory: the
    same selection and rows, alone and through the fused attention call."""
    w = Workload("split", 28, 4, 128, torch.bfloat16, hot=128, cold=9000 + 3, top_pages=8, top_p=256, segment=1024)
    data = generate(w, seed=7)
    store, oracle, cfg = build(w, data, cuda, chunks=(1000, 1), cold_tier="split")
    check_rows(store, data)
    q, hk, hv = data["q"].to(cuda), data["hot_k"].to(cuda), data["hot_v"].to(cuda)
    out = store.retrieve_attend(q, w.scaling, cfg, hk, hv, None) if attend else None
    k_out, v_out, _ = check_retrieval(store, oracle, cfg, w, data, data["q"])
    if attend:
        attention_check(q, k_out, v_out, hk, hv, w.scaling, None, out=out)
    mem = store.memory_bytes()
    row = store.num_pages * 128 * 4 * 128 * 2
    assert mem["k_cold_gpu"] == row and mem["v_store_cpu"] == row
    assert mem["k_index_cpu"] == 0 and mem["v_cold_gpu"] == 0


PRUNE = [
    # name, workload, batch, clustered (pruning expected to skip pages)
    ("qwen_shape", Workload("prune_qwen", 28, 4, 128, torch.bfloat16, hot=64, cold=20000 + 37, top_pages=16,
                            top_p=256, segment=1024), 1, True),
    ("gqa_batch2", Workload("prune_b2", 8, 2, 64, torch.bfloat16, hot=16, cold=8192 + 5, top_pages=8, top_p=128,
                            segment=512), 2, True),
    # 8 kv heads in 2 batch rows: 16 kv rows build the page bound tables,
    # and the speculative scan (8 kv heads) reads the bound keys itself
    ("gqa8_batch2", Workload("prune_g8b2", 16, 8, 64, torch.bfloat16, hot=16, cold=6000 + 3, top_pages=4,
                             top_p=128, segment=512, n_targets=2), 2, True),
    ("mqa_f16_d256", Workload("prune_mqa", 8, 1, 256, torch.float16, hot=16, cold=12000, top_pages=12,
                              top_p=300, segment=512), 1, True),
    ("mha_targets", Workload("prune_mha", 8, 8, 96, torch.bfloat16, hot=16, cold=6000 + 1, top_pages=6,
                             top_p=200, segment=256, n_targets=4), 1, True),
    # every token its own centroid: no page structure to prune on
    ("unclustered", Workload("prune_rand", 8, 2, 64, torch.bfloat16, hot=16, cold=5000, top_pages=8, top_p=128,
                             segment=1), 1, False),
]


PLAN_FEW = ("qwen_shape", "mqa_f16_d256")  # plans of at most a quarter of the union pages


@pytest.mark.parametrize("tier", ["host", "hbm", "split", "hbm_plan", "split_plan"])
@pytest.mark.parametrize("name,w,batch,clustered", PRUNE, ids=[c[0] for c in PRUNE])
def test_fine_pruning_keeps_the_selection(cuda, monkeypatch, name, w, batch, clustered, tier):
    """The pruned fine scan against the full scan on the same store: the
    same union, selected ids in the same order and the same K/V rows bit for
    bit (pruning skips only slices whose upper bound is below a lower bound
    of the P-th largest key).  Where pages were skipped the fine mean, which
    covers the scored candidates only, differs.  On the HBM-resident tiers
    pruning is forced (KIV_PRUNE_DEVICE_BYTES=0; by default it starts at
    256 MiB of union K) and the full scan is the MFMA scan.  *_plan: the
    default threshold, so the MFMA scan reads every slice and its plan
    blocks list the pages the fine select reads (whose keys it then clears
    whole: the next calls would show stale keys)."""
    from dataclasses import replace

    plan = tier.endswith("_plan")
    if tier in ("hbm", "split"):
        monkeypatch.setenv("KIV_PRUNE_DEVICE_BYTES", "0")
    data = generate(w, seed=2, batch=batch)
    store, oracle, cfg = build(w, data, cuda, chunks=(3000, 1, 511), cold_tier=tier.split("_")[0])
    q = data["q"]
    runs = {}
    # Pruned, full, pruned again: after a call that skipped little (the
    # unclustered case) the store pauses pruning and scans everything.
    for i, prune in enumerate((True, False, True)):
        c = replace(cfg, fine_pruning=prune)
        if i == 0:
            k_out, v_out, sel = check_retrieval(store, oracle, c, w, data, q)
        else:
            k_out, v_out = store.retrieve_top_kv(q.to(cuda), w.scaling, c)
        snap = store.telemetry_snapshot()["recent"]
        runs[i] = (k_out.cpu(), v_out.cpu(), snap[-2]["pages_selected"], snap[-1], store.fine_scan_stats())
        if i == 0:
            # The host tier's pruned scan takes each kv row's first
            # speculative page from the coarse select's read-ahead copy
            # (not where more than 8 kv rows build the page bound tables,
            # nor past 128 KiB of copies).
            kr, slice_bytes = batch * w.num_kv_heads, store._page_size * w.head_dim * w.dtype.itemsize
            want = kr * slice_bytes if tier == "host" and kr <= 8 and kr * slice_bytes <= (128 << 10) else 0
            assert store.readahead_bytes() == want
    (k1, v1, u1, f1, s1), (k0, v0, u0, f0, s0), (k2, v2, u2, f2, s2) = runs[0], runs[1], runs[2]
    assert u2 == u0 and f2["selected_token_indices"] == f0["selected_token_indices"]
    assert torch.equal(k2, k0) and torch.equal(v2, v0) and s2 == (s1 if clustered else s0)  # pruning kept / paused
    print(f"{name} ({tier}): union {len(u1)} pages, slices read pruned {s1} full {s0}, "
          f"fine mean pruned {f1['mean_score']} full {f0['mean_score']}", flush=True)
    assert s0[0] == s0[1] == s1[1] == len(u1) * batch * w.num_kv_heads and s1[0] <= s1[1]
    assert u1 == u0
    assert f1["selected_token_indices"] == f0["selected_token_indices"]
    assert torch.equal(k1, k0) and torch.equal(v1, v0)
    assert f1["top_score"] == f0["top_score"]
    if plan:
        assert s1 == s0  # the scan read every slice
        # The select reads the listed pages alone when they are at most a
        # quarter of the union (then their mean is higher), else the row.
        assert f1["mean_score"] >= f0["mean_score"]
        if name in PLAN_FEW:
            assert f1["mean_score"] > f0["mean_score"]
    elif clustered:
        assert s1[0] < s1[1] and f1["mean_score"] > f0["mean_score"]  # the skipped pages score low


def test_fine_pruning_speculative_pages_that_miss(cuda):
    """The pruned scan reads the top pages of each kv row's first query row
    before the threshold is known and scores them only if their bound
    reaches it.  Here kv row 1's queries are 8x longer, so the threshold
    comes from its pages and every page of kv row 0 falls below it: kv row
    0's speculative reads are all dropped and it scans nothing.  Two calls in
    a row (the second with other queries, so that a dropped slice's stale
    keys would show) return the full scan's ids and rows bit for bit."""
    from dataclasses import replace

    w = Workload("prune_spec_miss", 4, 2, 64, torch.bfloat16, hot=16, cold=8192 + 5, top_pages=8, top_p=128,
                 segment=512)
    data = generate(w, seed=31)
    store, oracle, cfg = build(w, data, cuda, chunks=(4096, 1, 511), pruning=True)
    gen = torch.Generator().manual_seed(32)
    for call in range(2):
        q = data["q"].float() + (0.2 * call) * torch.randn(data["q"].shape, generator=gen)
        q[:, 2:] *= 8.0  # query heads 2, 3 read kv row 1
        q = q.to(data["q"].dtype)
        k1, v1, sel1 = check_retrieval(store, oracle, cfg, w, data, q)
        s1 = store.fine_scan_stats()
        union = store.telemetry_snapshot()["recent"][-2]["pages_selected"]
        k0, v0 = store.retrieve_top_kv(q.to(cuda), w.scaling, replace(cfg, fine_pruning=False))
        sel0 = store.telemetry_snapshot()["recent"][-1]["selected_token_indices"]
        print(f"speculative misses, call {call}: union {len(union)} pages, slices read {s1}", flush=True)
        assert 0 < s1[0] <= len(union)  # kv row 1's slices at most: kv row 0 scanned none
        assert sel1.reshape(-1).tolist() == sel0
        assert torch.equal(k1.cpu(), k0.cpu()) and torch.equal(v1.cpu(), v0.cpu())


def _random_prune_case(seed: int):
    import random

    rng = random.Random(seed)
    hkv = rng.choice([1, 2, 4, 8, 16])
    G = max(1, min(rng.choice([1, 2, 4, 7, 8]), 64 // hkv))
    w = Workload(f"prune_rand{seed}", G * hkv, hkv, rng.choice([64, 96, 128, 256]),
                 rng.choice([torch.bfloat16, torch.float16]), hot=16,
                 cold=rng.choice([6000, 12000, 30000]) + rng.randrange(0, 127), top_pages=rng.choice([4, 8, 16, 32]),
                 top_p=rng.choice([64, 128, 256, 300]), segment=rng.choice([1, 256, 512, 1024]),
                 n_targets=rng.choice([1, 2]))
    return w, rng.choice([1, 1, 2])


@pytest.mark.parametrize("tier", ["host", "hbm"])
@pytest.mark.parametrize("seed", [1, 2, 3, 4, 5, 6])
def test_fine_pruning_random_shapes(cuda, monkeypatch, seed, tier):
    """Seeded random shapes (kv heads 1-16, head dims 64-256, one or two
    batch rows, clustered and unclustered keys): the pruned call (with the
    read-ahead, speculation or the page bound tables, as the shape selects)
    returns the full scan's ids and rows bit for bit; on the HBM tier with
    pruning forced."""
    from dataclasses import replace

    if tier == "hbm":
        monkeypatch.setenv("KIV_PRUNE_DEVICE_BYTES", "0")
    w, batch = _random_prune_case(seed)
    data = generate(w, seed=seed + 100, batch=batch)
    store, _, cfg = build(w, data, cuda, chunks=(3000,), cold_tier=tier, pruning=True)
    q = data["q"].to(cuda)
    k1, v1 = store.retrieve_top_kv(q, w.scaling, cfg)
    sel1 = store.telemetry_snapshot()["recent"][-1]["selected_token_indices"]
    s1 = store.fine_scan_stats()
    k0, v0 = store.retrieve_top_kv(q, w.scaling, replace(cfg, fine_pruning=False))
    sel0 = store.telemetry_snapshot()["recent"][-1]["selected_token_indices"]
    print(f"{w.name} ({tier}, B {batch}, hkv {w.num_kv_heads}, D {w.head_dim}): slices {s1}", flush=True)
    assert sel1 == sel0
    assert torch.equal(k1.cpu(), k0.cpu()) and torch.equal(v1.cpu(), v0.cpu())


def test_read_ahead_after_refill(cuda):
    """The coarse select's read-ahead copies each kv row's first speculative
    page into HBM on every pruned call.  A store reset and refilled with
    other rows (the same page numbers, new contents) must score the new
    rows: against the oracle of the new rows, and bit for bit against the
    full scan of the same store."""
    from dataclasses import replace

    w = Workload("read_ahead_refill", 28, 4, 128, torch.bfloat16, hot=16, cold=20000 + 37, top_pages=16,
                 top_p=256, segment=1024)
    data = generate(w, seed=51)
    store, oracle, cfg = build(w, data, cuda, chunks=(4096,), pruning=True)
    check_retrieval(store, oracle, cfg, w, data, data["q"])
    assert store.readahead_bytes() > 0
    store.reset()
    data2 = generate(w, seed=52)
    oracle2 = OracleColdStore(w.page_size, w.groups)
    dk, dv = data2["cold_k"].to(cuda), data2["cold_v"].to(cuda)
    for t in range(0, w.cold, 4096):
        n = min(4096, w.cold - t)
        store.evict_from_hot(dk[:, :, t:t + n], dv[:, :, t:t + n])
        oracle2.evict(data2["cold_k"][:, :, t:t + n], data2["cold_v"][:, :, t:t + n])
    k1, v1, sel1 = check_retrieval(store, oracle2, cfg, w, data2, data2["q"])
    assert store.readahead_bytes() > 0
    k0, v0 = store.retrieve_top_kv(data2["q"].to(cuda), w.scaling, replace(cfg, fine_pruning=False))
    sel0 = store.telemetry_snapshot()["recent"][-1]["selected_token_indices"]
    assert sel1.reshape(-1).tolist() == sel0
    assert torch.equal(k1.cpu(), k0.cpu()) and torch.equal(v1.cpu(), v0.cpu())


def test_fine_pruning_speculative_wide_union(cuda):
    """Speculation with a union of more than 256 pages (a row list of 1024
    entries, the most it takes): the threshold and the page list read the
    union's bound keys from the LDS tables by rank (not one page per
    thread).  Unclustered keys, so most pages reach T; the same ids and rows
    as the full scan (random query rows, so that their top pages differ)."""
    from dataclasses import replace

    w = Workload("prune_spec_wide", 32, 4, 64, torch.bfloat16, hot=16, cold=1024 * 128 + 3, top_pages=32,
                 top_p=256, segment=1)
    data = generate(w, seed=41)
    store, oracle, cfg = build(w, data, cuda, chunks=(65536,), pruning=True)
    # independent query rows: their top pages barely overlap
    q = torch.randn(1, 32, 1, 64, generator=torch.Generator().manual_seed(42)).to(torch.bfloat16)
    k1, v1, sel1 = check_retrieval(store, oracle, cfg, w, data, q, min_det_c=0.0)
    union = store.telemetry_snapshot()["recent"][-2]["pages_selected"]
    s1 = store.fine_scan_stats()
    k0, v0 = store.retrieve_top_kv(q.to(cuda), w.scaling, replace(cfg, fine_pruning=False))
    sel0 = store.telemetry_snapshot()["recent"][-1]["selected_token_indices"]
    print(f"speculative wide union: {len(union)} pages, slices read {s1}", flush=True)
    assert len(union) > 256
    assert sel1.reshape(-1).tolist() == sel0
    assert torch.equal(k1.cpu(), k0.cpu()) and torch.equal(v1.cpu(), v0.cpu())


def test_fine_pruning_union_wider_than_a_window(cuda):
    """A union of more than 4096 pages: the pruned scan lists its pages in
    two windows (and the fine select falls back to the whole row); the same
    ids and rows as the full scan."""
    from dataclasses import replace

    w = Workload("prune_wide", 8, 1, 32, torch.float32, hot=8, cold=6000 * 16 + 3, top_pages=1000, top_p=256,
                 segment=16, page_size=16)
    data = generate(w, seed=21)
    q = torch.randn(1, 8, 1, 32, generator=torch.Generator().manual_seed(22))
    store, oracle, cfg = build(w, data, cuda, chunks=(20000,), pruning=True)
    k1, v1, sel1 = check_retrieval(store, oracle, cfg, w, data, q)
    union = store.telemetry_snapshot()["recent"][-2]["pages_selected"]
    s1 = store.fine_scan_stats()
    k0, v0 = store.retrieve_top_kv(q.to(cuda), w.scaling, replace(cfg, fine_pruning=False))
    sel0 = store.telemetry_snapshot()["recent"][-1]["selected_token_indices"]
    print(f"wide union: {len(union)} pages, slices read {s1}", flush=True)
    assert len(union) > 4096
    assert sel1.reshape(-1).tolist() == sel0
    assert torch.equal(k1.cpu(), k0.cpu()) and torch.equal(v1.cpu(), v0.cpu())


@pytest.mark.parametrize("clustered", [True, False])
def test_fine_pruning_compact_staging(cuda, monkeypatch, clustered):
    """A staging cap too small for candidate-indexed K staging: the pruned
    scan stages one slice per kv row compactly (the slot table) and the
    selected rows' K of the others comes from host memory; unclustered keys
    prune nothing, so the second call runs paused (full scan, slots by union
    rank).  Every call returns the full scan's ids and rows."""
    from dataclasses import replace

    w = Workload("prune_cstage", 8, 8, 96, torch.bfloat16, hot=16, cold=6000 + 1, top_pages=6, top_p=200,
                 segment=256 if clustered else 1, n_targets=4)
    data = generate(w, seed=2)
    store, oracle, cfg = build(w, data, cuda, chunks=(3000, 1, 511), pruning=True)
    # a slice is 128 tokens x 192 bytes; 8 kv rows: a 256 KiB cap holds one slot per row
    monkeypatch.setenv("KIV_STAGE_CAP_BYTES", str(256 << 10))
    q = data["q"]
    k1, v1, sel1 = check_retrieval(store, oracle, cfg, w, data, q)
    s1 = store.fine_scan_stats()
    k2, v2 = store.retrieve_top_kv(q.to(cuda), w.scaling, cfg)
    sel2 = store.telemetry_snapshot()["recent"][-1]["selected_token_indices"]
    k0, v0 = store.retrieve_top_kv(q.to(cuda), w.scaling, replace(cfg, fine_pruning=False))
    sel0 = store.telemetry_snapshot()["recent"][-1]["selected_token_indices"]
    print(f"compact staging ({'clustered' if clustered else 'unclustered'}): slices read {s1}", flush=True)
    if clustered:
        assert s1[0] < s1[1]
    assert sel1.reshape(-1).tolist() == sel0 == sel2
    assert torch.equal(k1.cpu(), k0.cpu()) and torch.equal(v1.cpu(), v0.cpu())
    assert torch.equal(k2.cpu(), k0.cpu()) and torch.equal(v2.cpu(), v0.cpu())


def test_width_depends_on_union(cuda):
    """top_p > top_pages * page_size: the width follows the union size."""
    w = Workload("wide", 4, 1, 64, torch.bfloat16, hot=8, cold=64 * 10, top_pages=2, top_p=300, segment=64,
                 page_size=64)
    data = generate(w, seed=7)
    store, oracle, cfg = build(w, data, cuda, chunks=(640,))
    k_out, _, sel = check_retrieval(store, oracle, cfg, w, data, data["q"])
    union = store.telemetry_snapshot()["recent"][-2]["pages_selected"]
    assert k_out.shape[2] == min(300, len(union) * 64)
    # A shared layer's call in the same step takes its width from that union too.
    q2 = (data["q"].float() + 0.3 * torch.randn(data["q"].shape, generator=torch.Generator().manual_seed(8)))
    k1, _ = store.retrieve_top_kv(data["q"].to(cuda), w.scaling, cfg, step=1)
    k2, _ = store.retrieve_top_kv(q2.to(w.dtype).to(cuda), w.scaling, cfg, step=1)
    recent = store.telemetry_snapshot()["recent"]
    assert recent[-2]["skipped"] is True and recent[-4]["skipped"] is False
    assert k2.shape[2] == k1.shape[2] == min(300, len(recent[-4]["pages_selected"]) * 64)
    assert recent[-1]["actual_P"] == k2.shape[2]


def test_reuse_candidates_by_step(cuda):
    """bf16: a shared layer's call in the same decode step, with a different
    query, skips the coarse pass and scores the first call's union with its
    own query rows, as the oracle's reuse does (kiv/cold_store.py:303-317):
    within the bands over that union's candidates, ids apart from the
    oracle's only within 1e-3 of the boundary, rows bit-exact.  An eviction
    in between drops the union (kiv/cold_store.py:148-151)."""
    from oracle import gaps

    w = Workload("reuse", 8, 2, 64, torch.bfloat16, hot=8, cold=4096 + 77, top_pages=4, top_p=64, segment=256)
    data = generate(w, seed=8)
    store, oracle, cfg = build(w, data, cuda)
    q1 = data["q"]
    q2 = (q1.float() + 0.5 * torch.randn(q1.shape, generator=torch.Generator().manual_seed(81))).to(w.dtype)
    store.retrieve_top_kv(q1.to(cuda), w.scaling, cfg, step=5)
    k2, v2 = store.retrieve_top_kv(q2.to(cuda), w.scaling, cfg, step=5)
    _, _, t1 = oracle.retrieve(q1, w.scaling, cfg.top_p, cfg.top_pages, step=5)
    _, _, t2 = oracle.retrieve(q2, w.scaling, cfg.top_p, cfg.top_pages, step=5)
    assert t2.extra["reused"]
    rec = store.telemetry_snapshot()["recent"]
    assert rec[-2]["skipped"] is True and rec[-4]["skipped"] is False
    union, sel = rec[-4]["pages_selected"], rec[-1]["selected_token_indices"]
    N, ps = store.num_pages, w.page_size
    cand = exact.candidate_ids(np.array(union, dtype=np.int64), ps, N * ps, store.cold_length - N * ps)
    ck = data["cold_k"][:, :, torch.from_numpy(cand)]
    lo, hi = score_interval(q2.float().numpy(), ck.float().numpy(), w.scaling, "bfloat16", "activation")
    pos = {int(g): i for i, g in enumerate(cand)}
    check_topk({pos[g] for g in sel}, lo.max(axis=(1, 2)), hi.max(axis=(1, 2)), w.top_p)
    cond = oracle.retrieve_given_union(q2, w.scaling, cfg.top_p, np.array(union, dtype=np.int64))
    if union == t1.pages.tolist():
        assert torch.equal(cond.selected_ids, t2.selected_ids)   # the oracle's own reuse
    s64, semu = gaps.scores_both(q2.double().numpy(), ck.double().numpy(), w.scaling, "bfloat16")
    f = gaps.topk_differences({pos[g] for g in sel}, {pos[int(g)] for g in cond.selected_ids[0]},
                              s64.max(axis=(1, 2))[0], semu.max(axis=(1, 2))[0], w.top_p)
    assert not f["violations"], f
    idx = torch.tensor(sel)
    assert torch.equal(k2[0].cpu(), data["cold_k"][0][:, idx]) and torch.equal(v2[0].cpu(), data["cold_v"][0][:, idx])
    snap = store.telemetry_snapshot()
    assert snap["aggregates"]["coarse_real_calls"] == 1 and snap["aggregates"]["coarse_skipped_calls"] == 1
    store.evict_from_hot(data["hot_k"][:, :, :1].to(cuda), data["hot_v"][:, :, :1].to(cuda))
    assert store._cached_candidate_k is None
    store.retrieve_top_kv(q2.to(cuda), w.scaling, cfg, step=5)  # same step, after an eviction: a fresh pass
    assert store.telemetry_snapshot()["recent"][-2]["skipped"] is False


def test_tie_break_lowest_index(cuda):
    """Identical K rows tie exactly: the lower token id wins, deterministically."""
    dev = cuda
    cfg = KIVConfig(top_p=5, top_pages=2, page_size=8)
    topo = ModelTopology.manual(global_layer_indices=(0,), num_query_heads=2, num_kv_heads=1, head_dim=16,
                                num_hidden_layers=1)
    store = ColdKVStore(cfg, topo, dev)
    k = torch.ones(1, 1, 64, 16, dtype=torch.bfloat16)
    v = torch.arange(64, dtype=torch.bfloat16)[None, None, :, None].repeat(1, 1, 1, 16)
    store.evict_from_hot(k.to(dev), v.to(dev))
    q = torch.ones(1, 2, 1, 16, dtype=torch.bfloat16)
    ko, vo = store.retrieve_top_kv(q.to(dev), 0.25, cfg)
    snap = store.telemetry_snapshot()["recent"]
    assert snap[-2]["pages_selected"] == [0, 1]
    assert snap[-1]["selected_token_indices"] == [0, 1, 2, 3, 4]
    assert torch.equal(vo[0, 0, :, 0].cpu(), torch.arange(5, dtype=torch.bfloat16))


@pytest.mark.parametrize("mask_kind", ["none", "bool", "float"])
def test_attention_masks_and_edges(cuda, mask_kind):
    g = torch.Generator().manual_seed(11)
    B, hq, hkv, D, P, T = 2, 12, 4, 128, 37, 301
    q = torch.randn(B, hq, 1, D, generator=g).to(torch.bfloat16)
    ck = torch.randn(B, hkv, P, D, generator=g).to(torch.bfloat16)
    cv = torch.randn(B, hkv, P, D, generator=g).to(torch.bfloat16)
    hk = torch.randn(B, hkv, T, D, generator=g).to(torch.bfloat16)
    hv = torch.randn(B, hkv, T, D, generator=g).to(torch.bfloat16)
    mask = None
    if mask_kind == "bool":
        mask = torch.rand(B, 1, 1, T, generator=g) > 0.3
    elif mask_kind == "float":
        mask = torch.where(torch.rand(B, 1, 1, T, generator=g) > 0.3, 0.0, -1e9).to(torch.bfloat16)
    d = lambda t: None if t is None else t.to(cuda)
    attention_check(d(q), d(ck), d(cv), d(hk), d(hv), D ** -0.5, d(mask))
    attention_check(d(q), None, None, d(hk), d(hv), D ** -0.5, d(mask))       # no cold keys
    attention_check(d(q), d(ck), d(cv), d(hk)[:, :, :0], d(hv)[:, :, :0], D ** -0.5)  # no hot keys
    # Non-contiguous hot window (a slice of a longer cache).
    big_k = torch.randn(B, hkv, T + 50, D, generator=g).to(torch.bfloat16)
    big_v = torch.randn(B, hkv, T + 50, D, generator=g).to(torch.bfloat16)
    attention_check(d(q), d(ck), d(cv), d(big_k)[:, :, 50:], d(big_v)[:, :, 50:], D ** -0.5)


@pytest.mark.parametrize("dtype,d", [(torch.bfloat16, 512), (torch.float32, 256)])
def test_full_wave_rows(cuda, dtype, d):
    """Rows of 64 chunks: a whole wave cooperates on one row."""
    w = Workload("wide_rows", 4, 2, d, dtype, hot=40, cold=1300, top_pages=3, top_p=70, segment=200)
    data = generate(w, seed=12)
    store, oracle, cfg = build(w, data, cuda, chunks=(500,))
    check_summaries(store, data, w)
    k_out, v_out, _ = check_retrieval(store, oracle, cfg, w, data, data["q"])
    attention_check(data["q"].to(cuda), k_out, v_out, data["hot_k"].to(cuda), data["hot_v"].to(cuda), w.scaling)


def test_large_union_multi_tile(cuda):
    """Random queries spread the per-head top pages: the union exceeds 256
    pages, more keys (> 32768) than the fine select holds in registers, so
    it reads the row from memory on every pass."""
    w = Workload("bigunion", 32, 8, 64, torch.bfloat16, hot=16, cold=65536 + 50, top_pages=32, top_p=512,
                 segment=128)
    data = generate(w, seed=13)
    g = torch.Generator().manual_seed(14)
    q = (torch.randn(1, 32, 1, 64, generator=g) * 2).to(torch.bfloat16)
    store, oracle, cfg = build(w, data, cuda, chunks=(65536, 50))
    check_retrieval(store, oracle, cfg, w, data, q)
    union = store.telemetry_snapshot()["recent"][-2]["pages_selected"]
    assert len(union) * 128 > 32768


@pytest.mark.parametrize("n_pages,top_pages,top_p", [(1500, 300, 200), (3000, 300, 600), (3000, 300, 2500)])
def test_select_large_k_paths(cuda, n_pages, top_pages, top_p):
    """top-k larger than the select block makes every key a candidate: the
    coarse threshold then comes from the block search over the LDS
    candidates (1500 <= 2048) or over the row itself (3000).  In the fine
    select, top_p = 2500 leaves every wave short of its share of maxima, so
    all of the row's keys (more than 2048) are candidates: the k-th largest
    comes from the search over the row in memory and the gather ranks 2500
    listed entries.  On the host tier the pruned fine scan lists the union
    pages whose bound reaches its threshold in windows; the list must stop
    at the union size even where a zero threshold passes every key (a
    regression: padding threads once did and listed pages past it)."""
    w = Workload("largek", 4, 1, 32, torch.float32, hot=8, cold=n_pages * 16 + 5, top_pages=top_pages,
                 top_p=top_p, segment=64, page_size=16)
    data = generate(w, seed=16)
    q = torch.randn(1, 4, 1, 32, generator=torch.Generator().manual_seed(17))
    store, oracle, cfg = build(w, data, cuda, chunks=(8192,), pruning=True)
    check_retrieval(store, oracle, cfg, w, data, q)
    union = store.telemetry_snapshot()["recent"][-2]["pages_selected"]
    assert len(union) >= top_pages


def test_fine_select_lds_search(cuda):
    """Fewer keys (1024 < n <= 2048) than the fine select block has key
    sub-slots: the waves set no bound, all n keys are candidates, more than
    the 1024 the gather ranks, so the k-th largest comes from the block
    search over the LDS candidates."""
    w = Workload("fineB", 4, 1, 32, torch.float32, hot=8, cold=4000, top_pages=16, top_p=600, segment=64,
                 page_size=32)
    data = generate(w, seed=18)
    q = torch.randn(1, 4, 1, 32, generator=torch.Generator().manual_seed(19))
    store, oracle, cfg = build(w, data, cuda, chunks=(4000,))
    check_retrieval(store, oracle, cfg, w, data, q)
    union = store.telemetry_snapshot()["recent"][-2]["pages_selected"]
    assert 1024 < len(union) * 32 <= 2048


@pytest.mark.parametrize("P,T,masked", [(256, 2048, False), (37, 301, True), (0, 129, False), (64, 0, False)])
def test_attention_retrieved_and_hot_ranges(cuda, P, T, masked):
    """Retrieved and hot keys sit in separate splits: only-retrieved, only-hot
    and mixed sequences stay within the bar."""
    g = torch.Generator().manual_seed(21)
    B, hq, hkv, D = 1, 28, 4, 128
    mk = lambda *s: torch.randn(*s, generator=g).to(torch.bfloat16).to(cuda)
    q, ck, cv, hk, hv = mk(B, hq, 1, D), mk(B, hkv, P, D), mk(B, hkv, P, D), mk(B, hkv, T, D), mk(B, hkv, T, D)
    if P == 0:
        ck = cv = None
    mask = (torch.rand(B, 1, 1, T, generator=g) > 0.3).to(cuda) if masked else None
    attention_check(q, ck, cv, hk, hv, D ** -0.5, mask)


def test_attention_repeated_calls_share_workspace(cuda):
    """Consecutive calls reuse one workspace (split partials and counters)."""
    g = torch.Generator().manual_seed(15)
    B, hq, hkv, D, P, T = 1, 28, 4, 128, 256, 2048
    for _ in range(4):
        mk = lambda *s: torch.randn(*s, generator=g).to(torch.bfloat16).to(cuda)
        attention_check(mk(B, hq, 1, D), mk(B, hkv, P, D), mk(B, hkv, P, D), mk(B, hkv, T, D), mk(B, hkv, T, D),
                        D ** -0.5)


FUSED = [
    # name, workload overrides, hot-column mask
    ("qwen_shape_bf16", dict(num_q_heads=28, num_kv_heads=4, head_dim=128, dtype=torch.bfloat16, cold=9000,
                             hot=2048, top_pages=8, top_p=256, segment=1024), None),
    ("gqa_f16_masked", dict(num_q_heads=32, num_kv_heads=4, head_dim=64, dtype=torch.float16, cold=5000, hot=300,
                            top_pages=4, top_p=200, segment=512), "bool"),
    ("mqa_d256_at_capacity", dict(num_q_heads=8, num_kv_heads=1, head_dim=256, dtype=torch.bfloat16, cold=5000,
                                  hot=64, top_pages=4, top_p=128, segment=512), None),
    ("one_hot_row", dict(num_q_heads=8, num_kv_heads=2, head_dim=96, dtype=torch.bfloat16, cold=3000, hot=1,
                         top_pages=4, top_p=100, segment=256), None),
    # past one lane group's 8 keys: the final kernel's 16-key variant
    ("mha_d96_wide_final", dict(num_q_heads=8, num_kv_heads=8, head_dim=96, dtype=torch.float16, cold=6000, hot=100,
                                top_pages=6, top_p=500, segment=256, n_targets=4), "bool"),
    ("mqa_d256_wide_at_capacity", dict(num_q_heads=8, num_kv_heads=1, head_dim=256, dtype=torch.bfloat16, cold=5000,
                                       hot=64, top_pages=4, top_p=256, segment=512), None),
    # outside the fused path: two launches behind the same call
    ("over_capacity", dict(num_q_heads=8, num_kv_heads=1, head_dim=256, dtype=torch.bfloat16, cold=5000, hot=64,
                           top_pages=8, top_p=300, segment=512), None),
    ("fp32", dict(num_q_heads=4, num_kv_heads=2, head_dim=32, dtype=torch.float32, cold=1500, hot=50,
                  top_pages=5, top_p=40, segment=100), "float"),
]


@pytest.mark.parametrize("name,over,mask_kind", FUSED, ids=[c[0] for c in FUSED])
def test_retrieve_attend(cuda, name, over, mask_kind):
    """kiv_retrieve_attend: the hot window's splits run in the gather launch
    and one final kernel per query row attends the retrieved keys and merges.
    The output must meet the attention bar over the rows the retrieval
    selects (checked by a second, identical retrieval)."""
    w = Workload(name, **over)
    data = generate(w, seed=31)
    store, oracle, cfg = build(w, data, cuda)
    q, hk, hv = data["q"].to(cuda), data["hot_k"].to(cuda), data["hot_v"].to(cuda)
    g = torch.Generator().manual_seed(32)
    mask = None
    if mask_kind == "bool":
        mask = (torch.rand(1, 1, 1, w.hot, generator=g) > 0.3).to(cuda)
    elif mask_kind == "float":
        mask = torch.where(torch.rand(1, 1, 1, w.hot, generator=g) > 0.3, 0.0, -1e4).to(cuda)
    out = store.retrieve_attend(q, w.scaling, cfg, hk, hv, mask)
    assert out.shape == (1, 1, w.num_q_heads, w.head_dim) and out.dtype == w.dtype
    k_out, v_out, _ = check_retrieval(store, oracle, cfg, w, data, data["q"])
    attention_check(q, k_out, v_out, hk, hv, w.scaling, mask, out=out)


LONG_QUERIES = [
    # name, workload, batch, positions: long queries run the scans in passes
    # of query positions and build the union with the union kernels
    ("qwen_shape_two_passes", Workload("lq1", 28, 4, 128, torch.bfloat16, hot=64, cold=9000 + 21, top_pages=8,
                                       top_p=256, segment=1024), 1, 40),
    ("mha_long_row_list", Workload("lq2", 32, 32, 64, torch.float16, hot=64, cold=6000, top_pages=32, top_p=300,
                                   segment=512, n_targets=4), 1, 16),
    ("fp32_many_passes", Workload("lq3", 4, 2, 64, torch.float32, hot=16, cold=3000 + 5, top_pages=4, top_p=128,
                                  segment=256), 2, 200),
    # G * Q >= 32 query rows per kv row: the MFMA fine scan (first case too);
    # 32-token pages make slices shorter than its 64-token tile
    ("gqa_f16_mfma_scan_small_pages", Workload("lq4", 8, 2, 64, torch.float16, hot=32, cold=5000 + 77, top_pages=6,
                                               top_p=200, segment=256, page_size=32), 2, 24),
]


@pytest.mark.parametrize("batch", [1, 2])
@pytest.mark.parametrize("tier", ["host", "hbm"])
def test_long_query_select_plan(cuda, tier, batch):
    """A one-pass query of G * Q >= 32 rows per kv row runs the MFMA fine
    scan; with pruning on, its plan blocks list the pages the fine select
    reads.  Against the oracle and against the same store without pruning:
    the same ids in the same order and the same rows, twice in a row (the
    select clears the whole key row the full scan wrote); the plan is a few
    of the union's pages here, so the select reads them alone (on the HBM
    tier in a 1024-thread block whose waves past the eighth leave, one
    block per batch row)."""
    from dataclasses import replace

    w = Workload("lq_plan", 28, 4, 128, torch.bfloat16, hot=64, cold=20000 + 37, top_pages=16, top_p=256,
                 segment=1024)
    data = generate(w, seed=2, batch=batch)
    g = torch.Generator().manual_seed(44)
    store, oracle, cfg = build(w, data, cuda, cold_tier=tier)
    listed_fewer = 0
    for call in range(2):
        q = data["q"].float().repeat(1, 1, 5, 1)  # 35 rows per kv row
        q = (q + (0.05 + 0.05 * call) * torch.randn(q.shape, generator=g)).to(w.dtype)
        k1, v1, sel1 = check_retrieval(store, oracle, replace(cfg, fine_pruning=True), w, data, q)
        f1 = store.telemetry_snapshot()["recent"][-1]
        k0, v0 = store.retrieve_top_kv(q.to(cuda), w.scaling, cfg)
        f0 = store.telemetry_snapshot()["recent"][-1]
        assert f1["selected_token_indices"] == f0["selected_token_indices"]
        assert torch.equal(k1.cpu(), k0.cpu()) and torch.equal(v1.cpu(), v0.cpu())
        assert f1["top_score"] == f0["top_score"]
        listed_fewer += f1["mean_score"] > f0["mean_score"]  # the select read only the high pages
    assert listed_fewer > 0


@pytest.mark.parametrize("name,w,batch,positions", LONG_QUERIES, ids=[c[0] for c in LONG_QUERIES])
def test_long_query_retrieval(cuda, name, w, batch, positions):
    """Queries with many positions (a prefill chunk with live retrieval, as
    the reference's reuse-path prefill runs it): the union over every
    (batch, head, position) and the fine max over heads and positions must
    meet the same bar as decode."""
    data = generate(w, seed=41, batch=batch)
    g = torch.Generator().manual_seed(42)
    q = data["q"].float().repeat(1, 1, positions, 1)
    q = (q + 0.2 * torch.randn(q.shape, generator=g)).to(w.dtype)
    store, oracle, cfg = build(w, data, cuda)
    check_retrieval(store, oracle, cfg, w, data, q)
