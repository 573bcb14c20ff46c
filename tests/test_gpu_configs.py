"""Parity at every decode configuration's stated size.

Each configuration (TinyLlama shape with 32,768 cold tokens, Qwen2.5-7B
shape with 262,144, Phi-3.5 MHA shape with 131,072, MQA with 1,048,576, and
the Qwen2.5-7B shape with 1,048,576, the headline workload) is generated on
the GPU with the seeded generator at its full cold length, evicted into the
HIP store in ragged pieces, copied to the host and evicted into the CPU
oracle.  Then:

  * every page summary: fp32 mean within 1e-5 relative of the fp64 mean,
    dtype summary = RNE(fp32 mean) bit for bit; every cold row bit-exact;
  * one decode-step retrieval with the host tier's full fine scan, and one
    with the pruned fine scan: both within the rounding bands, both equal
    to the oracle (the reference's op sequence) wherever the bands
    determine the selection, identical to each other (union, ids, order,
    K/V rows), the K/V rows bit-exact copies of the selected cold rows;
  * the selection is led by the target segment's tokens (the workload's
    intent), and the merged attention over [retrieved ; hot] meets the
    attention bar.

A separated-score case on the headline shape plants 256 tokens whose scores
stand far above every other candidate, so that the fine top-P is fully
determined under the bf16 score rounding: the selection must then equal the
planted set and the oracle's selection exactly.

Finally a union wider than one 4,096-page window with the bf16 MFMA coarse
scan writing the page bounds: pruned and full fine scans must agree.
"""

from __future__ import annotations

from dataclasses import replace

import numpy as np
import pytest
import torch

from kiv_amd import ColdKVStore, KIVConfig, ModelTopology
from kiv_amd.synthetic import WORKLOADS, Workload, generate
from oracle import exact
from oracle.torch_ref import OracleColdStore
from tests.test_gpu_retrieval import attention_check, check_retrieval, separation_line

pytestmark = pytest.mark.gpu

CONFIGS = ["tinyllama_32k", "qwen7b_256k", "phi35_128k", "mqa_1m", "qwen7b_1m"]


def fill(w: Workload, data: dict, device, pieces=(65536, 1000, 1), cfg: KIVConfig | None = None):
    """The HIP store filled from GPU-resident rows in ragged pieces, and the
    oracle from a host copy (the oracle cuts the same pages)."""
    cfg = cfg or KIVConfig(hot_budget=w.hot, top_p=w.top_p, page_size=w.page_size, top_pages=w.top_pages)
    topo = ModelTopology.manual(global_layer_indices=(0,), num_query_heads=w.num_q_heads,
                                num_kv_heads=w.num_kv_heads, head_dim=w.head_dim, num_hidden_layers=1)
    store = ColdKVStore(cfg, topo, device)
    t, i = 0, 0
    while t < w.cold:
        n = min(pieces[i % len(pieces)], w.cold - t)
        store.evict_from_hot(data["cold_k"][:, :, t:t + n], data["cold_v"][:, :, t:t + n])
        t += n
        i += 1
    host = {key: (val.cpu() if torch.is_tensor(val) else val) for key, val in data.items()}
    oracle = OracleColdStore(w.page_size, w.groups)
    oracle.evict(host["cold_k"], host["cold_v"])
    return store, oracle, cfg, host


def check_summaries_in_pieces(store: ColdKVStore, cold_k_host: torch.Tensor, w: Workload, pages: int = 512):
    s, s32 = store.read_summaries()
    s, s32 = s.cpu(), s32.cpu()
    N = store.num_pages
    assert s.shape[0] == N == w.cold // w.page_size
    assert torch.equal(s, s32.to(s.dtype))  # the dtype summary is RNE(fp32 mean)
    ps = w.page_size
    for p0 in range(0, N, pages):
        p1 = min(N, p0 + pages)
        m64 = exact.page_means(cold_k_host[:, :, p0 * ps:p1 * ps].float().numpy(), ps)   # [B, H, n, D]
        got = s32[p0:p1].numpy().astype(np.float64).transpose(1, 2, 0, 3)
        err = np.abs(got - m64)
        assert np.all(err <= 1e-5 * np.abs(m64) + 1e-30), f"pages {p0}..{p1}: max rel err {np.max(err / (np.abs(m64) + 1e-30))}"


def check_rows_on_device(store: ColdKVStore, data: dict, w: Workload, piece: int = 1 << 18):
    for t in range(0, w.cold, piece):
        n = min(piece, w.cold - t)
        k, v = store.read_tokens(t, n)
        assert torch.equal(k, data["cold_k"][:, :, t:t + n]) and torch.equal(v, data["cold_v"][:, :, t:t + n]), t


@pytest.mark.timeout(600)
@pytest.mark.parametrize("key", CONFIGS)
def test_config_at_stated_size(cuda, key):
    w = WORKLOADS[key]
    print(f"config {key}: Hq={w.num_q_heads} Hkv={w.num_kv_heads} D={w.head_dim} {w.dtype} cold={w.cold} "
          f"top_pages={w.top_pages} top_p={w.top_p}", flush=True)
    data = generate(w, seed=0, device=cuda)
    store, oracle, cfg, host = fill(w, data, cuda)
    assert store.cold_length == w.cold and store.num_pages == w.cold // w.page_size
    check_summaries_in_pieces(store, host["cold_k"], w)
    check_rows_on_device(store, data, w)
    q = host["q"]
    runs = {}
    for prune in (False, True):
        c = replace(cfg, fine_pruning=prune)
        info = {}
        k_out, v_out, sel = check_retrieval(store, oracle, c, w, host, q, min_det_c=0.0, info=info)
        runs[prune] = (k_out, v_out, sel, info["union"], store.fine_scan_stats())
        print(f"  pruning={prune}: union {len(info['union'])} pages, determined coarse {info['det_c']:.2f} "
              f"fine {min(info['det_f']):.2f}, slices read {runs[prune][4]}", flush=True)
        print("  " + separation_line(info["separation"]), flush=True)
    (k0, v0, sel0, u0, s0), (k1, v1, sel1, u1, s1) = runs[False], runs[True]
    assert u0 == u1 and np.array_equal(sel0, sel1)
    assert torch.equal(k0, k1) and torch.equal(v0, v1)
    assert s0[0] == s0[1] and s1[0] <= s1[1] == s0[1]
    # The target segments' tokens lead the selection.
    targets = host["targets"][0].tolist()
    lead = sel0[0][: min(64, sel0.shape[1])]
    assert np.isin(lead // w.segment, targets).all()
    assert np.isin(sel0[0] // w.segment, targets).mean() > 0.9
    attention_check(data["q"], k0, v0, data["hot_k"], data["hot_v"], w.scaling)


@pytest.mark.timeout(600)
@pytest.mark.parametrize("pruning", [False, True])
def test_headline_shape_separated_selection(cuda, pruning):
    """Qwen2.5-7B shape at 1,048,576 cold tokens with 256 planted tokens
    (every fourth token of the target segment, K doubled) whose scores
    (about 22) stand far above every other candidate (about 11 in the
    target segment, |s| < 6 elsewhere): the fine top-256 is determined under
    the bf16 rounding, and it must equal the planted set and the oracle's
    selection exactly, with the K/V rows of those tokens."""
    w = WORKLOADS["qwen7b_1m"]
    data = generate(w, seed=3, device=cuda)
    seg = int(data["targets"][0, 0])
    planted = torch.arange(seg * w.segment, (seg + 1) * w.segment, 4, device=cuda)
    assert planted.numel() == w.top_p
    data["cold_k"][:, :, planted] = (data["cold_k"][:, :, planted].float() * 2).to(w.dtype)
    store, oracle, cfg, host = fill(w, data, cuda, cfg=KIVConfig(top_p=w.top_p, top_pages=w.top_pages,
                                                                   fine_pruning=pruning))
    info = {}
    k_out, v_out, sel = check_retrieval(store, oracle, cfg, w, host, host["q"], min_det_c=0.0, info=info)
    print(f"separated ({'pruned' if pruning else 'full'} fine scan): union {len(info['union'])}, determined "
          f"coarse {info['det_c']:.2f} fine {info['det_f'][0]:.2f}, slices {store.fine_scan_stats()}", flush=True)
    print("  " + separation_line(info["separation"]), flush=True)
    assert info["separation"]["fine"][0]["differ"] == 0
    assert info["det_f"] == [1.0]
    want = set(planted.cpu().tolist())
    assert set(sel[0].tolist()) == want
    assert set(info["oracle_selected"][0].tolist()) == want
    idx = torch.from_numpy(sel[0])
    assert torch.equal(k_out[0].cpu(), host["cold_k"][0][:, idx]) and torch.equal(v_out[0].cpu(), host["cold_v"][0][:, idx])
    attention_check(data["q"], k_out, v_out, data["hot_k"], data["hot_v"], w.scaling)
    # The decode step's call (retrieval and attention in one; with pruning,
    # the fine select runs inside the gather's launch): the same selection.
    out = store.retrieve_attend(data["q"], w.scaling, cfg, data["hot_k"], data["hot_v"], None)
    rec = store.telemetry_snapshot()["recent"][-1]
    assert rec["selected_token_indices"] == sel[0].tolist()
    attention_check(data["q"], k_out, v_out, data["hot_k"], data["hot_v"], w.scaling, out=out)


@pytest.mark.timeout(600)
@pytest.mark.parametrize("tier", ["hbm", "split"])
def test_mha_pruning_on_device_tiers_at_stated_size(cuda, tier):
    """The Phi-3.5 MHA shape at 131,072 cold tokens with K in HBM: its union
    (up to 1,024 pages x 32 kv rows) is past the device tiers' pruning
    threshold, so the pruned fine scan runs by default; it must read a small
    part of the union's slices and return the full MFMA scan's ids, order
    and rows, within the bands and the 1e-3 rule against the oracle."""
    w = WORKLOADS["phi35_128k"]
    data = generate(w, seed=0, device=cuda)
    cfg0 = KIVConfig(hot_budget=w.hot, top_p=w.top_p, page_size=w.page_size, top_pages=w.top_pages, cold_tier=tier)
    store, oracle, cfg, host = fill(w, data, cuda, cfg=cfg0)
    runs = {}
    for prune in (True, False):
        info = {}
        k_out, v_out, sel = check_retrieval(store, oracle, replace(cfg, fine_pruning=prune), w, host, host["q"],
                                            min_det_c=0.0, info=info)
        runs[prune] = (k_out, v_out, sel, info["union"], store.fine_scan_stats())
        print(f"  {tier} pruning={prune}: union {len(info['union'])}, slices read {runs[prune][4]}; "
              + separation_line(info["separation"]), flush=True)
    (k1, v1, sel1, u1, s1), (k0, v0, sel0, u0, s0) = runs[True], runs[False]
    assert u1 == u0 and np.array_equal(sel1, sel0)
    assert torch.equal(k1, k0) and torch.equal(v1, v0)
    assert s0[0] == s0[1] == s1[1] and s1[0] < s1[1] // 10
    attention_check(data["q"], k1, v1, data["hot_k"], data["hot_v"], w.scaling)


@pytest.mark.timeout(300)
def test_pruned_mfma_bounds_union_wider_than_a_window(cuda):
    """bf16, head_dim 64 (the MFMA coarse scan writes the page bounds), 16
    kv heads with random queries over 9,000 pages of 16 tokens, each page
    its own cluster: the union exceeds 4,096 pages, so the pruned scan lists
    its pages in several windows.  Pruned and full scans must return the
    same ids, order and rows, and both must meet the oracle's bands."""
    w = Workload("prune_wide_bf16", 16, 16, 64, torch.bfloat16, hot=16, cold=9000 * 16 + 7, top_pages=500,
                 top_p=256, segment=16, page_size=16)
    data = generate(w, seed=23, device=cuda)
    g = torch.Generator().manual_seed(24)
    q = (torch.randn(1, 16, 1, 64, generator=g) * 1.5).to(w.dtype)
    store, oracle, cfg, host = fill(w, data, cuda, pieces=(50000, 3))
    runs = {}
    for prune in (True, False):
        info = {}
        k_out, v_out, sel = check_retrieval(store, oracle, replace(cfg, fine_pruning=prune), w, host, q,
                                            min_det_c=0.0, info=info)
        runs[prune] = (k_out.cpu(), v_out.cpu(), sel, info["union"], store.fine_scan_stats())
    (k1, v1, sel1, u1, s1), (k0, v0, sel0, u0, s0) = runs[True], runs[False]
    print(f"wide bf16 union: {len(u1)} pages, slices read pruned {s1} full {s0}", flush=True)
    assert len(u1) > 4096 and u1 == u0
    assert np.array_equal(sel1, sel0) and torch.equal(k1, k0) and torch.equal(v1, v0)
