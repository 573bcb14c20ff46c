"""Decode µs/layer of the tiered-cache hot path on one MI355X.

    python bench.py [--steps K] [--warmup W] [--workload qwen7b_1m] [--cold-tier host|hbm]
                    [--cache cold|warm]
    python bench.py --workload qwen15b_model_1m [--model-tokens T] [--decode-steps S]
    python bench.py --workload qwen15b_prefill_chunk [--steps K] [--warmup W]

One step = one global layer's decode step for one new token: evict the
oldest hot row to the cold tier (as the cache does at decode: the row is
written by the retrieval's first launch), coarse-to-fine retrieval over the cold
tier (page scan, per-head top pages, union, fine scores, top-P, K/V gather)
and the merged softmax over [retrieved ; hot].  Inputs are resident before
the timed region: the cold tier is filled (1,048,576 tokens for the default
workload) and the query / hot window live in HBM.

Caches.  In a model, a layer's summaries and hot window are evicted from
L2 and the memory-side cache by the other layers' traffic before the layer
runs again, so by default every step starts cold: an untimed 512 MiB read
precedes it and HIP events bracket the step alone.  --cache warm times
back-to-back steps of the one layer instead (reported as a variant too).

The JSON line carries the headline µs/layer/step, a second pass with HIP
events bracketing every kernel on its launch stream (per-stage average
durations), the summary scan's HBM roofline and the host-link kernels'
bandwidth against vendor peaks and against measured ceilings (the
kiv_probe_read_bandwidth read probes, same cache state), the union size,
the other cold tier, warm caches, and the reference's op sequence timed on
the host CPU (the oracle, as a baseline).

--workload qwen15b_model_1m runs a whole model instead: a random-init
Qwen2.5-1.5B-shaped decoder (28 layers, hidden 1536, 12 q / 2 kv heads,
head_dim 128, bf16) through KIVMiddleware: chunked prefill of 1,048,576
uniform random token ids (chunk 4096, hot cap 4096), then greedy decode
steps with retrieval in every layer.  It reports the prefill time and its
dense-FLOP rate against the bf16 MFMA peak, the decode step time, the
per-layer retrieval stages (store events) and the same model's step over
a plain 2048-token cache (no cold tier) for comparison.

--workload qwen15b_prefill_chunk times the matrix-core attention of one
prefill chunk of that model on its own: 4096 query positions over a hot
window of 8192 keys (the 4096-token cap plus the chunk), 12 q / 2 kv heads,
head_dim 128, bf16, under the boolean causal mask the model builds (mask
classification kernel included), against the bf16 MFMA peak, with torch's
SDPA on the same inputs beside it.
"""

from __future__ import annotations

import argparse
import ctypes as C
import json
from dataclasses import replace
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "decode µs/layer at 1M cold tokens; achieved HBM + host-link GB/s vs peak"
HBM_PEAK_GBS = 8000.0
HOST_LINK_PEAK_GBS = 63.0  # PCIe Gen5 x16, one direction


def parse():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="qwen7b_1m")
    ap.add_argument("--cold-tier", default="host", choices=("host", "hbm", "split"))
    ap.add_argument("--no-variant", action="store_true", help="skip the other cold tiers")
    ap.add_argument("--cpu-seconds", type=float, default=15.0, help="CPU baseline sample budget")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--no-pruning", action="store_true", help="host tier: full fine scan (KIVConfig.fine_pruning=False)")
    ap.add_argument("--cache", default="cold", choices=("cold", "warm"))
    ap.add_argument("--model-tokens", type=int, default=1 << 20, help="prompt length of the model workload")
    ap.add_argument("--decode-steps", type=int, default=128, help="greedy decode steps of the model workload")
    ap.add_argument("--profile-pass", action="store_true",
                    help="for rocprofv3 runs: the headline tier's steps only, plus a 64 MiB device copy "
                         "that calibrates the FETCH_SIZE / WRITE_SIZE counters")
    ap.add_argument("--trace-summary", metavar="KERNEL_TRACE_CSV",
                    help="print the per-kernel durations of the timed layer's steps in a rocprofv3 "
                         "--kernel-trace CSV of a --profile-pass run, and exit (no GPU)")
    return ap.parse_args()


SCRUB_BYTES = 512 << 20  # larger than L2 (8 x 4 MiB) plus the 256 MiB memory-side cache
# GPU clock cycles of a spin kernel after each scrub (about half a
# millisecond): the launching thread enqueues the whole step meanwhile, so
# the events around a step time the GPU's work and never wait for a launch.
HEAD_START_CYCLES = 1_000_000
MFMA_BF16_PEAK_TFLOPS = 2500.0  # dense
MODEL_WORKLOAD = "qwen15b_model_1m"
CHUNK_WORKLOAD = "qwen15b_prefill_chunk"


def make_scrub(dev):
    """A read of SCRUB_BYTES that leaves no workload data in L2 or the MALL,
    then `then()` if given, then a bounded spin (torch.cuda._sleep, no memory
    traffic) that gives the host its head start on the next step."""
    import torch

    buf = torch.ones(SCRUB_BYTES // 4, dtype=torch.int32, device=dev)

    def scrub(then=None):
        buf.sum()
        if then is not None:
            then()
        torch.cuda._sleep(HEAD_START_CYCLES)

    return scrub


def layer_before(scrub, w, cfg, dev, seed):
    """The scrub, then one decode step of another layer of the same shape
    (its own store, filled from another seed) before each timed step, as in
    a model whose layers run one after another: the timed layer's data is
    cold (the scrub evicted it and the other layer reads none of it) while
    the step's kernels are resident in the instruction caches and their
    code's translations in the TLBs.  After the scrub alone the code too
    comes from HBM, which adds 2-4 us to a step and makes its time depend
    on where the linker placed each kernel (kernels of identical machine
    code measured 26.4 and 28.9 us in two builds; 0.1 us apart with the
    other layer's step first).  Returns (scrub function, other layer's
    store), or (None, None) with warm caches."""
    if scrub is None:
        return None, None
    other, hk, hv, q = build_cold(w, cfg, dev, seed + 1)
    n = [0]

    def step():
        one_step(other, cfg, q, hk, hv, n[0], w.scaling)
        n[0] += 1

    return (lambda: scrub(then=step)), other


def build_cold(w, cfg, dev, seed):
    """Fill a store with the workload's cold tier; returns (store, hot_k, hot_v, q, incoming rows)."""
    import torch

    from kiv_amd import ColdKVStore, ModelTopology
    from kiv_amd.synthetic import generate_streaming

    topo = ModelTopology.manual(global_layer_indices=(0,), num_query_heads=w.num_q_heads,
                                num_kv_heads=w.num_kv_heads, head_dim=w.head_dim, num_hidden_layers=1)
    store = ColdKVStore(cfg, topo, dev)
    hot_k = hot_v = q = None
    for item in generate_streaming(w, seed, dev, chunk=65536):
        if item[0] == "cold":
            store.evict_from_hot(item[1], item[2])
        elif item[0] == "hot":
            hot_k, hot_v = item[1].contiguous(), item[2].contiguous()
        else:
            q = item[1].contiguous()
    torch.cuda.synchronize()
    return store, hot_k, hot_v, q


def one_step(store, cfg, q, hot_k, hot_v, i, scaling, attn_events=None, fused=True):
    """One decode step, as the middleware runs it: evict the oldest hot row (it
    cycles through the hot window's rows), then retrieval and the merged
    attention in one call (kiv_retrieve_attend).  fused=False runs them as
    two calls (kiv_retrieve, kiv_decode_attention), with attn_events around
    the attention."""
    from kiv_amd.attention import decode_attention

    T = hot_k.shape[2]
    j = (store.cold_length + i) % T
    store.evict_deferred(hot_k[:, :, j:j + 1], hot_v[:, :, j:j + 1])
    if fused:
        store.retrieve_attend(q, scaling, cfg, hot_k, hot_v, None)
        return
    k_out, v_out = store.retrieve_top_kv(q, scaling, cfg)
    if attn_events is not None:
        attn_events[0].record()
    decode_attention(q, k_out, v_out, hot_k, hot_v, None, scaling)
    if attn_events is not None:
        attn_events[1].record()


class StepTimer:
    """Pairs of HIP events without the system-scope fence (the kind the
    store's per-stage profiling uses), recorded on torch's current stream
    through the HIP runtime torch loaded: a default event adds a cache
    writeback and invalidate to every timestamp (an empty pair reads 5.1 µs,
    a fence-free one 3.9 µs on MI355X)."""

    FLAGS = 0x20000000  # hipEventDisableSystemFence

    def __init__(self, n, dev):
        import ctypes as C

        from kiv_amd import _native as nat

        self.C, self.stream = C, C.c_void_p(nat.stream_ptr(dev))
        hip = self.hip = C.CDLL("libamdhip64.so")  # the runtime torch already loaded
        hip.hipEventCreateWithFlags.argtypes = [C.POINTER(C.c_void_p), C.c_uint]
        hip.hipEventRecord.argtypes = [C.c_void_p, C.c_void_p]
        hip.hipEventElapsedTime.argtypes = [C.POINTER(C.c_float), C.c_void_p, C.c_void_p]
        hip.hipEventDestroy.argtypes = [C.c_void_p]
        self.ev = []
        for _ in range(2 * n):
            e = C.c_void_p()
            if hip.hipEventCreateWithFlags(C.byref(e), self.FLAGS) != 0:
                raise RuntimeError("hipEventCreateWithFlags failed")
            self.ev.append(e)

    def start(self, i):
        self.hip.hipEventRecord(self.ev[2 * i], self.stream)

    def stop(self, i):
        self.hip.hipEventRecord(self.ev[2 * i + 1], self.stream)

    def elapsed_us(self):
        out, ms = [], self.C.c_float()
        for i in range(len(self.ev) // 2):
            if self.hip.hipEventElapsedTime(self.C.byref(ms), self.ev[2 * i], self.ev[2 * i + 1]) != 0:
                raise RuntimeError("hipEventElapsedTime failed")
            out.append(ms.value * 1e3)
        return out

    def __del__(self):
        for e in getattr(self, "ev", []):
            self.hip.hipEventDestroy(e)


def event_pair_us(dev, scrub, n=50):
    """Median of an empty fence-free event pair after a scrub (the timer's own cost)."""
    import statistics

    import torch

    t = StepTimer(n, dev)
    for i in range(n):
        scrub()
        t.start(i)
        t.stop(i)
    torch.cuda.synchronize()
    return statistics.median(t.elapsed_us())


def time_steps(store, cfg, q, hot_k, hot_v, steps, warmup, scaling, scrub, fused=True):
    """µs per step: the mean of back-to-back steps (scrub None), or the
    median of steps each timed alone after a scrub (fence-free events).

    Python's cyclic garbage collector is paused while the steps are enqueued:
    a collection pass stalls the launching thread for milliseconds, which
    the GPU events would count as idle time inside a step."""
    import gc

    import torch

    gc.collect()
    gc.disable()
    try:
        return _time_steps(store, cfg, q, hot_k, hot_v, steps, warmup, scaling, scrub, fused)
    finally:
        gc.enable()


def _time_steps(store, cfg, q, hot_k, hot_v, steps, warmup, scaling, scrub, fused):
    import torch

    for i in range(warmup):
        one_step(store, cfg, q, hot_k, hot_v, i, scaling, fused=fused)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    if scrub is None:
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        ev0.record()
        for i in range(steps):
            one_step(store, cfg, q, hot_k, hot_v, i, scaling, fused=fused)
        ev1.record()
        torch.cuda.synchronize()
        gpu_us = ev0.elapsed_time(ev1) * 1e3 / steps
    else:
        import statistics

        timer = StepTimer(steps, q.device)
        for i in range(steps):
            scrub()
            timer.start(i)
            one_step(store, cfg, q, hot_k, hot_v, i, scaling, fused=fused)
            timer.stop(i)
        torch.cuda.synchronize()
        # The median: a page-end finalize lands in one step of page_size and
        # is added to the headline separately, amortized.
        gpu_us = statistics.median(timer.elapsed_us())
    wall_us = (time.perf_counter() - t0) * 1e6 / steps
    return gpu_us, wall_us


def profile_steps(store, cfg, q, hot_k, hot_v, steps, scaling, scrub, fused=True):
    """Per-stage average durations (µs) from HIP events bracketing each launch
    on its stream (the store's events; for the two-call step, events around
    the attention call)."""
    import torch

    from kiv_amd import _native as nat

    lib = nat.lib()
    n = min(max(steps, 2 * w_page_size(store)), 256)  # at least one page completes
    nat.check(lib.kiv_profile_enable(store._handle, 1), "kiv_profile_enable")
    counts, totals = (C.c_int64 * len(nat.STAGES))(), (C.c_double * len(nat.STAGES))()
    nat.check(lib.kiv_profile_read(store._handle, counts, totals), "kiv_profile_read")  # clear
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n)]
    for i in range(n):
        if scrub is not None:
            scrub()
        one_step(store, cfg, q, hot_k, hot_v, i, scaling, attn_events=ev[i], fused=fused)
    torch.cuda.synchronize()
    nat.check(lib.kiv_profile_read(store._handle, counts, totals), "kiv_profile_read")
    nat.check(lib.kiv_profile_enable(store._handle, 0), "kiv_profile_enable")
    stages = {}
    for i, name in enumerate(nat.STAGES):
        if counts[i]:
            stages[name] = {"launches": int(counts[i]), "avg_us": totals[i] / counts[i] * 1e3}
    if not fused:
        att = [a.elapsed_time(b) for a, b in ev]
        stages["attention"] = {"launches": n, "avg_us": sum(att) / n * 1e3}
    return stages


def w_page_size(store) -> int:
    return store._page_size


def host_inclusive(store, cfg, q, hot_k, hot_v, scaling, steps=200, warmup=20):
    """Wall-clock µs per step of back-to-back steps (no scrub) as a caller sees
    them: Python, ctypes, launches and the GPU, synchronised at both ends."""
    import gc

    import torch

    for i in range(warmup):
        one_step(store, cfg, q, hot_k, hot_v, i, scaling)
    torch.cuda.synchronize()
    gc.collect()
    gc.disable()
    try:
        t0 = time.perf_counter()
        for i in range(steps):
            one_step(store, cfg, q, hot_k, hot_v, i, scaling)
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) * 1e6 / steps
    finally:
        gc.enable()


def probes(dev, summary_bytes, host_bytes, cold):
    """Measured read ceilings (GB/s): HBM streaming, HBM at the summary scan's size and
    grid in the same cache state, and the host link (mapped pinned memory)."""
    from kiv_amd import _native as nat

    lib = nat.lib()
    st = nat.stream_ptr(dev)

    def run(where, nbytes, blocks, iters, cold_flag):
        g = C.c_double(0)
        nat.check(lib.kiv_probe_read_bandwidth(where, nbytes, blocks, iters, 1 if cold_flag else 0, C.byref(g), st),
                  "kiv_probe_read_bandwidth")
        return round(g.value, 1)

    scan_blocks = max(1, (summary_bytes // 16 + 2047) // 2048)  # 8 x 16 B per thread, as the scan's lanes
    # The same-size read is a latency floor, not a bandwidth ceiling: its
    # median over single timed reads, with the spread.
    same = sorted(run(nat.TIER_HBM, summary_bytes, scan_blocks, 1, cold) for _ in range(50))
    return {
        "hbm_stream_2GiB": run(nat.TIER_HBM, 2 << 30, 4096, 5, False),
        "hbm_summary_size": same[len(same) // 2],
        "hbm_summary_size_spread": [same[0], same[len(same) // 4], same[3 * len(same) // 4], same[-1]],
        "host_link_256MiB": run(nat.TIER_HOST, 256 << 20, 2048, 3, False),
        "host_link_fine_size": run(nat.TIER_HOST, max(host_bytes, 1 << 20), 1024, 5, False),
    }


def roofline_and_links(w, store, stages, union_pages, tier, scanned_slices=None, pruning=False, readahead=0):
    """Algorithmic bytes per launch / measured duration for every stage.
    scanned_slices: (union page, kv row) slices the fine scan read (fewer
    than union_pages * Hkv when the host tier's scan is pruned).
    readahead: host bytes the coarse select read ahead into HBM for the
    pruned scan (one slice per kv row, the first speculative page's)."""
    b = 2 if w.dtype.itemsize == 2 else 4
    row = w.num_kv_heads * w.head_dim * b          # one token, all kv heads
    if scanned_slices is None:
        scanned_slices = union_pages * w.num_kv_heads
    N = store.num_pages
    P = min(w.top_p, store.cold_length)
    p = store.cold_length - N * w.page_size
    cand = union_pages * w.page_size + p
    rows = w.num_q_heads
    # With the host tier's pruning the summary scan also reads each page
    # row's radius and norm (8 bytes) and writes its two bound keys (8 bytes).
    bounds = 16 * N * w.num_kv_heads if tier == "host" and pruning else 0
    # The read-ahead slices are host reads of the coarse select; the fine scan
    # takes them from HBM (when scanned: counting every one as scanned gives
    # the scan's host bytes from below).
    fine_bytes = scanned_slices * w.page_size * w.head_dim * b
    traffic = {
        # (bytes per launch, memory it streams from)
        "coarse_scan": (N * row + bounds, "hbm"),
        "coarse_select": (rows * N * 4 + readahead, "hbm"),
        # Pruned (host tier): the bytes are the (page, kv row) slices read.
        "fine_scan": (fine_bytes - readahead, "host") if tier == "host" else (fine_bytes, "hbm"),
        "fine_select": (cand * 4, "hbm"),
        # Host and split tiers: only V of the selected rows crosses the host
        # link (the host tier takes K from the fine scan's HBM staging, the
        # split tier keeps K in HBM; a pruned scan leaves a selected token's
        # K rows of skipped slices to be read from the host, at most P rows
        # per kv head, not counted here).  The fused step's gather launch also
        # runs the hot-window attention splits, which read the hot K/V from
        # HBM; they are not host-link bytes.
        "gather": ((2 if tier == "hbm" else 1) * P * row, "hbm" if tier == "hbm" else "host"),
        "attend": (2 * P * row, "hbm"),
        "attention": (2 * (P + w.hot) * row, "hbm"),
    }
    out = {}
    for name, (nbytes, where) in traffic.items():
        if name in stages:
            us = stages[name]["avg_us"]
            out[name] = {"bytes": nbytes, "from": where, "avg_us": us, "GB_s": nbytes / (us * 1e-6) / 1e9,
                         "host_bytes": nbytes if where == "host" else 0}
    if readahead and "coarse_select" in out:
        out["coarse_select"]["host_bytes"] = readahead
    return out


def host_cores() -> dict:
    """Host cores this process may use: the affinity mask, capped by a cgroup
    CPU quota when one is set (a GPU box gives each GPU a share of the host)."""
    cpus = len(os.sched_getaffinity(0))
    quota = None
    try:
        with open("/sys/fs/cgroup/cpu.max") as f:
            q, period = f.read().split()
        if q != "max":
            quota = max(1, int(int(q) / int(period)))
    except (OSError, ValueError):
        pass
    return {"threads": min(cpus, quota) if quota else cpus, "os_cpu_count": os.cpu_count(), "affinity": cpus,
            "cgroup_quota": quota}


def host_copy(store, piece=1 << 18):
    """The store's cold rows ([B, Hkv, cold, D] K and V) on the host."""
    ks, vs = [], []
    for t in range(0, store.cold_length, piece):
        k, v = store.read_tokens(t, min(piece, store.cold_length - t))
        ks.append(k.cpu())
        vs.append(v.cpu())
    import torch

    return torch.cat(ks, dim=2), torch.cat(vs, dim=2)


def selection_check(w, store, cfg, q, oracle, cold_k):
    """One retrieval on the GPU store against the oracle on the same rows: the
    union and the selected ids within the rounding bands (oracle.bands),
    equal to the oracle's where the bands determine them, and every id on
    which they differ within 1e-3 of a selection boundary in float64 or in
    the dtype rounding (oracle.gaps; the fine ids against the oracle's top-P
    over the same union)."""
    import numpy as np

    from oracle import exact, gaps
    from oracle.bands import check_topk, score_interval

    dt = {2: "bfloat16" if "bfloat" in str(w.dtype) else "float16", 4: "float32"}[w.dtype.itemsize]
    store.retrieve_top_kv(q, w.scaling, cfg)
    rec = store.telemetry_snapshot()["recent"]
    union, sel = rec[-2]["pages_selected"], rec[-1]["selected_token_indices"]
    _, _, trace = oracle.retrieve(q.cpu(), w.scaling, cfg.top_p, cfg.top_pages)
    N, ps = store.num_pages, w.page_size
    qh = q.float().cpu().numpy()
    summ = store.read_summaries()[0].cpu().permute(1, 2, 0, 3).float().numpy()
    lo, hi = score_interval(qh, summ, w.scaling, dt, "activation")
    out = {"union_pages": len(union), "oracle_union_pages": int(trace.pages.numel())}
    try:
        det_c = check_topk(set(union), lo.reshape(-1, N), hi.reshape(-1, N), min(cfg.top_pages, N))
        check_topk(set(trace.pages.tolist()), lo.reshape(-1, N), hi.reshape(-1, N), min(cfg.top_pages, N))
        cand = exact.candidate_ids(np.array(union, dtype=np.int64), ps, N * ps, store.cold_length - N * ps)
        import torch

        flo, fhi = score_interval(qh, cold_k[:, :, torch.from_numpy(cand)].float().numpy(), w.scaling, dt,
                                  "activation")
        pos = {int(g): i for i, g in enumerate(cand)}
        det_f = check_topk({pos[g] for g in sel}, flo.max(axis=(1, 2)), fhi.max(axis=(1, 2)),
                           rec[-1]["actual_P"])
        same_union = union == trace.pages.tolist()
        equal = None
        if same_union and det_f == 1.0:
            equal = set(sel) == set(trace.selected_ids[0].tolist())
        # The 1e-3 rule: union pages against the oracle's per-row selections,
        # fine ids against the oracle's top-P over this union.
        qd = q.double().cpu().numpy()
        kc = min(cfg.top_pages, N)
        m64 = np.concatenate([exact.page_means(cold_k[:, :, p0 * ps:min(N, p0 + 512) * ps].double().numpy(), ps)
                              for p0 in range(0, N, 512)], axis=2)
        osumm = torch.cat(oracle.summaries, dim=2).double().numpy()
        c = gaps.union_differences(set(union), set(trace.pages.tolist()),
                                   exact.scores64(qd, m64, w.scaling, w.groups).reshape(-1, N),
                                   exact.emulate_scores(exact.dots32(qd, osumm, w.groups), w.scaling, dt).reshape(-1, N),
                                   kc, [set(r.tolist()) for r in trace.extra["top_idx"].reshape(-1, kc)])
        cond = oracle.retrieve_given_union(q.cpu(), w.scaling, cfg.top_p, np.array(union, dtype=np.int64))
        ck = cold_k[:, :, cond.candidate_ids].double().numpy()
        s64 = exact.scores64(qd, ck, w.scaling, w.groups).max(axis=(1, 2))[0]
        semu = exact.emulate_scores(exact.dots32(qd, ck, w.groups), w.scaling, dt).max(axis=(1, 2))[0]
        cpos = {int(g): i for i, g in enumerate(cond.candidate_ids.tolist())}
        f = gaps.topk_differences({cpos[g] for g in sel}, {cpos[int(g)] for g in cond.selected_ids[0]}, s64, semu,
                                  len(sel))
        rule = {"union_ids_differing": c["differ"], "union_max_gap_f64": c["max_gap64"],
                "union_max_gap_dtype": c["max_gap_emu"], "fine_ids_differing": f["differ"],
                "fine_max_gap_f64": f["max_gap64"], "fine_max_gap_dtype": f["max_gap_emu"],
                "violations": len(c["violations"]) + len(f["violations"])}
        out.update(within_bands=True, coarse_rows_determined=round(det_c, 3), fine_determined=det_f == 1.0,
                   union_equal=same_union, selection_equal_where_determined=equal, rule_1e3=rule,
                   ok=equal is not False and (det_c < 1.0 or same_union) and rule["violations"] == 0)
    except AssertionError as e:
        out.update(within_bands=False, ok=False, error=str(e)[:200])
    return out


def cpu_baseline(w, store, cfg, q, hot_k, hot_v, budget_s):
    """The reference's op sequence (oracle.torch_ref) on host cores over the
    GPU store's own cold rows, query and hot window, after a selection check
    of the GPU retrieval against it."""
    import torch

    from oracle.torch_ref import OracleColdStore, decode_step

    cores = host_cores()
    torch.set_num_threads(cores["threads"])
    k, v = host_copy(store)
    oracle = OracleColdStore(w.page_size, w.groups)
    oracle.evict(k, v)
    oracle.flat()  # the reference materialises once before scoring (kiv/cold_store.py:122-136)
    check = selection_check(w, store, cfg, q, oracle, k)
    print(f"[bench] selection check against the oracle: {check}", file=sys.stderr, flush=True)
    qh, hk, hv = q.cpu(), hot_k.cpu(), hot_v.cpu()
    decode_step(oracle, qh, hk, hv, None, w.scaling, w.top_p, w.top_pages)  # warm-up
    times = []
    t_end = time.perf_counter() + budget_s
    while time.perf_counter() < t_end or len(times) < 3:
        t0 = time.perf_counter()
        decode_step(oracle, qh, hk, hv, None, w.scaling, w.top_p, w.top_pages)
        times.append(time.perf_counter() - t0)
    times.sort()
    med = times[len(times) // 2]
    return {"value": med * 1e6, "unit": "us/layer/step", "cores": cores["threads"], "kind": "port",
            "host": cores,
            "sample": f"{len(times)} retrieve+attention calls (median) over the GPU store's own "
                      f"{store.cold_length} cold tokens, query and hot window, copied to the host; torch CPU "
                      "ops of the reference sequence in the activation dtype"}, check


def profile_pass(w, args, dev, scrub):
    """The steps a profiler attributes per kernel, and the counters' calibration copy."""
    import torch

    from kiv_amd import KIVConfig

    cfg = KIVConfig(hot_budget=w.hot, top_p=w.top_p, page_size=w.page_size, top_pages=w.top_pages,
                    cold_tier=args.cold_tier, reserve_tokens=w.cold + args.steps + args.warmup + 1024,
                    fine_pruning=not args.no_pruning)
    store, hot_k, hot_v, q = build_cold(w, cfg, dev, args.seed)
    scrub_l, _other = layer_before(scrub, w, cfg, dev, args.seed)
    us, _ = time_steps(store, cfg, q, hot_k, hot_v, args.steps, args.warmup, w.scaling, scrub_l)
    src = torch.ones(64 << 20, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    for _ in range(3):
        if scrub is not None:
            scrub()
        dst.copy_(src)  # calibration: reads and writes 64 MiB
    torch.cuda.synchronize()
    print(json.dumps({"profile_pass": w.name, "cold_tier": args.cold_tier, "caches": args.cache, "steps": args.steps,
                      "us_per_step": round(us, 2), "calibration_copy_bytes": 64 << 20}), flush=True)


# Kernel families of the decode step in the counter summaries.
STAGE_KERNELS = {"coarse_scan": "coarse_scan", "coarse_select": "coarse_select", "fine_scan": "fine_scan",
                 "fine_select": "fine_select", "gather": "gather", "attend": "decode_attn_final"}


def load_pmc(workload, tier):
    """Memory traffic per launch of each decode-step kernel, from the rocprofv3
    --pmc summary committed under profiles/ (median per dispatch of the L2's
    read and write requests by destination, in 32-byte units: HBM and the
    host link), as {stage: {"hbm_read", "hbm_write", "host_read",
    "host_write", "traffic"}} in bytes, or {} when there is none."""
    path = os.path.join(ROOT, "profiles", f"decode_step_{workload}_{tier}_pmc.txt")
    out = {}
    if not os.path.exists(path):
        return out
    with open(path) as f:
        for line in f:
            parts = line.split()  # kernel name (it may hold spaces), then five byte counts
            if len(parts) < 6 or not parts[0].startswith("kiv::"):
                continue
            for stage, fam in STAGE_KERNELS.items():
                if parts[0].startswith(f"kiv::{fam}_"):
                    hr, hw, ir, iw = (int(x) for x in parts[-5:-1])
                    out[stage] = {"hbm_read": hr, "hbm_write": hw, "host_read": ir, "host_write": iw,
                                  "traffic": hr + hw + ir + iw}
    return out


def model_flops(cfg, tokens, chunk, cap):
    """Dense FLOPs of the chunked prefill: projections and MLP (2 per weight per
    token), attention QK^T and PV over each chunk's keys (hot cap + causal
    chunk), and the last token's LM head."""
    d, f, L = cfg.hidden_size, cfg.intermediate_size, cfg.num_hidden_layers
    hq, hkv, hd = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.hidden_size // cfg.num_attention_heads
    per_layer = d * hq * hd + 2 * d * hkv * hd + hq * hd * d + 3 * d * f
    linear = 2 * per_layer * L * tokens
    attn = 0
    for start in range(0, tokens, chunk):
        q = min(chunk, tokens - start)
        hot = min(start, cap)
        keys = q * hot + q * (q + 1) // 2          # query i sees the hot window and chunk rows <= i
        attn += 4 * hq * hd * keys * L
    head = 2 * d * cfg.vocab_size
    return linear + attn + head


def model_run(args):
    """Whole-model prefill + decode through KIVMiddleware (see the module docstring)."""
    import torch
    from transformers import DynamicCache, Qwen2Config, Qwen2ForCausalLM

    from kiv_amd import KIVConfig, KIVMiddleware
    from kiv_amd import _native as nat

    dev = torch.device("cuda", 0)
    T, chunk, cap = args.model_tokens, 4096, 4096
    cfg = Qwen2Config(vocab_size=151936, hidden_size=1536, intermediate_size=8960, num_hidden_layers=28,
                      num_attention_heads=12, num_key_value_heads=2, max_position_embeddings=T + 8192,
                      rope_theta=1e6, tie_word_embeddings=True)
    cfg._attn_implementation = "sdpa"
    torch.manual_seed(args.seed)
    with torch.device(dev):
        model = Qwen2ForCausalLM(cfg)
    model = model.to(torch.bfloat16).eval()
    kcfg = KIVConfig(hot_budget=2048, top_p=256, page_size=128, top_pages=32, cold_tier=args.cold_tier,
                     fine_pruning=not args.no_pruning)
    mw = KIVMiddleware(model, kcfg)
    mw.install()
    cache = mw.create_cache(dev)
    ids = torch.randint(0, cfg.vocab_size, (1, T), generator=torch.Generator().manual_seed(args.seed)).to(dev)
    calls = [0]

    def progress(*_):
        calls[0] += 1
        if calls[0] % 32 == 0:
            print(f"[bench] prefill chunk {calls[0]}/{(T + chunk - 1) // chunk}", file=sys.stderr, flush=True)

    hook = model.register_forward_hook(progress)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    logits = mw.chunked_prefill(ids, cache, chunk_size=chunk, prefill_hot_cap=cap)
    torch.cuda.synchronize()
    prefill_s = time.perf_counter() - t0
    hook.remove()
    cold = cache.get_cold_store(0).cold_length
    flops = model_flops(cfg, T, chunk, cap)
    print(f"[bench] prefill {T} tokens in {prefill_s:.1f}s; cold {cold} per layer", file=sys.stderr, flush=True)

    def decode(cache_, tok, n, events=None):
        with torch.no_grad():
            for i in range(n):
                if events is not None:
                    events[i][0].record()
                out = model(input_ids=tok, past_key_values=cache_, use_cache=True)
                tok = out.logits[:, -1:].argmax(-1)
                if events is not None:
                    events[i][1].record()
        return tok

    tok = logits.argmax(-1, keepdim=True)
    tok = decode(cache, tok, args.warmup)
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(args.decode_steps)]
    tok = decode(cache, tok, args.decode_steps, ev)
    torch.cuda.synchronize()
    step_ms = sorted(a.elapsed_time(b) for a, b in ev)
    print(f"[bench] decode median {step_ms[len(step_ms) // 2]:.2f} ms/step", file=sys.stderr, flush=True)
    slices = [st.fine_scan_stats() for st in cache.cold_stores.values() if st._handle]
    slices_read = [sum(x[0] for x in slices), sum(x[1] for x in slices)]  # last step, all layers
    print(f"[bench] fine-scan slices read (last step, all layers): {slices_read}", file=sys.stderr, flush=True)

    # Per-layer stages over a few more steps: the store's events bracket the
    # eviction, retrieval and attention kernels of every layer.
    lib = nat.lib()
    stores = [st for st in cache.cold_stores.values() if st._handle]
    counts, totals = (C.c_int64 * len(nat.STAGES))(), (C.c_double * len(nat.STAGES))()
    for st in stores:
        nat.check(lib.kiv_profile_enable(st._handle, 1), "kiv_profile_enable")
        nat.check(lib.kiv_profile_read(st._handle, counts, totals), "kiv_profile_read")
    prof_steps = 16
    tok = decode(cache, tok, prof_steps)
    torch.cuda.synchronize()
    stage_us = {}
    for st in stores:
        nat.check(lib.kiv_profile_read(st._handle, counts, totals), "kiv_profile_read")
        nat.check(lib.kiv_profile_enable(st._handle, 0), "kiv_profile_enable")
        for i, name in enumerate(nat.STAGES):
            if counts[i]:
                stage_us.setdefault(name, []).append(totals[i] / counts[i] * 1e3)
    stage_us = {k: round(sum(v) / len(v), 2) for k, v in stage_us.items()}
    layer_us = sum(v for k, v in stage_us.items() if k != "evict_finalize")
    union = [r["num_pages_selected"] for st in stores for r in st.telemetry_snapshot()["recent"]
             if r["kind"] == "coarse" and not r["skipped"]]

    # The same model over a plain 2048-token cache (no cold tier).
    mw.uninstall()
    plain = DynamicCache()
    with torch.no_grad():
        out = model(input_ids=ids[:, :2048], past_key_values=plain, use_cache=True, logits_to_keep=1)
    ptok = decode(plain, out.logits[:, -1:].argmax(-1), args.warmup)
    pev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(args.decode_steps)]
    decode(plain, ptok, args.decode_steps, pev)
    torch.cuda.synchronize()
    plain_ms = sorted(a.elapsed_time(b) for a, b in pev)
    step = step_ms[len(step_ms) // 2]
    pstep = plain_ms[len(plain_ms) // 2]
    L = cfg.num_hidden_layers
    line = {
        "metric": METRIC,
        "value": round(layer_us, 2),
        "unit": "us/layer/step",
        "n_gpus": 1,
        "steps": args.decode_steps,
        "warmup": args.warmup,
        "ms_per_step": round(step, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (random-init weights, uniform random token ids)",
        "config": {"workload": f"{MODEL_WORKLOAD}: Qwen2.5-1.5B-shaped decoder, {L} layers, hidden 1536, "
                               f"12/2 heads, D 128; prompt {T} tokens", "chunk_size": chunk,
                   "prefill_hot_cap": cap, "hot_budget": kcfg.hot_budget, "top_pages": kcfg.top_pages,
                   "top_p": kcfg.top_p, "cold_tier": kcfg.cold_tier, "fine_pruning": kcfg.fine_pruning},
        "value_meaning": "GPU time per layer per decode step of the tiered-cache path: eviction append, "
                         "retrieval kernels and merged attention (the store's HIP events, averaged over all "
                         "28 layers)",
        "decode_ms_per_step": {"kiv": round(step, 3), "plain_2048": round(pstep, 3),
                               "kiv_min": round(step_ms[0], 3), "kiv_max": round(step_ms[-1], 3),
                               "kiv_minus_plain_per_layer_us": round((step - pstep) * 1e3 / L, 2)},
        "per_layer_stages_us": stage_us,
        "fine_scan_slices_last_step": {"read": slices_read[0], "union": slices_read[1]},
        "union_pages": int(round(sum(union) / len(union))) if union else 0,
        "cold_tokens_per_layer": cold,
        "prefill": {"seconds": round(prefill_s, 2), "tokens_per_s": round(T / prefill_s, 1),
                    "dense_tflop": round(flops / 1e12, 1),
                    "tflops": round(flops / prefill_s / 1e12, 1),
                    "frac_of_mfma_bf16_peak": round(flops / prefill_s / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4)},
    }
    if not args.no_cpu_baseline:
        print("[bench] CPU baseline (layer 0's retrieval + attention) ...", file=sys.stderr, flush=True)
        line["cpu_baseline"], line["selection_check"] = layer_cpu_baseline(mw, cache, model, tok, kcfg, args)
    print(json.dumps(line), flush=True)


def layer_cpu_baseline(mw, cache, model, tok, kcfg, args):
    """The CPU leg on the model's own layer 0: its cold tier, hot window and
    the query it used in one more decode step (the model's union width)."""
    import torch

    from kiv_amd import ColdKVStore
    from kiv_amd.synthetic import Workload

    store = cache.get_cold_store(0)
    seen = {}
    orig = ColdKVStore._retrieve

    def spy(self, query, scaling, kiv_config, step, attend, *rest, **kw):
        if self is store:
            seen["q"] = query.detach().clone()
        return orig(self, query, scaling, kiv_config, step, attend, *rest, **kw)

    mw.install()
    mw.activate_cache(cache)
    ColdKVStore._retrieve = spy
    try:
        with torch.no_grad():
            model(input_ids=tok, past_key_values=cache, use_cache=True)
    finally:
        ColdKVStore._retrieve = orig
        mw.uninstall()
    torch.cuda.synchronize()
    layer = cache.layers[0]
    w = Workload("qwen15b_model_layer0", 12, 2, 128, torch.bfloat16, hot=layer.keys.shape[2], cold=store.cold_length,
                 top_pages=kcfg.top_pages, top_p=kcfg.top_p, segment=1)
    return cpu_baseline(w, store, kcfg, seen["q"], layer.keys.contiguous(), layer.values.contiguous(),
                        args.cpu_seconds)


def prefill_chunk_run(args):
    """The MFMA attention of one prefill chunk (kiv_prefill_attention)."""
    import torch
    import torch.nn.functional as F

    from kiv_amd.attention import prefill_attention

    dev = torch.device("cuda", 0)
    Q, T, hq, hkv, D = 4096, 8192, 12, 2, 128
    gen = torch.Generator(device=dev).manual_seed(args.seed)
    q = torch.randn(1, Q, hq, D, device=dev, dtype=torch.bfloat16, generator=gen).transpose(1, 2)
    k = torch.randn(1, hkv, T, D, device=dev, dtype=torch.bfloat16, generator=gen)
    v = torch.randn(1, hkv, T, D, device=dev, dtype=torch.bfloat16, generator=gen)
    mask = torch.ones(Q, T, dtype=torch.bool, device=dev).tril(T - Q)[None, None]
    scaling = D ** -0.5
    visible = int(mask.sum().item())
    useful_flop = 4.0 * D * hq * visible  # QK^T and PV over the visible (row, key) pairs

    def timed(fn, steps, warmup):
        for _ in range(warmup):
            fn()
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
        torch.cuda.synchronize()
        for a, b in ev:
            a.record()
            fn()
            b.record()
        torch.cuda.synchronize()
        ts = sorted(a.elapsed_time(b) * 1e3 for a, b in ev)
        return ts[len(ts) // 2], sum(ts) / len(ts)

    steps, warmup = min(args.steps, 100), min(args.warmup, 10)
    med, avg = timed(lambda: prefill_attention(q, None, None, k, v, mask, scaling), steps, warmup)
    kk = k.repeat_interleave(hq // hkv, 1)
    vv = v.repeat_interleave(hq // hkv, 1)
    sdpa_med, _ = timed(lambda: F.scaled_dot_product_attention(q, kk, vv, attn_mask=mask, scale=scaling),
                        max(steps // 4, 5), 2)
    tflops = useful_flop / (avg * 1e-6) / 1e12
    line = {
        "metric": "prefill chunk attention TFLOP/s (useful, visible pairs)",
        "value": round(tflops, 1),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(avg / 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (standard normal q, K, V)",
        "config": {"workload": f"{CHUNK_WORKLOAD}: 4096 query positions over 8192 hot keys (hot cap 4096 + "
                               "chunk 4096), 12/2 heads, D 128, boolean causal mask with offset 4096"},
        "roofline": {"kernel": "prefill_attn_kernel (+ mask_tiles_kernel)", "bound": "mfma",
                     "achieved": round(tflops, 1), "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4), "traffic": None,
                     "flop_per_launch": useful_flop, "avg_us": round(avg, 2), "median_us": round(med, 2)},
        "sdpa_same_inputs_us": round(sdpa_med, 2),
        "speedup_vs_sdpa": round(sdpa_med / med, 2),
        "cpu_baseline": None,
    }
    print(json.dumps(line), flush=True)


def trace_summary(path):
    """Durations of the kiv:: kernels of the timed layer's steps in a
    --profile-pass kernel trace.  Dispatches in start order: a reduction
    kernel opens a scrub (the other layer's step follows it), the spin kernel
    after it opens the timed step; the warm-up steps before the first scrub
    and the other layer's steps are left out."""
    import csv
    import statistics

    with open(path, newline="") as f:
        rows = sorted(csv.DictReader(f), key=lambda r: int(r["Start_Timestamp"]))
    state, durs, spans, cur = None, {}, [], None
    for r in rows:
        name = r["Kernel_Name"]
        if "reduce_kernel" in name:
            state = "other"
            if cur:
                spans.append(cur[1] - cur[0])
            cur = None
            continue
        if "spin_kernel" in name:
            state = "timed" if state == "other" else None
            continue
        if state != "timed" or "kiv::" not in name:
            continue
        short = name.split("(")[0].replace("void ", "")
        t0, t1 = int(r["Start_Timestamp"]), int(r["End_Timestamp"])
        durs.setdefault(short, []).append((t1 - t0) / 1e3)
        cur = (t0, t1) if cur is None else (cur[0], t1)
    if cur:
        spans.append(cur[1] - cur[0])
    out = [f"{'kernel':48s}{'calls':>7s}{'avg_us':>10s}{'median_us':>11s}{'min_us':>9s}{'max_us':>9s}"]
    for k, v in sorted(durs.items(), key=lambda kv: -sum(kv[1]) / len(kv[1])):
        out.append(f"{k:48s}{len(v):7d}{sum(v) / len(v):10.2f}{statistics.median(v):11.2f}{min(v):9.2f}"
                   f"{max(v):9.2f}")
    total = sum(sum(v) / len(v) for v in durs.values())
    out.append("")
    out.append(f"sum of the kernel averages: {total:.2f} us")
    if spans:
        out.append(f"step span, first kernel start to last kernel end: median {statistics.median(spans) / 1e3:.2f} us "
                   f"({len(spans)} steps)")
    print("\n".join(out))


def main():
    args = parse()
    if args.trace_summary:
        trace_summary(args.trace_summary)
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported (the tiered-cache path "
              "runs on one GPU; across GPUs it would shard by cold page range or by kv head)", file=sys.stderr)
        sys.exit(2)
    import torch

    if args.workload == MODEL_WORKLOAD:
        model_run(args)
        return
    if args.workload == CHUNK_WORKLOAD:
        prefill_chunk_run(args)
        return

    from kiv_amd import KIVConfig
    from kiv_amd.synthetic import WORKLOADS

    w = WORKLOADS[args.workload]
    dev = torch.device("cuda", 0)
    scrub = make_scrub(dev) if args.cache == "cold" else None
    if args.profile_pass:
        profile_pass(w, args, dev, scrub)
        return
    extra = 4 * (args.steps + args.warmup) + 1024
    results = {}
    tiers = [args.cold_tier] + ([] if args.no_variant else [t for t in ("host", "hbm", "split")
                                                             if t != args.cold_tier])
    for tier in tiers:
        cfg = KIVConfig(hot_budget=w.hot, top_p=w.top_p, page_size=w.page_size, top_pages=w.top_pages,
                        cold_tier=tier, reserve_tokens=w.cold + extra, fine_pruning=not args.no_pruning)
        t0 = time.perf_counter()
        store, hot_k, hot_v, q = build_cold(w, cfg, dev, args.seed)
        fill_s = time.perf_counter() - t0
        print(f"[bench] {tier}: filled {store.cold_length} cold tokens in {fill_s:.1f}s", file=sys.stderr,
              flush=True)
        scrub_l, other = layer_before(scrub, w, cfg, dev, args.seed)
        us, wall = time_steps(store, cfg, q, hot_k, hot_v, args.steps, args.warmup, w.scaling, scrub_l)
        print(f"[bench] {tier} ({args.cache} caches): {us:.1f} us/step (wall {wall:.1f})", file=sys.stderr,
              flush=True)
        stages = profile_steps(store, cfg, q, hot_k, hot_v, args.steps, w.scaling, scrub_l)
        slices = store.fine_scan_stats()  # the last step's (scanned, union) page slices
        readahead = store.readahead_bytes()  # host bytes its coarse select read ahead for the fine scan
        entry = {"us_per_step": us, "wall_us_per_step": wall, "stages": stages, "fine_scan_slices": slices,
                 "readahead_bytes": readahead}
        if scrub is not None:
            # The scrub alone before each step: the kernels' code is cold too.
            entry["code_cold_us_per_step"], _ = time_steps(store, cfg, q, hot_k, hot_v, args.steps, 0, w.scaling,
                                                           scrub)
            print(f"[bench] {tier} (scrub only, code cold too): {entry['code_cold_us_per_step']:.1f} us/step",
                  file=sys.stderr, flush=True)
        if tier == args.cold_tier and scrub is not None and not args.no_variant:
            warm_us, _ = time_steps(store, cfg, q, hot_k, hot_v, args.steps, args.warmup, w.scaling, None)
            entry["warm_us_per_step"] = warm_us
            print(f"[bench] {tier} (warm caches): {warm_us:.1f} us/step", file=sys.stderr, flush=True)
            two_us, _ = time_steps(store, cfg, q, hot_k, hot_v, args.steps, 0, w.scaling, scrub_l, fused=False)
            two_stages = profile_steps(store, cfg, q, hot_k, hot_v, args.steps, w.scaling, scrub_l, fused=False)
            entry["two_call"] = {"us_per_step": round(two_us, 2),
                                 "stages_us": {k: round(v["avg_us"], 2) for k, v in two_stages.items()}}
            print(f"[bench] {tier} (retrieve, then attention): {two_us:.1f} us/step", file=sys.stderr, flush=True)
            if tier == "host" and cfg.fine_pruning:  # the same store with the full scan
                full_us, _ = time_steps(store, replace(cfg, fine_pruning=False), q, hot_k, hot_v, args.steps, 0,
                                        w.scaling, scrub_l)
                entry["unpruned_us_per_step"] = full_us
                print(f"[bench] {tier} (fine scan not pruned): {full_us:.1f} us/step", file=sys.stderr, flush=True)
        if tier == args.cold_tier:
            entry["host_inclusive_us_per_step"] = host_inclusive(store, cfg, q, hot_k, hot_v, w.scaling)
            print(f"[bench] {tier} host-inclusive back-to-back: {entry['host_inclusive_us_per_step']:.1f} us/step",
                  file=sys.stderr, flush=True)
            if not args.no_cpu_baseline:
                print("[bench] CPU baseline ...", file=sys.stderr, flush=True)
                entry["cpu_baseline"], entry["selection_check"] = cpu_baseline(w, store, cfg, q, hot_k, hot_v,
                                                                               args.cpu_seconds)
        snap = store.telemetry_snapshot()
        unions = [r["num_pages_selected"] for r in snap["recent"] if r["kind"] == "coarse" and not r["skipped"]]
        entry["union_pages"] = int(round(sum(unions) / len(unions))) if unions else 0
        entry["traffic"] = roofline_and_links(w, store, stages, entry["union_pages"], tier, slices[0],
                                              cfg.fine_pruning, readahead)
        entry["num_pages"] = store.num_pages
        results[tier] = entry
        del store, other
        torch.cuda.synchronize()
        torch.cuda.empty_cache()

    head = results[args.cold_tier]
    links = head["traffic"]
    scan = links["coarse_scan"]
    host = {k: v for k, v in links.items() if v["host_bytes"] > 0}
    host_bytes = sum(v["host_bytes"] for v in host.values())
    host_us = sum(v["avg_us"] for v in host.values())
    ceil = probes(dev, scan["bytes"], links["fine_scan"]["bytes"], scrub is not None)
    print(f"[bench] probes: {ceil}", file=sys.stderr, flush=True)
    # The roofline entry is the step's dominant kernel (the longest stage):
    # on the host tier the fine scan, bound by the host link; on the HBM
    # tiers an HBM-bound kernel.
    dom_name, dom = max(links.items(), key=lambda kv: kv[1]["avg_us"])
    on_host = dom["from"] == "host"
    peak = HOST_LINK_PEAK_GBS if on_host else HBM_PEAK_GBS
    pmc = load_pmc(w.name, args.cold_tier)
    dom_pmc = pmc.get(dom_name)
    roofline = {
        "kernel": dom_name, "bound": "host_link" if on_host else "hbm", "achieved": round(dom["GB_s"], 2),
        "peak": peak, "unit": "GB/s", "frac": round(dom["GB_s"] / peak, 4),
        "traffic": dom_pmc["traffic"] if dom_pmc else None,
        "traffic_by_memory": dom_pmc, "bytes_per_launch": dom["bytes"], "avg_us": round(dom["avg_us"], 2),
        "achievable": ({"same_size_read": ceil["host_link_fine_size"], "read_256MiB": ceil["host_link_256MiB"]}
                       if on_host else {"stream_2GiB": ceil["hbm_stream_2GiB"]}),
    }
    # The summary scan, the HBM-bound kernel the target names.
    summary_scan = {
        "kernel": "coarse_scan", "bound": "hbm", "achieved": round(scan["GB_s"], 1), "peak": HBM_PEAK_GBS,
        "unit": "GB/s", "frac": round(scan["GB_s"] / HBM_PEAK_GBS, 4),
        "frac_of_stream_probe": round(scan["GB_s"] / ceil["hbm_stream_2GiB"], 4),
        "stream_probe_2GiB": ceil["hbm_stream_2GiB"],
        "latency_floor": {"what": "a cold read of the same bytes with the same grid (median of 50 single reads; "
                                  "min, quartiles, max)", "GB_s": ceil["hbm_summary_size"],
                          "spread": ceil["hbm_summary_size_spread"],
                          "scan_over_floor": round(scan["GB_s"] / ceil["hbm_summary_size"], 4)},
        "traffic": pmc["coarse_scan"]["traffic"] if "coarse_scan" in pmc else None,
        "traffic_by_memory": pmc.get("coarse_scan"), "bytes_per_launch": scan["bytes"],
        "avg_us": round(scan["avg_us"], 2),
    }
    host_link = None
    if host:
        gbs = host_bytes / (host_us * 1e-6) / 1e9
        # Host-link bytes measured by the counters (reads and writes of host
        # memory by the step's kernels, from the committed summary).
        measured = sum(v["host_read"] + v["host_write"] for v in pmc.values()) if pmc else None
        host_link = {"kernels": sorted(host), "achieved": round(gbs, 2), "peak": HOST_LINK_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HOST_LINK_PEAK_GBS, 4), "bytes_per_step": host_bytes,
                     "bytes_per_step_measured": measured,
                     "achievable": {"same_size_read": ceil["host_link_fine_size"],
                                    "read_256MiB": ceil["host_link_256MiB"]},
                     "frac_of_achievable": round(gbs / ceil["host_link_fine_size"], 4)}
    # A page completes every page_size steps; its finalize (summary, radius,
    # rows to the arena) is spread over them in the headline.
    fin = head["stages"].get("evict_finalize")
    fin_us = fin["avg_us"] / w.page_size if fin else 0.0
    value = head["us_per_step"] + fin_us
    variants = {t: {"us_per_step": round(r["us_per_step"], 2), "union_pages": r["union_pages"],
                    "fine_scan_slices": list(r["fine_scan_slices"]),
                    "stages_us": {k: round(v["avg_us"], 2) for k, v in r["stages"].items()}}
                for t, r in results.items() if t != args.cold_tier}
    for t, r in results.items():
        if t != args.cold_tier and "code_cold_us_per_step" in r:
            variants[t]["code_cold_us_per_step"] = round(r["code_cold_us_per_step"], 2)
    if "warm_us_per_step" in head:
        variants["warm_caches"] = {"us_per_step": round(head["warm_us_per_step"], 2)}
    if "two_call" in head:
        variants["two_call"] = head["two_call"]
    if "unpruned_us_per_step" in head:
        variants["fine_scan_not_pruned"] = {"us_per_step": round(head["unpruned_us_per_step"], 2)}
    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "us/layer/step",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(value / 1e3, 5),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if w.dtype == torch.bfloat16 else "f16",
        "data": "synthetic (seeded clustered-K / Gaussian-V generator, drawn on the GPU)",
        "config": {"workload": f"{w.name}: one decode layer, Hq={w.num_q_heads} Hkv={w.num_kv_heads} "
                               f"D={w.head_dim}, hot {w.hot}, cold {w.cold}", "batch": 1,
                   "top_pages": w.top_pages, "top_p": w.top_p, "page_size": w.page_size,
                   "cold_tier": args.cold_tier, "fine_pruning": not args.no_pruning, "caches": args.cache},
        "value_meaning": ("GPU time of one layer's decode step as a model runs it: a cache scrub (no data "
                          "of this layer in L2 or the MALL), then another layer's step of the same shape "
                          "(its own store: the kernels' code is resident, as between the layers of a "
                          "model), then fence-free HIP events around this layer's step; median over the "
                          "timed steps, plus the page-end finalize (measured in the same run) spread over "
                          "the page's steps"
                          if scrub is not None else
                          "GPU time of one layer's decode step: HIP events around the timed steps run "
                          "back to back (warm caches), mean, plus the page-end finalize spread over the "
                          "page's steps"),
        "us_per_step_timed": round(head["us_per_step"], 2),
        "code_cold_us_per_step": (round(head["code_cold_us_per_step"] + fin_us, 2)
                                  if "code_cold_us_per_step" in head else None),
        "event_pair_overhead_us": (round(event_pair_us(dev, scrub), 2) if scrub is not None else None),
        "evict_finalize_amortized_us": round(fin_us, 3),
        "host_inclusive_us_per_step": round(head.get("host_inclusive_us_per_step", float("nan")), 2),
        "roofline": roofline,
        "summary_scan": summary_scan,
        "host_link": host_link,
        "union_pages": head["union_pages"],
        "fine_scan_slices": {"read": head["fine_scan_slices"][0], "union": head["fine_scan_slices"][1]},
        "stages_us": {k: round(v["avg_us"], 2) for k, v in head["stages"].items()},
        "wall_us_per_step": round(head["wall_us_per_step"], 2),
        "probes_GB_s": ceil,
        "variants": variants,
    }
    if "cpu_baseline" in head:
        line["cpu_baseline"] = head["cpu_baseline"]
        line["selection_check"] = head["selection_check"]
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
