"""Decode µs/layer of the tiered-cache hot path on one MI355X.

    python bench.py [--steps K] [--warmup W] [--workload qwen7b_1m] [--cold-tier host|hbm]

One step = one global layer's decode step for one new token: evict the
oldest hot row to the cold tier, coarse-to-fine retrieval over the cold
tier (page scan, per-head top pages, union, fine scores, top-P, K/V gather)
and the merged softmax over [retrieved ; hot].  Inputs are resident before
the timed region: the cold tier is filled (1,048,576 tokens for the default
workload) and the query / hot window live in HBM.

The JSON line carries the headline µs/layer/step, a second timed pass with
HIP events bracketing every kernel on its launch stream (per-stage average
durations, the roofline of the dominant HBM kernel and the host-link
traffic), the union size, the same step with the cold rows in HBM, and the
reference's op sequence timed on the host CPU (the oracle, as a baseline).
"""

from __future__ import annotations

import argparse
import ctypes as C
import json
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
    ap.add_argument("--cold-tier", default="host", choices=("host", "hbm"))
    ap.add_argument("--no-variant", action="store_true", help="skip the other cold tier")
    ap.add_argument("--cpu-seconds", type=float, default=15.0, help="CPU baseline sample budget")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--seed", type=int, default=0)
    return ap.parse_args()


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


def run_steps(store, cfg, q, hot_k, hot_v, n, scaling, attn_events=None):
    """n decode steps; the evicted row cycles through the hot window's rows."""
    from kiv_amd.attention import decode_attention

    T = hot_k.shape[2]
    for i in range(n):
        j = (store.cold_length + i) % T
        store.evict_from_hot(hot_k[:, :, j:j + 1], hot_v[:, :, j:j + 1])
        k_out, v_out = store.retrieve_top_kv(q, scaling, cfg)
        if attn_events is not None:
            attn_events[i][0].record()
        decode_attention(q, k_out, v_out, hot_k, hot_v, None, scaling)
        if attn_events is not None:
            attn_events[i][1].record()


def time_steps(store, cfg, q, hot_k, hot_v, steps, warmup, scaling):
    import torch

    run_steps(store, cfg, q, hot_k, hot_v, warmup, scaling)
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record()
    run_steps(store, cfg, q, hot_k, hot_v, steps, scaling)
    ev1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    return ev0.elapsed_time(ev1) / steps, wall / steps * 1e3


def profile_steps(store, cfg, q, hot_k, hot_v, steps, scaling):
    """Per-stage average launch durations (ms) from HIP events on the launch stream."""
    import torch

    from kiv_amd import _native as nat

    lib = nat.lib()
    n = min(steps, 256)
    nat.check(lib.kiv_profile_enable(store._handle, 1), "kiv_profile_enable")
    counts, totals = (C.c_int64 * 7)(), (C.c_double * 7)()
    nat.check(lib.kiv_profile_read(store._handle, counts, totals), "kiv_profile_read")  # clear
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n)]
    run_steps(store, cfg, q, hot_k, hot_v, n, scaling, attn_events=ev)
    torch.cuda.synchronize()
    nat.check(lib.kiv_profile_read(store._handle, counts, totals), "kiv_profile_read")
    nat.check(lib.kiv_profile_enable(store._handle, 0), "kiv_profile_enable")
    stages = {}
    for i, name in enumerate(nat.STAGES):
        if counts[i]:
            stages[name] = {"launches": int(counts[i]), "avg_us": totals[i] / counts[i] * 1e3}
    att = [a.elapsed_time(b) for a, b in ev]
    stages["attention"] = {"launches": n, "avg_us": sum(att) / n * 1e3}
    return stages


def roofline_and_links(w, store, stages, union_pages, tier):
    """Algorithmic bytes per launch / measured duration for every stage."""
    b = 2 if w.dtype.itemsize == 2 else 4
    row = w.num_kv_heads * w.head_dim * b          # one token, all kv heads
    N = store.num_pages
    P = min(w.top_p, store.cold_length)
    p = store.cold_length - N * w.page_size
    cand = union_pages * w.page_size + p
    rows = w.num_q_heads
    traffic = {
        # (bytes per launch, memory it streams from)
        "coarse_scan": (N * row, "hbm"),
        "coarse_select": (rows * N * 4, "hbm"),
        "fine_scan": (union_pages * w.page_size * row, tier),
        "fine_select": (cand * 4, "hbm"),
        "gather": (2 * P * row, tier),
        "attention": (2 * (P + w.hot) * row, "hbm"),
    }
    out = {}
    for name, (nbytes, where) in traffic.items():
        if name in stages:
            us = stages[name]["avg_us"]
            out[name] = {"bytes": nbytes, "from": where, "avg_us": us, "GB_s": nbytes / (us * 1e-6) / 1e9}
    return out


def cpu_baseline(w, seed, budget_s):
    """The reference's op sequence (oracle.torch_ref) on host cores, NS-sized store."""
    import torch

    from kiv_amd.synthetic import generate_streaming
    from oracle.torch_ref import OracleColdStore, decode_step

    store = OracleColdStore(w.page_size, w.groups)
    hot_k = hot_v = q = None
    for item in generate_streaming(w, seed, "cpu", chunk=65536):
        if item[0] == "cold":
            store.evict(item[1], item[2])
        elif item[0] == "hot":
            hot_k, hot_v = item[1], item[2]
        else:
            q = item[1]
    store.flat()  # the reference materialises once before scoring (kiv/cold_store.py:122-136)
    decode_step(store, q, hot_k, hot_v, None, w.scaling, w.top_p, w.top_pages)  # warm-up
    times = []
    t_end = time.perf_counter() + budget_s
    while time.perf_counter() < t_end or len(times) < 3:
        t0 = time.perf_counter()
        decode_step(store, q, hot_k, hot_v, None, w.scaling, w.top_p, w.top_pages)
        times.append(time.perf_counter() - t0)
    times.sort()
    med = times[len(times) // 2]
    return {"value": med * 1e6, "unit": "us/layer/step", "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"{len(times)} retrieve+attention calls (median) on the {w.name} store "
                      f"({w.cold} cold tokens, CPU-generated, same generator), torch CPU ops of the "
                      "reference sequence in bf16"}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported (the tiered-cache path "
              "runs per GPU; see DESIGN.md for how it would shard)", file=sys.stderr)
        sys.exit(2)
    import torch

    from kiv_amd import KIVConfig
    from kiv_amd.synthetic import WORKLOADS

    w = WORKLOADS[args.workload]
    dev = torch.device("cuda", 0)
    extra = args.steps + args.warmup + 512
    results = {}
    tiers = [args.cold_tier] + ([] if args.no_variant else [t for t in ("host", "hbm") if t != args.cold_tier])
    for tier in tiers:
        cfg = KIVConfig(hot_budget=w.hot, top_p=w.top_p, page_size=w.page_size, top_pages=w.top_pages,
                        cold_tier=tier, reserve_tokens=w.cold + extra)
        t0 = time.perf_counter()
        store, hot_k, hot_v, q = build_cold(w, cfg, dev, args.seed)
        fill_s = time.perf_counter() - t0
        print(f"[bench] {tier}: filled {store.cold_length} cold tokens in {fill_s:.1f}s", file=sys.stderr,
              flush=True)
        ms_gpu, ms_wall = time_steps(store, cfg, q, hot_k, hot_v, args.steps, args.warmup, w.scaling)
        print(f"[bench] {tier}: {ms_gpu * 1e3:.1f} us/step (wall {ms_wall * 1e3:.1f})", file=sys.stderr, flush=True)
        stages = profile_steps(store, cfg, q, hot_k, hot_v, args.steps, w.scaling)
        snap = store.telemetry_snapshot()
        unions = [r["num_pages_selected"] for r in snap["recent"] if r["kind"] == "coarse" and not r["skipped"]]
        U = int(round(sum(unions) / len(unions))) if unions else 0
        links = roofline_and_links(w, store, stages, U, tier)
        results[tier] = {"us_per_step": ms_gpu * 1e3, "wall_us_per_step": ms_wall * 1e3, "stages": stages,
                         "traffic": links, "union_pages": U, "cold_tokens": store.cold_length}
        del store
        torch.cuda.synchronize()
        torch.cuda.empty_cache()

    head = results[args.cold_tier]
    links = head["traffic"]
    hbm_kernels = {k: v for k, v in links.items() if v["from"] == "hbm"}
    dominant = max(hbm_kernels, key=lambda k: hbm_kernels[k]["avg_us"])
    dom = hbm_kernels[dominant]
    roofline = {"kernel": dominant, "bound": "hbm", "achieved": round(dom["GB_s"], 1), "peak": HBM_PEAK_GBS,
                "unit": "GB/s", "frac": round(dom["GB_s"] / HBM_PEAK_GBS, 4), "traffic": None,
                "bytes_per_launch": dom["bytes"], "avg_us": round(dom["avg_us"], 2)}
    scan = links["coarse_scan"]
    host = {k: v for k, v in links.items() if v["from"] == "host"}
    host_bytes = sum(v["bytes"] for v in host.values())
    host_us = sum(v["avg_us"] for v in host.values())
    line = {
        "metric": METRIC,
        "value": round(head["us_per_step"], 2),
        "unit": "us/layer/step",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["us_per_step"] / 1e3, 5),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if w.dtype == torch.bfloat16 else "f16",
        "data": "synthetic (seeded clustered-K / Gaussian-V generator, drawn on the GPU)",
        "config": {"workload": f"{w.name}: one decode layer, Hq={w.num_q_heads} Hkv={w.num_kv_heads} "
                               f"D={w.head_dim}, hot {w.hot}, cold {w.cold}", "batch": 1,
                   "top_pages": w.top_pages, "top_p": w.top_p, "page_size": w.page_size,
                   "cold_tier": args.cold_tier},
        "roofline": roofline,
        "summary_scan": {"achieved": round(scan["GB_s"], 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(scan["GB_s"] / HBM_PEAK_GBS, 4), "avg_us": round(scan["avg_us"], 2),
                         "bytes_per_launch": scan["bytes"]},
        "host_link": ({"achieved": round(host_bytes / (host_us * 1e-6) / 1e9, 2), "peak": HOST_LINK_PEAK_GBS,
                       "unit": "GB/s", "frac": round(host_bytes / (host_us * 1e-6) / 1e9 / HOST_LINK_PEAK_GBS, 4),
                       "bytes_per_step": host_bytes, "kernels": sorted(host)} if host else None),
        "union_pages": head["union_pages"],
        "stages_us": {k: round(v["avg_us"], 2) for k, v in head["stages"].items()},
        "wall_us_per_step": round(head["wall_us_per_step"], 2),
        "variants": {t: {"us_per_step": round(r["us_per_step"], 2),
                         "stages_us": {k: round(v["avg_us"], 2) for k, v in r["stages"].items()}}
                     for t, r in results.items() if t != args.cold_tier},
    }
    if not args.no_cpu_baseline:
        print("[bench] CPU baseline ...", file=sys.stderr, flush=True)
        line["cpu_baseline"] = cpu_baseline(w, args.seed, args.cpu_seconds)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
