#!/usr/bin/env python3
"""Benchmark of the MI355X PaxBlock64 bitplane scan (prints one JSON line).

A step is one pass of the hot path over one batch of queries: the batched
query-plan kernel on the resident queries, then every scan pass + top-K
selection, all enqueued on a context's stream with the index already in
HBM.  The timed steps go round `--streams` contexts (default 3) that scan the
one index, each with its own plans and results, so the latency-bound launches
of one step (plan, sampling, selection) overlap another step's on the GPU:
`ms_per_step` and `value` are that throughput (K steps between
synchronisations of every stream), `single_stream_ms_per_step` the same K
steps on one context, one batch in flight at a time (the latency of a step).
The default run measures the two workloads BASELINE's metric is quoted
on: the headline is configs[3] (8.8M x 768 clustered, batch 64, K_cand 256,
the north-star target); configs[1] (1M x 768, batch 1, K_cand 256) is
reported beside it under "batch1", and one GPU's share of configs[3]
sharded over 8 GPUs by block range (the first 1.1M documents, the same 64
queries) under "shard_1of8".  --config N runs BASELINE configs[N-1] alone as
the headline.

`roofline` uses the dominant kernel's durations from HIP events that each
dispatch records at its own start and end (hipExtLaunchKernelGGL), from a
second run of the same steps after the timed one (events stay out of the
timed region), on the library's stream; `traffic` is the committed rocprofv3
FETCH_SIZE + WRITE_SIZE reading for the same workload.  Batches under 8 run
the one-query k_scan, HBM-bound: 4096 B per block scanned.  Batches of 8+
run the MFMA-bounded scan, whose final pass (k_scan_mma over every block)
dominates: 2 x 261 f16 MACs per (query, vector) pair with full tiles, 2 x 80
in a bounded pass (no S1 / S4 bits, their bound columns instead), and 4096 B
per block; the roof that binds is the larger floor (MACs at the dense f16
MFMA peak or bytes at the HBM peak), and both fractions are reported.  `cold_cache` repeats the
profiled steps with a 1 GiB read before each (the L2s and the 256 MB
Infinity Cache evicted).  `reruns_per_step` counts the queries whose final
floor needed a re-run (safe: done on the device inside the step, by two
launches every sampled scan enqueues) or whose list overflowed (dense: done
at fetch time, outside the timed step, so a non-zero count would mean the
timed step left work out).
Before each workload's warmup, `clock_settle` reads a 1 GiB device buffer
(mrl_ctx_evict_caches, the library's k_read_sweep) for about 200 ms: the
corpus is generated on the host for seconds with the GPU idle, and after
such an idle the first steps run up to ~15 % slower until the GPU has seen
some 100 ms of memory traffic (measured after a 13 s idle, config 4 over
three streams: 0.341 ms per step with no settle, 0.311 after 30 ms of
reads, 0.298 after 165 ms; VALU-bound work did not help), which the few
warmup steps of a short run do not give.  It runs no step and leaves
nothing the steps use (it evicts the caches instead).
`cpu_baseline` times the C restatement of the reference's scan_blocks
(oracle/, Rayon-equivalent sharding on host threads) on query 0 of the same
index, on the host's cores and on one thread; the batch figure is the time
of the same batch pass with queries one after another (the reference has no
batch API).  The same run checks the GPU top-K of query 0 (`parity_query0`).
`host_boundary` is the PCIe-inclusive rate of the synchronous host-buffer
calls.  `rerank` reranks every query's device-resident shortlist at fp32 /
fp16 / int8 after the scan; `encode` runs the GPU encoder over the
workload's rows (1M-vector workloads only).
"""
import argparse
import ctypes as C
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "mrl-index-rust-vector_amd"))

HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFS = 2500.0  # dense f16 MFMA, MI355X
# MACs per (query, vector) pair of the MFMA bound: 64 prefix dims, 128 S1
# bits, 64 S4 bits and the 5 meta / error columns of the last K-step; a
# bounded final pass (profile flag MRL_KT_S4_BOUNDED) runs no S1 or S4 bits,
# and 3 S1 and 8 S4 bound columns instead
MMA_MACS_PER_PAIR = 64 + 128 + 64 + 5
MMA_MACS_PER_PAIR_BOUNDED = 64 + 5 + 3 + 8
KT_S4_BOUNDED = 1
EVICT_BYTES = 1 << 30  # cold-cache runs read this much between steps
SETTLE_MS = 200.0  # clock settle before each workload's warmup (device reads, no steps)
KIND_NAMES = {0: "plan", 1: "scan", 2: "select", 3: "thresh", 6: "finish", 7: "mma_prep", 8: "exact", 9: "bounds",
              10: "plan+scan", 11: "plan+mma_prep"}


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def host_threads():
    """Threads for host work: the box's CPU share (OMP_NUM_THREADS there) or the core count."""
    n = os.cpu_count() or 1
    share = os.environ.get("OMP_NUM_THREADS")
    if share and share.isdigit() and int(share) > 0:
        n = min(n, int(share))
    return max(1, min(n, 64))


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", type=int, default=0, choices=[0, 1, 2, 3, 4, 5],
                    help="0 (default): configs 4 and 2 (BASELINE configs[3] and [1]); N: that config alone")
    ap.add_argument("--cpu-seconds", type=float, default=8.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--streams", type=int, default=3,
                    help="contexts (one stream each) sharing the index; the timed steps go round them")
    ap.add_argument("--no-cold", action="store_true", help="skip the cold-cache runs")
    ap.add_argument("--no-rerank", action="store_true", help="skip the post-scan rerank and encode legs")
    ap.add_argument("--layout", choices=["standard", "clustered"], default="standard",
                    help="with --config N: the documents in row order (standard) or grouped by centroid (clustered)")
    ap.add_argument("--stratum4-weight", type=float, default=None,
                    help="with --config N: EngineConfig.stratum4_weight (default: the reference's 0.20)")
    ap.add_argument("--no-cluster-layout", action="store_true",
                    help="default run: skip config 4 in the cluster-grouped layout")
    ap.add_argument("--rerank-reps", type=int, default=100)
    ap.add_argument("--settle-ms", type=float, default=SETTLE_MS,
                    help="device reads before each workload's warmup, in ms (0: none)")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run the library's fill and read-sweep kernels over MIB MiB (PMC byte-counter calibration) and exit")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one GPU; runs across several GPUs are not part of it "
              "(the scan would shard by contiguous block range, one top-K merge per query).", file=sys.stderr)
        sys.exit(2)
    if args.copy_calibration:
        copy_calibration(args.copy_calibration)
        return

    import mrl_index_amd as m
    n_threads = host_threads()
    dev = m.default_device()
    head_id = args.config or 4
    out = run_workload(head_id, args, m, dev, n_threads, legs=not args.no_rerank and m_rows_fit(head_id),
                       layout=args.layout if args.config else "standard")
    if args.config == 0 and not args.no_cluster_layout:
        # the same documents and queries grouped by centroid: block skipping
        out["cluster_layout"] = run_workload(4, args, m, dev, n_threads, legs=False, layout="clustered",
                                             cpu_seconds=0.5)
    if args.config == 0:
        # one GPU's share of config 4 sharded over 8 GPUs by block range
        out["shard_1of8"] = run_workload(4, args, m, dev, n_threads, legs=False, shard=8, cpu=False)
        out["batch1"] = run_workload(2, args, m, dev, n_threads, legs=not args.no_rerank)
        for k in ("rerank", "encode", "host_boundary"):
            if k in out["batch1"]:
                out[k] = out["batch1"].pop(k)
    print(json.dumps(out), flush=True)


def m_rows_fit(cfg_id):
    from mrl_index_amd import synth
    return synth.CONFIGS[cfg_id].n_docs <= 2_000_000


def kernel_groups(L, _lib, dev, cap):
    """Collects the recorded launches: {(kind, pass): {"ms": [...], "blocks": [...], "flags": [...]}}."""
    kt = (_lib.KernelTimeC * cap)()
    nrec = C.c_uint32()
    _lib.check(L.mrl_ctx_profile_collect(dev.handle, kt, cap, C.byref(nrec)))
    groups = {}
    for i in range(min(nrec.value, cap)):
        r = kt[i]
        g = groups.setdefault((KIND_NAMES.get(r.kind, str(r.kind)), r.pass_), {"ms": [], "blocks": [], "flags": []})
        g["ms"].append(r.ms)
        g["blocks"].append(r.n_blocks)
        g["flags"].append(r.flags)
    return groups


def roofline_of(groups, nq, prof_steps, w, cold=False, scanned=None):
    """The dominant kernel's roofline from the recorded launches.  scanned:
    the (block, query) pairs the MFMA final pass actually scored per step (its
    ScanStats.blocks counter), which a cluster-grouped index's block lists make
    fewer than blocks x queries; by default every block for every query."""
    import numpy as np
    mma = any(kind in ("mma_prep", "plan+mma_prep") for kind, _ in groups)
    src = {}
    if not mma:
        # One-query path: the dominant kernel is k_scan (every pass launches
        # it; a sampling pass that also builds the plan is its own
        # instantiation, "plan+scan"); its roofline is taken over all of its
        # launches, as rocprofv3's per-kernel average is: algorithmic bytes
        # per launch = 4096 B x blocks scanned by that launch.
        # (pass -1: the safe-floor re-run, which ends at once unless a query
        # was flagged, is left out)
        scan_ms = [ms for (kind, p), g in groups.items() if kind == "scan" and p >= 0 for ms in g["ms"]]
        scan_blk = [b for (kind, p), g in groups.items() if kind == "scan" and p >= 0 for b in g["blocks"]]
        avg_ms = float(np.mean(scan_ms))
        bytes_per_launch = 4096.0 * float(np.mean(scan_blk))
        achieved = bytes_per_launch / (avg_ms / 1000.0) / 1e9
        traffic = None if cold else committed_traffic("k_scan", w.name)
        r = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
             "frac": round(achieved / HBM_PEAK_GBS, 4),
             "traffic": traffic["bytes_per_launch"] if traffic else None,
             "kernel": "k_scan", "launches_per_step": len(scan_ms) / prof_steps,
             "kernel_avg_ms": round(avg_ms, 5), "algorithmic_bytes_per_launch": bytes_per_launch}
        final = max(p for kind, p in groups if kind == "scan")
        g = groups[("scan", final)]
        fb = 4096.0 * float(np.mean(g["blocks"]))
        fm = float(np.mean(g["ms"]))
        r["final_pass"] = {"avg_ms": round(fm, 5), "achieved_gb_s": round(fb / (fm / 1000.0) / 1e9, 1),
                           "frac": round(fb / (fm / 1000.0) / 1e9 / HBM_PEAK_GBS, 4)}
    else:
        # MFMA path: the final pass (the highest pass index) scans every
        # block once for every query of the batch.
        final = max(p for kind, p in groups if kind == "scan")
        g = groups[("scan", final)]
        avg_ms = float(np.mean(g["ms"]))
        block_queries = float(scanned) if scanned is not None else float(np.mean(g["blocks"])) * nq
        pairs = 64.0 * block_queries
        # the MACs of the pass that ran: the S4-bounded pass needs fewer per pair
        s4_bounded = float(np.mean([(f & KT_S4_BOUNDED) != 0 for f in g["flags"]]))
        macs = s4_bounded * MMA_MACS_PER_PAIR_BOUNDED + (1.0 - s4_bounded) * MMA_MACS_PER_PAIR
        flops = 2.0 * macs * pairs
        tflops = flops / (avg_ms / 1000.0) / 1e12
        # the blocks one query scanned (a block shared by the batch is read once)
        bytes_per_launch = 4096.0 * block_queries / nq
        hbm = bytes_per_launch / (avg_ms / 1000.0) / 1e9
        # the roof that binds is the larger floor: the MACs at the dense f16 MFMA peak, or the bytes at
        # the HBM peak (a bounded final pass runs so few MACs that its bytes bind)
        hbm_bound = bytes_per_launch / (HBM_PEAK_GBS * 1e9) >= flops / (MFMA_F16_PEAK_TFS * 1e12)
        # (the committed counters cover the standard layout; a block-listed pass reads other bytes)
        traffic = None if cold or scanned is not None else committed_traffic("k_scan_mma", w.name)
        r = {"bound": "hbm" if hbm_bound else "mfma",
             "achieved": round(hbm if hbm_bound else tflops, 1),
             "peak": HBM_PEAK_GBS if hbm_bound else MFMA_F16_PEAK_TFS,
             "unit": "GB/s" if hbm_bound else "TFLOP/s",
             "frac": round(hbm / HBM_PEAK_GBS if hbm_bound else tflops / MFMA_F16_PEAK_TFS, 4),
             "traffic": traffic["bytes_per_launch"] if traffic else None,
             "kernel": "k_scan_mma (final pass)", "launches_per_step": len(g["ms"]) / prof_steps,
             "kernel_avg_ms": round(avg_ms, 5), "algorithmic_flops_per_launch": flops,
             "macs_per_pair": round(macs, 2), "s4_bounded_launches": round(s4_bounded, 4),
             "algorithmic_bytes_per_launch": bytes_per_launch,
             "mfma_achieved_tflops": round(tflops, 1), "mfma_frac": round(tflops / MFMA_F16_PEAK_TFS, 4),
             "hbm_achieved_gb_s": round(hbm, 1), "hbm_frac": round(hbm / HBM_PEAK_GBS, 4)}
    if traffic:
        r["traffic_source"] = traffic["source"]
    return r


def kernels_of(groups):
    import numpy as np
    return {f"{kind}[{p}]": {"avg_ms": round(float(np.mean(g["ms"])), 5), "launches": len(g["ms"]),
                             "avg_blocks": float(np.mean(g["blocks"]))}
            for (kind, p), g in sorted(groups.items())}


def run_workload(cfg_id, args, m, dev, n_threads, legs, layout="standard", cpu_seconds=None, shard=1, cpu=True):
    """One workload as a bench record.  layout "clustered": the documents of a
    clustered corpus grouped by centroid (mrl_synth_encode_clustered), so the
    index carries block bounds and the final passes skip blocks no query of
    the batch can reach; the queries are the same.  shard > 1: one GPU's
    share of the index sharded by contiguous block range, the first
    1/shard of the documents, scanned for the workload's full query batch."""
    import numpy as np
    from mrl_index_amd import _lib, synth
    L = _lib.lib
    wq = synth.CONFIGS[cfg_id]
    w = wq.scaled(wq.n_docs // shard) if shard > 1 else wq
    t0 = time.time()
    fit = synth.eden_fit(w)
    log(f"config {cfg_id} ({layout}): generating + encoding {w.name}: {w.n_docs} x {w.dims} on {n_threads} threads")
    if layout == "clustered":
        if not w.n_centroids:
            raise SystemExit(f"config {cfg_id} has no clusters")
        blocks, _ = synth.encode_clustered(w, fit, n_threads)
    else:
        blocks = synth.encode(w, fit, n_threads)
    queries, _ = synth.queries(wq)
    log(f"corpus ready in {time.time() - t0:.1f}s ({blocks.nbytes / 1e6:.1f} MB of codes)")

    ix = m.DeviceIndex.upload(blocks, dev)
    plan = m.QueryPlan.from_query_codec(queries, w.dims, w.prefix_codec, m.MidCodec.RABITQ, fit, None, dev)
    cfg = m.ScanConfig(shortlist_cand=w.k, strata_depth=w.strata, exhaustive=w.exhaustive)
    if args.stratum4_weight is not None:
        cfg.stratum4_weight = args.stratum4_weight
    ccfg = cfg.to_c()
    tr = _lib.TimeRangeC(0, 0, 0, 0)
    nq = w.n_queries
    res = C.c_void_p()
    _lib.check(L.mrl_results_create(dev.handle, nq, w.k, C.byref(res)))
    # Further contexts (one stream each) scanning the same index with their
    # own plans and results: the timed steps go round them, so a step's
    # latency-bound kernels overlap the next step's on the GPU.
    lanes = [(dev, plan, res)]
    for _ in range(1, max(1, args.streams)):
        d = m.Device(dev.device)
        p = m.QueryPlan.from_query_codec(queries, w.dims, w.prefix_codec, m.MidCodec.RABITQ, fit, None, d)
        r = C.c_void_p()
        _lib.check(L.mrl_results_create(d.handle, nq, w.k, C.byref(r)))
        lanes.append((d, p, r))

    def lane_step(i):
        d, p, r = lanes[i]
        _lib.check(L.mrl_plans_rebuild(d.handle, p.handle))
        _lib.check(L.mrl_scan_async(d.handle, ix.handle, p.handle, C.byref(ccfg), C.byref(tr), r))

    def step():
        lane_step(0)

    ids = np.zeros((nq, w.k), dtype=np.uint64)
    scores = np.zeros((nq, w.k), dtype=np.float32)
    counts = np.zeros(nq, dtype=np.uint32)
    st = _lib.ScanStatsC()

    def fetch(with_out=True):
        _lib.check(L.mrl_results_fetch(dev.handle, res, _lib.u64ptr(ids) if with_out else None,
                                       _lib.fptr(scores) if with_out else None,
                                       _lib.u32ptr(counts) if with_out else None, C.byref(st)))

    def lane_stats(i):
        s_i = _lib.ScanStatsC()
        _lib.check(L.mrl_results_fetch(lanes[i][0].handle, lanes[i][2], None, None, None, C.byref(s_i)))
        return {f: getattr(s_i, f) for f, _ in _lib.ScanStatsC._fields_}

    settle = settle_clocks(L, _lib, dev, args.settle_ms)
    log(f"clock settle: {settle['reads']} reads of {EVICT_BYTES >> 20} MiB in {settle['ms']} ms")
    log(f"warmup {args.warmup} steps on each of {len(lanes)} streams")
    for _ in range(args.warmup):
        for i in range(len(lanes)):
            lane_step(i)
    fetch()
    for i in range(1, len(lanes)):
        lane_stats(i)

    log(f"timed {args.steps} steps over {len(lanes)} streams")
    for d, _, _ in lanes:
        d.synchronize()
    t_start = time.perf_counter()
    for k in range(args.steps):
        lane_step(k % len(lanes))
    for d, _, _ in lanes:
        d.synchronize()
    t_end = time.perf_counter()
    fetch()
    timed_stats = {f: getattr(st, f) for f, _ in _lib.ScanStatsC._fields_}
    for i in range(1, len(lanes)):
        for f, v in lane_stats(i).items():
            timed_stats[f] += v

    # Latency: the same steps on one stream, one batch in flight at a time.
    log(f"timed {args.steps} steps on one stream")
    dev.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    dev.synchronize()
    single_ms = (time.perf_counter() - t0) * 1000.0 / args.steps
    fetch(False)

    # Per-kernel durations: the same steps again with dispatch-recorded events
    # (kept out of the timed region above).
    prof_steps = min(args.steps, 100)
    log(f"profiled {prof_steps} steps")
    _lib.check(L.mrl_ctx_set_profiling(dev.handle, 1))
    for _ in range(prof_steps):
        step()
    dev.synchronize()
    _lib.check(L.mrl_ctx_set_profiling(dev.handle, 0))
    groups = kernel_groups(L, _lib, dev, 64 * prof_steps + 64)
    fetch(False)

    ms_step = (t_end - t_start) * 1000.0 / args.steps
    vec_per_s = w.n_docs / (ms_step / 1000.0)
    step_bytes = 4096.0 * blocks.shape[0] + 4 * w.dims * nq + 12 * w.k * nq
    out = {
        "metric": "scan Mvec/s (vectors scored per second per query batch pass)",
        "value": round(vec_per_s / 1e6, 2),
        "unit": "Mvec/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "streams": len(lanes),
        "single_stream_ms_per_step": round(single_ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": (wq.name + (f"-shard-1of{shard}" if shard > 1 else "") +
                                ("-cluster-grouped" if layout == "clustered" else "")),
                   "baseline_config": cfg_id, "layout": layout, "n_vectors": w.n_docs, "dims": w.dims,
                   "blocks": int(blocks.shape[0]), "queries_per_step": nq, "k_cand": w.k,
                   "prefix_codec": w.prefix_codec.name.lower(), "strata": w.strata.name.lower(),
                   "pruning": "off (exhaustive)" if w.exhaustive else "on",
                   "stratum4_weight": round(float(cfg.stratum4_weight), 4),
                   "query_noise": f"isotropic, norm {w.query_noise}" if not w.fresh_queries else "fresh draw"},
        "queries_per_s": round(nq / (ms_step / 1000.0), 1),
        "pairs_per_s": round(w.n_docs * nq / (ms_step / 1000.0), 1),
        "step_algorithmic_gb_s": round(step_bytes / (ms_step / 1000.0) / 1e9, 1),
        "step_hbm_frac": round(step_bytes / (ms_step / 1000.0) / 1e9 / HBM_PEAK_GBS, 4),
        "roofline": roofline_of(groups, nq, prof_steps, w,
                                scanned=timed_stats["blocks"] / args.steps if layout == "clustered" else None),
        "kernels": kernels_of(groups),
        "scan_stats_per_step": {f: v / args.steps for f, v in timed_stats.items()},
        "reruns_per_step": {"safe": timed_stats["reruns_safe"] / args.steps,
                            "dense": timed_stats["reruns_dense"] / args.steps},
        "clock_settle": settle,
    }
    if layout == "clustered":
        # blocks the final pass scanned per query, against the index's
        out["final_pass_blocks_per_query"] = round(timed_stats["blocks"] / args.steps / nq, 1)

    if not args.no_cold:
        # the same steps, each after a 1 GiB read: per-kernel durations with cold caches
        log(f"cold-cache {prof_steps} steps")
        _lib.check(L.mrl_ctx_evict_caches(dev.handle, EVICT_BYTES))
        dev.synchronize()
        _lib.check(L.mrl_ctx_set_profiling(dev.handle, 1))
        for _ in range(prof_steps):
            _lib.check(L.mrl_ctx_evict_caches(dev.handle, EVICT_BYTES))
            step()
        dev.synchronize()
        _lib.check(L.mrl_ctx_set_profiling(dev.handle, 0))
        cg = kernel_groups(L, _lib, dev, 64 * prof_steps + 64)
        fetch(False)
        kernel_ms = sum(float(np.sum(g["ms"])) for g in cg.values()) / prof_steps
        warm_ms = sum(float(np.sum(g["ms"])) for g in groups.values()) / prof_steps
        out["cold_cache"] = {
            "method": f"{EVICT_BYTES >> 20} MiB device read before each step (L2 and Infinity Cache evicted); "
                      "durations from the dispatch-recorded events of the scan's kernels",
            "kernel_ms_per_step": round(kernel_ms, 5), "warm_kernel_ms_per_step": round(warm_ms, 5),
            "value": round(w.n_docs / (kernel_ms / 1000.0) / 1e6, 2), "unit": "Mvec/s",
            "step_algorithmic_gb_s": round(step_bytes / (kernel_ms / 1000.0) / 1e9, 1),
            "roofline": roofline_of(cg, nq, prof_steps, w, cold=True,
                                    scanned=timed_stats["blocks"] / args.steps if layout == "clustered" else None),
            "kernels": kernels_of(cg)}

    if legs:
        out["host_boundary"] = host_boundary_rate(L, _lib, dev, ix, queries, fit, w, ccfg, tr)
        out["rerank"], out["encode"] = rerank_leg(L, _lib, m, dev, w, step, res, queries, args.rerank_reps,
                                                  n_threads, not args.no_cpu_baseline, fit, blocks)
    if cpu and not args.no_cpu_baseline:
        step()
        fetch()
        out["cpu_baseline"], out["parity_query0"] = cpu_baseline(
            w, blocks, queries, fit, ids[0], scores[0], int(counts[0]),
            args.cpu_seconds if cpu_seconds is None else cpu_seconds, n_threads)
    L.mrl_results_destroy(res)
    plan.close()
    for d, p, r in lanes[1:]:
        L.mrl_results_destroy(r)
        p.close()
        d.close()
    ix.close()
    return out


def encode_leg(m, dev, w, rows, fit, blocks, n_threads, with_cpu, reps=5):
    """GPU encoder (mrl_encode_corpus_device) over the workload's rows already
    in HBM: median wall time of the synchronous call, algorithmic bytes = f32
    rows in + records out, and whether its records equal the bench index's
    (built by the host encoder).  cpu: the host C++ encoder on n_threads."""
    import numpy as np
    from mrl_index_amd import source
    d_rows = m.DeviceBuffer.from_array(rows, dev)
    d_out = m.DeviceBuffer(blocks.nbytes, dev)
    n, dims = rows.shape
    m.encode_corpus_device(d_rows.ptr, n, dims, d_out.ptr, dev, source.DOC, fit)
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        m.encode_corpus_device(d_rows.ptr, n, dims, d_out.ptr, dev, source.DOC, fit)
        ts.append(time.perf_counter() - t0)
    same = bool(np.array_equal(d_out.to_array(np.uint8, blocks.shape), blocks))
    d_rows.close()
    d_out.close()
    t = float(np.median(ts))
    alg = n * dims * 4 + blocks.nbytes
    rec = {"ms": round(t * 1000, 3), "rows_per_s": round(n / t, 1), "algorithmic_gb_s": round(alg / t / 1e9, 1),
           "identical_to_host_encoder": same}
    if with_cpu:
        t0 = time.perf_counter()
        m.encode_corpus(rows, source.DOC, fit, None, n_threads)
        rec["cpu_ms"] = round((time.perf_counter() - t0) * 1000, 1)
        rec["cpu_threads"] = n_threads
    return rec


def rerank_leg(L, _lib, m, dev, w, step, res, queries, reps, n_threads, with_cpu, fit, blocks):
    """Post-scan rerank of every query's shortlist, kept in HBM, at fp32 / fp16 /
    int8 (the reference's precision bench, retrieval_bench.rs:736-745).
    us_per_batch: host wall time of one mrl_results_rerank call after a
    finished scan (launches, sync and the copy of the reranked lists to the
    host).  kernel_*: dispatch-recorded durations of the score and sort
    kernels; the score kernel's algorithmic bytes are the shortlisted rows at
    the store's precision plus the query and the candidate ids."""
    import numpy as np
    if w.n_docs > 2_000_000:
        skip = {"skipped": f"corpus rows for {w.n_docs} vectors are not generated by the bench"}
        return skip, skip
    log(f"rerank: generating {w.n_docs} x {w.dims} f32 rows")
    rows = __import__("mrl_index_amd.synth", fromlist=["docs"]).docs(w, 0, w.n_docs, n_threads)
    nq, K = w.n_queries, w.k
    r_rows = np.zeros((nq, K), dtype=np.uint64)
    r_scores = np.zeros((nq, K), dtype=np.float32)
    r_counts = np.zeros(nq, dtype=np.uint32)
    out = {"queries_per_batch": nq, "k_cand": K}
    row_bytes = {m.RerankPrecision.FP32: 4 * w.dims, m.RerankPrecision.FP16: 2 * w.dims,
                 m.RerankPrecision.INT8: w.dims + 2}
    for prec in (m.RerankPrecision.FP32, m.RerankPrecision.FP16, m.RerankPrecision.INT8):
        if prec != m.RerankPrecision.FP32 and w.dims != 768:
            continue
        t0 = time.perf_counter()
        store = m.RerankStore.create(rows, prec, dev)
        t_store = time.perf_counter() - t0

        def rerank():
            _lib.check(L.mrl_results_rerank(dev.handle, res, store.handle, _lib.u64ptr(r_rows), _lib.fptr(r_scores),
                                            _lib.u32ptr(r_counts)))
        step()
        for _ in range(5):
            rerank()
        wall = []
        for _ in range(reps):
            step()
            dev.synchronize()
            t0 = time.perf_counter()
            rerank()
            wall.append(time.perf_counter() - t0)
        _lib.check(L.mrl_ctx_set_profiling(dev.handle, 1))
        for _ in range(reps):
            step()
            rerank()
        _lib.check(L.mrl_ctx_set_profiling(dev.handle, 0))
        cap = 64 * reps + 64
        kt = (_lib.KernelTimeC * cap)()
        nrec = C.c_uint32()
        _lib.check(L.mrl_ctx_profile_collect(dev.handle, kt, cap, C.byref(nrec)))
        sc = [kt[i].ms for i in range(min(nrec.value, cap)) if kt[i].kind == _lib.KERNEL_RERANK]
        so = [kt[i].ms for i in range(min(nrec.value, cap)) if kt[i].kind == _lib.KERNEL_RERANK_SORT]
        n_cand = float(r_counts.sum())
        alg = n_cand * (row_bytes[prec] + 8) + nq * 4 * w.dims
        k_ms = float(np.mean(sc))
        rec = {"store_build_s": round(t_store, 3), "us_per_batch": round(float(np.median(wall)) * 1e6, 2),
               "kernel_score_us": round(k_ms * 1000, 3), "kernel_sort_us": round(float(np.mean(so)) * 1000, 3),
               "score_algorithmic_bytes": alg,
               "score_achieved_gb_s": round(alg / (k_ms / 1000.0) / 1e9, 1)}
        if with_cpu:
            hit_ids = np.zeros((nq, K), dtype=np.uint64)
            _lib.check(L.mrl_results_fetch(dev.handle, res, _lib.u64ptr(hit_ids), None, None, None))
            c0 = int(r_counts[0])
            cand = (hit_ids[0, :c0] >> np.uint64(16)) * np.uint64(64) + (hit_ids[0, :c0] & np.uint64(0xFFFF))
            rec["cpu_us_per_query"], rec["parity_query0"] = cpu_rerank_us(
                prec, queries[0], rows, cand, r_rows[0, :c0], r_scores[0, :c0])
        out[prec.as_str()] = rec
        store.close()
    log("encode: GPU encoder over the same rows")
    enc = encode_leg(m, dev, w, rows, fit, blocks, n_threads, with_cpu)
    del rows
    return out, enc


def cpu_rerank_us(prec, q, rows, cand, gpu_rows, gpu_scores, budget_s=2.0):
    """The oracle's restatement of rerank_exact_rows (one host thread) on query
    0's shortlist (cand: its scan hits as rows, in hit order), timed; and
    whether the GPU's reranked rows and scores for that query are identical."""
    import numpy as np
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import ora
    cand = np.ascontiguousarray(cand, dtype=np.uint64)
    n = 0
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < budget_s or n == 0:
        ref = ora.rerank(int(prec), q, rows, cand)
        n += 1
    us = round((time.perf_counter() - t0) / n * 1e6, 2)
    ok = ref is not None and np.array_equal(ref[0], gpu_rows) and \
        np.array_equal(ref[1].view(np.uint32), np.asarray(gpu_scores, dtype=np.float32).view(np.uint32))
    return us, "identical" if ok else "MISMATCH"


def settle_clocks(L, _lib, dev, ms=SETTLE_MS):
    """Device reads of a 1 GiB buffer (k_read_sweep through
    mrl_ctx_evict_caches) for about `ms` milliseconds before a workload's
    warmup, so that the GPU's clocks have come up from the idle of the
    host-side corpus generation.  No scan step runs here."""
    t0 = time.perf_counter()
    n = 0
    while (time.perf_counter() - t0) * 1000.0 < ms:  # (ms <= 0: none)
        for _ in range(10):
            _lib.check(L.mrl_ctx_evict_caches(dev.handle, EVICT_BYTES))
        n += 10
        dev.synchronize()
    return {"method": f"{EVICT_BYTES >> 20} MiB device reads (k_read_sweep) before the warmup; no scan step",
            "reads": n, "ms": round((time.perf_counter() - t0) * 1000.0, 1)}


def host_boundary_rate(L, _lib, dev, ix, queries, fit, w, ccfg, tr, reps=20):
    """PCIe-inclusive rate of the synchronous host-buffer calls: queries copied
    from host memory (mrl_plans_build), scan, results copied back (mrl_scan).
    Reported beside `value`, never as it."""
    import numpy as np
    nq, k = w.n_queries, w.k
    ids = np.zeros((nq, k), dtype=np.uint64)
    scores = np.zeros((nq, k), dtype=np.float32)
    counts = np.zeros(nq, dtype=np.uint32)
    fitc = fit.to_c() if fit is not None else None
    q = np.ascontiguousarray(queries, dtype=np.float32)
    times = []
    for i in range(reps + 2):
        plans = C.c_void_p()
        dev.synchronize()
        t = time.perf_counter()
        _lib.check(L.mrl_plans_build(dev.handle, _lib.fptr(q), nq, w.dims, int(w.prefix_codec), 0,
                                     C.byref(fitc) if fitc is not None else None, None, C.byref(plans)))
        _lib.check(L.mrl_scan(dev.handle, ix.handle, plans, C.byref(ccfg), C.byref(tr), _lib.u64ptr(ids),
                              _lib.fptr(scores), _lib.u32ptr(counts), None))
        times.append(time.perf_counter() - t)
        L.mrl_plans_destroy(plans)
    t_med = float(np.median(times[2:]))
    return {"ms_per_call": round(t_med * 1000.0, 4), "value": round(w.n_docs / t_med / 1e6, 2), "unit": "Mvec/s",
            "calls": "mrl_plans_build (host queries) + mrl_scan (host results), synchronous, median of "
                     f"{reps}"}


def copy_calibration(mib):
    """Kernels of known traffic for the PMC byte counters' scale factor, from
    the library itself (no second HIP runtime in the process):
    mrl_ctx_evict_caches allocates and fills a buffer of MIB MiB once
    (k_fill_u32: MIB MiB written) and then reads all of it each call
    (k_read_sweep: MIB MiB read); five calls."""
    import mrl_index_amd as m
    from mrl_index_amd import _lib
    n = mib << 20
    dev = m.default_device()
    for _ in range(5):
        _lib.check(_lib.lib.mrl_ctx_evict_caches(dev.handle, n))
    dev.synchronize()
    print(json.dumps({"k_fill_u32_bytes_written_per_dispatch": n, "k_fill_u32_dispatches": 1,
                      "k_read_sweep_bytes_read_per_dispatch": n, "k_read_sweep_dispatches": 5}), flush=True)


def committed_traffic(kernel, workload):
    """HBM bytes per launch of `kernel` for this workload, from the committed
    rocprofv3 --pmc summary (FETCH_SIZE + WRITE_SIZE, scaled by the same
    counters' reading on a copy of known size); None when not measured."""
    name = f"{kernel}_traffic.txt"
    path = os.path.join(ROOT, "profiles", name)
    if not os.path.exists(path):
        return None
    for line in open(path):
        f = line.split()
        if len(f) == 3 and f[0] == "traffic_bytes_per_launch" and f[1] == workload:
            return {"bytes_per_launch": float(f[2]), "source": f"profiles/{name}"}
    return None


def cpu_baseline(w, blocks, queries, fit, gpu_ids, gpu_scores, gpu_count, seconds, n_threads):
    """The oracle's scan_blocks (restated reference, sharded like Rayon) on
    query 0, on n_threads host threads and on one; also the parity check of
    the GPU top-K for that query."""
    import numpy as np
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import ora
    fitc = ora.Fit(fit.mean, 4, fit.seed, fit.n_observed) if fit is not None else None
    op = ora.plan_build(queries[0], w.dims, int(w.prefix_codec), 0, fitc, None)

    def timed(threads, budget, min_runs, max_runs):
        cfg = ora.scan_config(w.k, depth=int(w.strata), sharding=True, threads=threads)
        ref = ora.scan_blocks(blocks, op, cfg)  # warm-up pass (mrl_index.rs:663-664)
        times = []
        t_end = time.time() + budget
        while (time.time() < t_end or len(times) < min_runs) and len(times) < max_runs:
            t = time.perf_counter()
            ref = ora.scan_blocks(blocks, op, cfg)
            times.append(time.perf_counter() - t)
        return float(np.median(times)), len(times), ref

    t_med, n_runs, ref = timed(n_threads, seconds, 5, 50)
    t_one, n_one, _ = timed(1, seconds / 2, 3, 10)
    ref_ids, ref_scores = ref
    # tie-aware top-K comparison (scores bit-exact)
    n = gpu_count
    ok = n == len(ref_ids)
    if ok and n:
        gs, rs = gpu_scores[:n], ref_scores
        ok = np.array_equal(np.sort(gs).view(np.uint32), np.sort(rs).view(np.uint32))
        kth = np.sort(rs)[0] if len(rs) >= w.k else -np.inf
        ok = ok and set(gpu_ids[:n][gs > kth].tolist()) == set(ref_ids[rs > kth].tolist())
    nq = w.n_queries
    base = {"value": round(w.n_docs / (t_med * nq) / 1e6, 3), "unit": "Mvec/s", "cores": n_threads, "kind": "port",
            "per_query_mvec_s": round(w.n_docs / t_med / 1e6, 2), "ms_per_query": round(t_med * 1000, 3),
            "one_thread": {"value": round(w.n_docs / (t_one * nq) / 1e6, 3),
                           "per_query_mvec_s": round(w.n_docs / t_one / 1e6, 2), "ms_per_query": round(t_one * 1000, 3),
                           "runs": n_one},
            "host_cpus": os.cpu_count(), "cpu_model": cpu_model(),
            "sample": f"query 0 of this workload over the full index: the oracle's sharded scan_blocks, one warm-up "
                      f"then {n_runs} runs on {n_threads} threads ({n_one} on one), median; value = N / ({nq} x "
                      f"the per-query time), the batch pass with queries one after another"}
    return base, {"checked": True, "identical_topk": bool(ok)}


if __name__ == "__main__":
    main()
