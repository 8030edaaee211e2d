#!/usr/bin/env python3
"""Benchmark: MTP verify decode attention over a 61,444-token int8 paged KV cache on one MI355X.

Workload: 1 sequence, 4 causal query tokens, 24 q heads / 4 kv heads (GQA 6 -> 24 rows per kv
head), head_dim 256, ctx 61,440 + 4, int8 per-token-head cache (K/V ~ N(0,1) quantised
absmax/127), block_size 16, random page permutation, fp16 out. One step = one operator call
(one attention layer: both kernels, all 24 heads).

Every call reads a different one of `--rotate` identical caches, so each layer reads its KV from
HBM as it would inside a model (a single 128 MB cache re-read back to back would be served
partly by the 256 MB Infinity Cache). The calls are captured in a HIP graph and replayed; the
timed region is bracketed by device synchronisation and measured with HIP events on the
stream the kernels run on. The split-K partial kernel, which moves the KV bytes, is timed the
same way on its own for the roofline. The CPU baseline is the float64 oracle on this host.

Prints one JSON line.

`--prefill` instead measures the chunked-prefill operator (forward_pth interface) on a 2048-token
causal chunk over 61,440 cached tokens (63,488 keys), 24 q / 4 kv heads, block_size 16: one step
is one operator call; the line reports TFLOP/s against the fp16 MFMA peak, and the CPU baseline is
the float64 oracle on a sample of query rows.
"""
import argparse
import json
import math
import os
import platform
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG_DIR = os.path.join(ROOT, "mi50-vllm-lab_amd")
sys.path.insert(0, ROOT)

METRIC = "µs/layer + achieved KV GB/s (% of HBM peak), MTP 24-row decode at 61k ctx"
HBM_PEAK_GBS = 8000.0
MFMA_FP16_PEAK_TFLOPS = 2500.0
PREFILL_METRIC = "TFLOP/s (MFMA fp16 peak 2.5 PF/s), 2048-token int8-KV chunked prefill over 63,488 keys"
NSEG = 128
CALIB_BYTES = 256 << 20
CALIB_COPIES = 8


def _pmc_dispatches(run_dir, counter):
    """{dispatch id: (kernel name, summed counter value)} from a rocprofv3 --pmc csv run directory."""
    import csv
    import glob

    files = glob.glob(os.path.join(run_dir, "**", "*counter_collection.csv"), recursive=True)
    if not files:
        raise SystemExit(f"no *counter_collection.csv under {run_dir}")
    out = {}
    for fn in files:
        with open(fn) as f:
            for r in csv.DictReader(f):
                if r["Counter_Name"] != counter:
                    continue
                key = (fn, int(r["Dispatch_Id"]))
                name, v = out.get(key, (r["Kernel_Name"], 0.0))
                out[key] = (name, v + float(r["Counter_Value"]))
    return out


def summarize_traffic(args):
    """HBM bytes per pd_partial_kernel launch from FETCH_SIZE and WRITE_SIZE runs of --profile-only.

    Both counters are read in KiB per dispatch. Each is scaled by what it reads for the calibration
    copy (CALIB_BYTES read and CALIB_BYTES written per launch, the last CALIB_COPIES dispatches)."""
    res = {}
    for counter, run_dir in (("FETCH_SIZE", args.traffic_summary[0]), ("WRITE_SIZE", args.traffic_summary[1])):
        d = _pmc_dispatches(run_dir, counter)
        order = sorted(d)
        part = [d[k][1] for k in order if "pd_partial_kernel" in d[k][0]]
        other = [d[k][1] for k in order if not d[k][0].startswith("pd_")]
        calib = other[-CALIB_COPIES:]
        if not part or len(calib) < CALIB_COPIES:
            raise SystemExit(f"{counter}: {len(part)} partial dispatches, {len(calib)} calibration copies")
        part.sort()
        calib.sort()
        p_kib, c_kib = part[len(part) // 2], calib[len(calib) // 2]
        factor = (CALIB_BYTES / 1024.0) / c_kib
        res[counter] = {"partial_kib_median": p_kib, "calib_copy_kib_median": c_kib, "calib_factor": factor,
                        "partial_bytes": p_kib * 1024.0 * factor, "dispatches": len(part)}
    total = res["FETCH_SIZE"]["partial_bytes"] + res["WRITE_SIZE"]["partial_bytes"]
    summary = {"kernel": "pd_partial_kernel", "workload": "MTP verify 4 x 24/4 heads, ctx 61440+4, bs 16",
               "nsplit": args.nsplit, "hbm_bytes_per_launch": round(total), "counters": res,
               "calibration": f"{CALIB_COPIES} copies of {CALIB_BYTES} bytes (read + write) after the partial "
                              f"launches; factor = known bytes / counter bytes"}
    with open(args.traffic_out, "w") as f:
        json.dump(summary, f, indent=1)
    print(json.dumps(summary))


def load_package():
    import importlib.util

    if "mi50_vllm_lab_amd" in sys.modules:
        return sys.modules["mi50_vllm_lab_amd"]
    spec = importlib.util.spec_from_file_location("mi50_vllm_lab_amd", os.path.join(PKG_DIR, "__init__.py"),
                                                  submodule_search_locations=[PKG_DIR])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["mi50_vllm_lab_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


def cpu_model() -> str:
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.startswith("Model name"):
                return line.split(":", 1)[1].strip()
    except Exception:
        pass
    return platform.processor() or "unknown"


def build_workload(kvc, ctx, qlen, seed):
    return kvc.make_case([ctx], [qlen], num_q_heads=24, num_kv_heads=4, block_size=16, seed=seed)


def time_graph(torch, graph, replays, stream):
    """Average ms per replay of `graph`, HIP events on `stream`, synchronised on both sides."""
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(replays):
        graph.replay()
    end.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(end) / replays


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=4000, help="timed operator calls")
    ap.add_argument("--warmup", type=int, default=200, help="untimed operator calls")
    ap.add_argument("--nsplit", type=int, default=64)
    ap.add_argument("--rotate", type=int, default=8, help="distinct KV caches cycled through")
    ap.add_argument("--ctx", type=int, default=61440)
    ap.add_argument("--qlen", type=int, default=4)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-runs", type=int, default=5)
    ap.add_argument("--profile-only", action="store_true",
                    help="replay the partial kernel only, then a plain copy of known size that calibrates the "
                         "rocprofv3 FETCH_SIZE / WRITE_SIZE counters (for counter runs)")
    ap.add_argument("--hot", action="store_true",
                    help="also time every call on the same (Infinity-Cache resident) cache; reported beside")
    ap.add_argument("--traffic-summary", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                    help="no GPU work: turn two rocprofv3 --pmc runs of --profile-only (FETCH_SIZE, WRITE_SIZE) "
                         "into HBM bytes per partial launch, written to --traffic-out")
    ap.add_argument("--traffic-out", default=os.path.join(ROOT, "profiles", "pd_partial_mtp61k_traffic.json"))
    ap.add_argument("--prefill", action="store_true", help="measure the chunked-prefill operator instead")
    ap.add_argument("--chunk", type=int, default=2048, help="--prefill: query tokens per chunk")
    ap.add_argument("--cpu-rows", type=int, default=24, help="--prefill: query rows in the CPU baseline sample")
    args = ap.parse_args()

    if args.traffic_summary:
        summarize_traffic(args)
        return

    if args.gpus != 1:
        print(json.dumps({"error": f"--gpus {args.gpus}: this benchmark measures one GPU; the operator is "
                                   "single-GPU (multi-GPU runs shard by kv head and are not part of this build)"}))
        sys.exit(2)

    import torch

    pkg = load_package()
    kvc, pd = pkg.kvcache, pkg.pth_dec
    pd.load_library()
    if not torch.cuda.is_available():
        print(json.dumps({"error": "no GPU visible"}))
        sys.exit(1)
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)

    if args.prefill:
        bench_prefill(args, torch, kvc, pd, dev)
        return

    seed = 1002
    case = build_workload(kvc, args.ctx, args.qlen, seed)
    alg_bytes = kvc.algorithmic_bytes(case)
    kv_bytes = kvc.visible_kv_bytes(case)
    flops = kvc.algorithmic_flops(case)
    partial_bytes = alg_bytes - 2 * case.num_tokens * case.num_q_heads * 256  # the partial pass writes no out

    d = case.to(dev)
    caches = [d.cache] + [kvc.clone_cache(d.cache) for _ in range(args.rotate - 1)]
    T, HQ, HKV = d.num_tokens, d.num_q_heads, d.cache.num_kv_heads
    out = torch.empty((T, HQ, 256), dtype=torch.float16, device=dev)
    po, pm, pl = kvc.partial_buffers(T, HQ, NSEG, dev)
    qmax = d.qmax

    def op(cache):
        pd.decode(d.q, cache.key_cache, cache.value_cache, cache.k_scale, cache.v_scale, d.block_table,
                  d.seq_lens, d.query_start_loc, out, d.scale, po, pm, pl, 1, qmax, args.nsplit)

    def partial(cache):
        rc = pd.launch_partial(d.q, cache.key_cache, d.block_table, d.seq_lens, d.query_start_loc, po, pm, pl,
                               num_seqs=1, heads_q=HQ, heads_kv=HKV, block_size=16, scale=d.scale, qmax=qmax,
                               nsplit=args.nsplit)
        if rc != 0:
            raise RuntimeError(f"pth_dec_launch_partial failed: {rc}")

    stream = torch.cuda.Stream()
    # eager warm-up on the side stream, then capture one rotation of calls per graph
    with torch.cuda.stream(stream):
        for c in caches:
            op(c)
    torch.cuda.synchronize()
    g_op, g_part = torch.cuda.CUDAGraph(), torch.cuda.CUDAGraph()
    with torch.cuda.graph(g_op, stream=stream):
        for c in caches:
            op(c)
    with torch.cuda.graph(g_part, stream=stream):
        for c in caches:
            partial(c)
    torch.cuda.synchronize()

    R = len(caches)
    if args.profile_only:
        for _ in range(max(1, args.steps // R)):
            g_part.replay()
        torch.cuda.synchronize()
        # calibration: CALIB_COPIES plain device copies of CALIB_BYTES each, launched last
        src = torch.ones(CALIB_BYTES // 4, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        for _ in range(CALIB_COPIES):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"profile_only": True, "partial_launches": R * max(1, args.steps // R),
                          "nsplit": args.nsplit, "calib_copies": CALIB_COPIES, "calib_bytes": CALIB_BYTES}))
        return

    warm_reps = max(1, math.ceil(args.warmup / R))
    reps = max(1, math.ceil(args.steps / R))
    steps = reps * R
    with torch.cuda.stream(stream):
        for _ in range(warm_reps):
            g_op.replay()
        ms_rot = time_graph(torch, g_op, reps, stream) / R           # per layer, cold caches
        for _ in range(warm_reps):
            g_part.replay()
        part_ms = time_graph(torch, g_part, reps, stream) / R         # partial kernel per launch
    ms_hot = None
    if args.hot:
        # same cache every call (Infinity-Cache resident): reported beside, never as `value`
        g_hot = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g_hot, stream=stream):
            for _ in range(R):
                op(caches[0])
        with torch.cuda.stream(stream):
            for _ in range(warm_reps):
                g_hot.replay()
            ms_hot = time_graph(torch, g_hot, reps, stream) / R

    us_layer = ms_rot * 1e3
    gbs = alg_bytes / (ms_rot * 1e-3) / 1e9
    part_gbs = partial_bytes / (part_ms * 1e-3) / 1e9

    traffic = None
    tpath = os.path.join(ROOT, "profiles", "pd_partial_mtp61k_traffic.json")
    if os.path.exists(tpath):
        try:
            with open(tpath) as f:
                t = json.load(f)
            if t.get("nsplit") == args.nsplit:
                traffic = t.get("hbm_bytes_per_launch")
        except Exception:
            traffic = None

    cpu = None
    if not args.no_cpu_baseline:
        import numpy as np

        from oracle import attention as orc

        def cpu_once():
            orc.paged_decode(case.q, case.cache.key_cache, case.cache.value_cache, case.cache.k_scale,
                             case.cache.v_scale, case.block_table, case.seq_lens, case.query_start_loc, 1,
                             case.scale, -1, True)

        cpu_once()  # warm-up
        times = []
        for _ in range(args.cpu_runs):
            t0 = time.perf_counter()
            cpu_once()
            times.append(time.perf_counter() - t0)
        med = float(np.median(times))
        cpu = {"value": alg_bytes / med / 1e9, "unit": "GB/s", "cores": os.cpu_count(), "kind": "port",
               "us_per_layer": med * 1e6,
               "sample": f"float64 numpy oracle (oracle/attention.py), the full config-2 layer, median of "
                         f"{args.cpu_runs} runs after 1 warm-up, numpy/BLAS threads on {os.cpu_count()} cores "
                         f"({cpu_model()})",
               "gpu_speedup": med * 1e6 / us_layer}

    line = {
        "metric": METRIC,
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warm_reps * R,
        "ms_per_step": round(ms_rot, 6),
        "us_per_layer": round(us_layer, 3),
        "pct_hbm_peak": round(100.0 * gbs / HBM_PEAK_GBS, 2),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8 KV / fp16 MFMA / fp32 softmax",
        "data": "synthetic (seeded N(0,1) K/V quantised absmax/127, random page permutation)",
        "config": {"workload": f"MTP verify decode: 1 seq x {args.qlen} query tokens, 24 q / 4 kv heads, "
                               f"head_dim 256, ctx {args.ctx}+{args.qlen} int8 per-token-head paged KV, "
                               f"block_size 16",
                   "nsplit": args.nsplit, "rotating_caches": R, "algorithmic_bytes": alg_bytes,
                   "kv_bytes": kv_bytes, "flops": flops},
        "roofline": {"bound": "hbm", "achieved": round(part_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(part_gbs / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "kernel": "pd_partial_kernel", "avg_launch_us": round(part_ms * 1e3, 3),
                     "bytes_per_launch": partial_bytes},
        "hot_cache_us_per_layer": None if ms_hot is None else round(ms_hot * 1e3, 3),
        "tflops": round(flops / (ms_rot * 1e-3) / 1e12, 2),
        "cpu_baseline": cpu,
    }
    print(json.dumps(line))


def bench_prefill(args, torch, kvc, pd, dev):
    """One JSON line for the chunked-prefill operator (see the module docstring)."""
    ctx, sq = args.ctx, args.chunk
    steps = max(1, min(args.steps, 200)) if args.steps != 4000 else 20
    warm = max(1, min(args.warmup, 20)) if args.warmup != 200 else 3
    case = kvc.make_case([ctx], [sq], num_q_heads=24, num_kv_heads=4, block_size=16, seed=1005)
    flops = kvc.prefill_flops([ctx + sq], [ctx], sq, 24)
    d = case.to(dev)
    caches = [d.cache, kvc.clone_cache(d.cache)]
    q = kvc.prefill_query(d)
    qa = torch.tensor([ctx], dtype=torch.int32, device=dev)
    out = torch.empty((1, sq, 24, 256), dtype=torch.float32, device=dev)

    def op(c):
        pd.forward_pth(q, c.key_cache, c.value_cache, d.block_table, d.seq_lens, d.scale, qa, out=out)

    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        for c in caches:
            op(c)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        for c in caches:
            op(c)
    torch.cuda.synchronize()
    R = len(caches)
    reps = max(1, math.ceil(steps / R))
    with torch.cuda.stream(stream):
        for _ in range(max(1, math.ceil(warm / R))):
            g.replay()
        ms = time_graph(torch, g, reps, stream) / R
    tflops = flops / (ms * 1e-3) / 1e12

    cpu = None
    if not args.no_cpu_baseline:
        import numpy as np

        from oracle import attention as orc

        rows = np.linspace(0, sq - 1, args.cpu_rows).astype(int).tolist()
        qcpu = kvc.prefill_query(case)
        qa_cpu = torch.tensor([ctx], dtype=torch.int32)

        def cpu_once():
            orc.paged_prefill(qcpu, case.cache.key_cache, case.cache.value_cache, case.cache.k_scale,
                              case.cache.v_scale, case.block_table, case.seq_lens, case.scale, qa_cpu, rows)

        cpu_once()
        times = []
        for _ in range(3):
            t0 = time.perf_counter()
            cpu_once()
            times.append(time.perf_counter() - t0)
        med = float(np.median(times))
        sample_flops = 4 * 256 * 24 * sum(min(ctx + sq, ctx + r + 1) for r in rows)
        cpu = {"value": round(sample_flops / med / 1e12, 6), "unit": "TFLOP/s", "cores": os.cpu_count(),
               "kind": "port",
               "sample": f"float64 numpy oracle (oracle/attention.py paged_prefill) on {len(rows)} of the {sq} "
                         f"query rows (all 24 heads, full visible context each), median of 3 runs after 1 "
                         f"warm-up, BLAS threads on {os.cpu_count()} cores ({cpu_model()})",
               "est_ms_full_chunk": round(flops / (sample_flops / med) * 1e3, 1)}

    line = {
        "metric": PREFILL_METRIC,
        "value": round(tflops, 1),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": reps * R,
        "warmup": max(1, math.ceil(warm / R)) * R,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8 KV widened to fp16 / fp16 MFMA / fp32 accumulate",
        "data": "synthetic (seeded N(0,1) K/V quantised absmax/127, fp16-valued Q, random page permutation)",
        "config": {"workload": f"chunked prefill: 1 seq, {sq}-token causal chunk over {ctx} cached tokens "
                               f"({ctx + sq} keys), 24 q / 4 kv heads, head_dim 256, int8 per-token-head "
                               f"paged KV, block_size 16", "flops": flops, "rotating_caches": R},
        "roofline": {"bound": "mfma", "achieved": round(tflops, 1), "peak": MFMA_FP16_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(tflops / MFMA_FP16_PEAK_TFLOPS, 4), "traffic": None,
                     "kernel": "pd_prefill_kernel", "avg_launch_us": round(ms * 1e3, 2)},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
