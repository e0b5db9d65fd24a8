#!/usr/bin/env python3
"""Decode-step benchmark of the MI355X split-KV decode-attention path.

Workload (the north-star shape): Llama-3-8B-shaped
GQA decode, 32 query heads over 8 KV heads, head dimension 128, batch 1,
32768 cached tokens, K/V ~ N(0,1) from the reference generator
(runtime/kvf_host.h:51-61, seed 1) with 1% outlier channels x8, quantized
int8:G=64 on the GPU by the product's quantize/place kernel, head-major
contiguous. One step = one decode-attention call of the plan (the split
kernel plus the log-sum-exp merge), exactly what the reference's generated
kvf_launch_<name> enqueues (runtime/kvf_kernels.cuh:309-320).

Timing. The cache is replicated into enough copies that consecutive steps
never find their bytes in the 256 MiB Infinity Cache (the reference flushes
with a memset instead, runtime/kvf_host.h:302-331; a rotation keeps the flush
out of the timed region). The GPU is held behind a spin kernel while the
host enqueues all K steps, so the timed region is the GPU's own back-to-back
rate, not Python's launch rate. HIP events bracket the K steps and, inside
each step, the split kernel alone (the roofline's dominant kernel).

The CPU baseline times the oracle's restatement of reference_attention
(runtime/kvf_host.h:202-234, double precision) on the same dequantised cache,
on every host core this job may use (OMP_NUM_THREADS, else all) and on one
core. Beside the measurement, config.cost_model gives the kvf planner's
predicted time for the benchmarked plan and the planner's own top-1 plan
(machines/mi355x.gpu, kvforge_amd/model/constants_mi355x.cal).
"""
import argparse
import ctypes
import json
import math
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
METRIC = ("\u00b5s/decode step + achieved HBM GB/s (% of peak), "
          "GQA32/8 d128 32k int8:64")


def parse():
    p = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=400)
    p.add_argument("--warmup", type=int, default=50)
    p.add_argument("--fmt", default="int8", choices=["f16", "int8", "int4"])
    p.add_argument("--group", type=int, default=64)
    p.add_argument("--n", type=int, default=32768)
    p.add_argument("--order", default="hm", choices=["hm", "tm"])
    p.add_argument("--block-tokens", type=int, default=0)
    p.add_argument("--splits", type=int, default=32)
    p.add_argument("--warps", type=int, default=4)
    p.add_argument("--unroll", type=int, default=2)
    p.add_argument("--pack", type=int, default=1)
    p.add_argument("--copies", type=int, default=0,
                   help="cache replicas rotated over steps (0: enough for 1 GiB)")
    p.add_argument("--cpu-seconds", type=float, default=12.0,
                   help="CPU baseline budget (0 skips it)")
    p.add_argument("--fused", action="store_true",
                   help="time the one-launch fused-merge entry point instead of the drop-in "
                        "two-launch kvf_launch_variant")
    p.add_argument("--json-only", action="store_true")
    return p.parse_args()


def log(*a, quiet=False):
    if not quiet:
        print(*a, file=sys.stderr, flush=True)


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; the path shards by "
                          "(batch, kv-head) with no exchange, see DESIGN.md"}), flush=True)
        sys.exit(2)
    import numpy as np
    import torch
    from kvforge_amd import runtime as R

    q_ = args.json_only
    B, H, Hkv, D, n = 1, 32, 8, 128, args.n
    fmt = R.FMT_BY_NAME[args.fmt]
    group = args.group if fmt != R.FMT_F16 else 0
    order = R.ORD_HEAD if args.order == "hm" else R.ORD_TOKEN
    bt = args.block_tokens
    G = H // Hkv if args.pack else 1
    vid = R.variant_id(fmt, order, bt > 0, G, args.unroll, D)
    dev = torch.device("cuda:0")
    R.hip_lib()
    host = R.host_lib()

    # ---- inputs: reference generator + outlier channels, quantized on GPU ----
    t_prep = time.perf_counter()
    q = np.empty((B, H, D), np.float32)
    K = np.empty((B, Hkv, n, D), np.float32)
    V = np.empty((B, Hkv, n, D), np.float32)
    P = ctypes.c_void_p
    host.kvfh_make_data(B, H, Hkv, D, n, 1, P(q.ctypes.data), P(K.ctypes.data), P(V.ctypes.data))
    host.kvfh_inject_outliers(B, Hkv, D, n, 1001, 0.01, 8.0, P(K.ctypes.data), P(V.ctypes.data))
    rows, mb = R.rows_alloc(B, Hkv, n, bt)
    table = None
    if bt:
        tbl = np.empty(B * mb, np.int32)
        host.kvfh_page_table(B * mb, 18, P(tbl.ctypes.data))
        table = torch.from_numpy(tbl).to(dev)
    rb = R.row_bytes(fmt, D)
    mw = D // group if group else 0
    k0 = torch.zeros(rows * rb, dtype=torch.uint8, device=dev)
    v0 = torch.zeros(rows * rb, dtype=torch.uint8, device=dev)
    km0 = torch.zeros(rows * mw, dtype=torch.int32, device=dev) if mw else None
    vm0 = torch.zeros(rows * mw, dtype=torch.int32, device=dev) if mw else None
    for src, dst, dm in ((K, k0, km0), (V, v0, vm0)):
        x = torch.from_numpy(src).to(dev)
        R.quantize_place(fmt, group, D, x, B, Hkv, n, order, bt, table, mb, dst, dm)
        del x
    torch.cuda.synchronize()
    qd = torch.from_numpy(q).to(dev)
    log(f"inputs ready in {time.perf_counter() - t_prep:.1f} s", quiet=q_)

    # algorithmic bytes per step (runtime/kvf_driver.cu:51: KV payload + group meta)
    alg_bytes = 2 * B * n * Hkv * (rb + mw * 4)
    cache_bytes = alg_bytes if not bt else 2 * rows * (rb + mw * 4)
    copies = args.copies or max(4, math.ceil((1 << 30) / cache_bytes))
    caches = [(k0, v0, km0, vm0)]
    for _ in range(copies - 1):
        caches.append(tuple(t.clone() if t is not None else None for t in (k0, v0, km0, vm0)))
    S = args.splits
    out = torch.zeros((B, H, D), dtype=torch.float32, device=dev)
    part_o = torch.zeros((B, H, S, D), dtype=torch.float32, device=dev)
    part_ml = torch.zeros((B, H, S, 2), dtype=torch.float32, device=dev)
    arg_list = [R.make_args(qd, k, v, km, vm, table, out, part_o, part_ml, B, H, Hkv, n, S,
                            args.warps, group=group, block_tokens=bt, max_blocks=mb, D=D)
                for (k, v, km, vm) in caches]
    L = R.hip_lib()
    vb = vid.encode()
    st = torch.cuda.current_stream()
    sh = ctypes.c_void_p(st.cuda_stream)
    launch_step = L.kvf_launch_variant
    launch_timed = L.kvf_launch_partial_variant_timed
    refs = [ctypes.byref(a) for a in arg_list]

    def step(i):
        e = launch_step(vb, refs[i % copies], sh)
        if e:
            raise R.KvfError(f"kvf_launch_variant({vid}) failed: {e}")

    # correctness guard: the plan's output must match a single-split run
    step(0)
    torch.cuda.synchronize()
    got = out.clone()
    a1 = R.make_args(qd, k0, v0, km0, vm0, table, out, None, None, B, H, Hkv, n, 1, 4,
                     group=group, block_tokens=bt, max_blocks=mb, D=D)
    R.launch(R.variant_id(fmt, order, bt > 0, G, 2, D), a1)
    torch.cuda.synchronize()
    rel = float(torch.linalg.vector_norm(got - out) / torch.linalg.vector_norm(out))
    if not (rel < 2e-3 and bool(torch.isfinite(got).all())):
        raise SystemExit(f"plan {vid} S={S} disagrees with S=1: rel_l2 {rel}")

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    K_ = args.steps

    # fused path: one launch per step, split merge inside the kernel
    counters = torch.zeros(B * (Hkv if G > 1 else H), dtype=torch.int32, device=dev)
    launch_fused = L.kvf_launch_fused_variant
    cptr = ctypes.c_void_p(counters.data_ptr())

    def step_fused(i):
        e = launch_fused(vb, refs[i % copies], None, cptr, sh)
        if e:
            raise R.KvfError(f"kvf_launch_fused_variant({vid}) failed: {e}")

    if S > 1 and args.fused:
        out.zero_()
        step_fused(0)
        torch.cuda.synchronize()
        relf = float(torch.linalg.vector_norm(got - out) / torch.linalg.vector_norm(got))
        if not (relf < 1e-5 and int(counters.abs().sum()) == 0):
            raise SystemExit(f"fused step disagrees with the two-launch step: {relf}")
        for i in range(args.warmup):
            step_fused(i)
        torch.cuda.synchronize()

    # ---- timed region: K decode steps back to back, as a serving loop issues
    # them; the GPU is held by a spin kernel while the host enqueues ---------
    def timed(fn):
        e_start = torch.cuda.Event(enable_timing=True)
        e_end = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        w0 = time.perf_counter()
        torch.cuda._sleep(int(5e7))
        e_start.record(st)
        for i in range(K_):
            fn(i)
        e_end.record(st)
        starved = e_start.query()
        torch.cuda.synchronize()
        w1 = time.perf_counter()
        if starved:
            log("warning: the GPU reached the timed region before the host finished "
                "enqueueing; the step time includes host launch gaps", quiet=q_)
        return e_start.elapsed_time(e_end) / K_, w1 - w0

    step2_ms, wall_2 = timed(step)
    if S > 1 and args.fused:
        step_ms, wall_t = timed(step_fused)
        path = "kvf_launch_fused_variant (one launch, in-kernel split merge)"
    else:
        step_ms, wall_t = step2_ms, wall_2
        path = "kvf_launch_variant (split kernel + merge kernel)"
    wall0, wall1 = 0.0, wall_t

    # ---- the split kernel alone, K launches, each timed by events bound to
    # its own dispatch (the duration a kernel trace reports) ------------------
    kev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(K_)]
    for e0, e1 in kev:  # create the events
        e0.record(st)
        e1.record(st)
    torch.cuda.synchronize()
    torch.cuda._sleep(int(5e7))
    for i in range(K_):
        e = launch_timed(vb, refs[i % copies], sh, kev[i][0], kev[i][1])
        if e:
            raise R.KvfError(f"kvf_launch_partial_variant_timed failed: {e}")
    torch.cuda.synchronize()
    part_ms = [e0.elapsed_time(e1) for e0, e1 in kev]
    part_avg_us = 1e3 * sum(part_ms) / K_
    part_med_us = 1e3 * statistics.median(part_ms)

    achieved = alg_bytes / (part_avg_us * 1e-6) / 1e9
    traffic = _traffic_from_profiles(vid, n)
    result = {
        "metric": METRIC,
        "value": round(step_ms * 1e3, 3),
        "unit": "us/step",
        "n_gpus": 1,
        "steps": K_,
        "warmup": args.warmup,
        "ms_per_step": round(step_ms, 6),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u8" if fmt == R.FMT_INT8 else ("u4" if fmt == R.FMT_INT4 else "f16"),
        "data": "synthetic: reference generator seed 1 + 1% outlier channels x8",
        "config": {
            "workload": f"GQA{H}/{Hkv} d{D} n{n} B{B} {args.fmt}{':' + str(group) if group else ''} "
                        f"{args.order}/{'paged:%d' % bt if bt else 'contiguous'}",
            "plan": f"{vid} splits={S} waves={args.warps}",
            "entry_point": path,
            "two_launch_us_per_step": round(step2_ms * 1e3, 3),
            "alg_bytes_per_step": alg_bytes,
            "step_hbm_gbs": round(alg_bytes / (step_ms * 1e-3) / 1e9, 1),
            "step_frac_of_peak": round(alg_bytes / (step_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "partial_kernel_us_avg": round(part_avg_us, 3),
            "partial_kernel_us_median": round(part_med_us, 3),
            "cache_copies_rotated": copies,
            "wall_s_timed_region": round(wall1 - wall0, 4),
        },
        "roofline": {
            "bound": "hbm",
            "kernel": "decode_partial",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic,
        },
        "cpu_baseline": None,
    }
    result["config"]["cost_model"] = _cost_model(args, H, Hkv, D, n, group, bt, vid, S)
    if args.cpu_seconds > 0:
        result["cpu_baseline"] = _cpu_baseline(args, K, V, q, fmt, group, D, step_ms, q_)
    print(json.dumps(result), flush=True)


def _traffic_from_profiles(vid, n):
    """HBM bytes per launch of the split kernel from the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE summary (scaled by the copy-kernel calibration
    recorded in that file), or None if no summary covers this plan."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            tab = json.load(f)
    except (OSError, ValueError):
        return None
    ent = tab.get(f"{vid}:n{n}")
    return ent.get("hbm_bytes_per_launch") if ent else None


def _cpu_baseline(args, K, V, q, fmt, group, D, step_ms, quiet):
    """Oracle reference_attention (runtime/kvf_host.h:202-234, double precision)
    on the dequantised cache: one core, then every host core this job may use
    (the (sequence, head) pairs spread over threads, identical output)."""
    import numpy as np
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import _oracle as O
    _, kdeq = O.quantize(fmt, group, D, K)[::2]
    _, vdeq = O.quantize(fmt, group, D, V)[::2]
    threads = int(os.environ.get("OMP_NUM_THREADS") or 0) or (os.cpu_count() or 1)
    threads = max(1, min(threads, os.cpu_count() or 1))

    def sample(fn, budget):
        times = []
        t_end = time.perf_counter() + budget
        while len(times) < 3 or (time.perf_counter() < t_end and len(times) < 50):
            t0 = time.perf_counter()
            fn()
            times.append(time.perf_counter() - t0)
        return statistics.median(times), len(times)

    one, n1 = sample(lambda: O.reference_attention(q, kdeq, vdeq), args.cpu_seconds * 0.7)
    allc, na = sample(lambda: O.reference_attention_mt(q, kdeq, vdeq, threads),
                      args.cpu_seconds * 0.3)
    log(f"cpu reference_attention: {one * 1e3:.1f} ms/step on 1 core ({n1} reps), "
        f"{allc * 1e3:.2f} ms/step on {threads} threads ({na} reps)", quiet=quiet)
    return {
        "value": round(allc * 1e6, 1),
        "unit": "us/step",
        "cores": threads,
        "kind": "port",
        "sample": f"full decode step (double-precision reference_attention over the dequantised "
                  f"cache, every (sequence, head) pair), median of {na} reps on {threads} threads; "
                  f"1 core: median of {n1} reps",
        "single_core_us": round(one * 1e6, 1),
        "gpu_speedup": round(allc * 1e3 / step_ms, 1),
    }


def _cost_model(args, H, Hkv, D, n, group, bt, vid, S):
    """The kvf planner's prediction for the benchmarked plan and its own top-1
    plan for the same shape (MI355X machine file and fitted constants), or
    None when the compiler binary is not built."""
    import csv
    import subprocess
    import tempfile
    kvf = os.path.join(ROOT, "kvforge_amd", "bin", "kvf")
    if not os.path.exists(kvf):
        return None
    spec = (f"decode bench(H: {H}, H_kv: {Hkv}, d: {D}, n: {n}) {{\n"
            f"  Q: query<H, d, f32>\n  K: kvcache<n, d, ?, ?, ?>\n  V: kvcache<n, d, ?, ?, ?>\n"
            f"  O = decode_attn(Q, K, V, scale = auto, splits = ?, gqa_pack = ?)\n}}\n")
    with tempfile.TemporaryDirectory() as tmp:
        path = os.path.join(tmp, "bench.kv")
        with open(path, "w") as f:
            f.write(spec)
        r = subprocess.run([kvf, "plan", path, "--quant", "--all", "--out", tmp,
                            "--machine", os.path.join(ROOT, "machines", "mi355x.gpu"),
                            "--calib", os.path.join(ROOT, "kvforge_amd", "model", "constants_mi355x.cal")],
                           capture_output=True, text=True)
        if r.returncode != 0:
            return None
        with open(os.path.join(tmp, "plans.csv")) as f:
            rows = list(csv.DictReader(f))
    fmt_name = vid.split("_")[0]
    want = {"fmt": fmt_name, "group": str(group), "order": "head_major" if args.order == "hm" else "token_major",
            "residency": "paged" if bt else "contiguous", "block_tokens": str(bt), "splits": str(S),
            "gqa_pack": str(args.pack), "warps": str(args.warps), "unroll": str(args.unroll)}
    mine = next((r for r in rows if all(r[k] == v for k, v in want.items())), None)
    live = [r for r in rows if r["rejected"] == "0"]
    best = min(live, key=lambda r: float(r["pred_us"])) if live else None
    out = {"predicted_us_per_step": round(float(mine["pred_us"]), 3) if mine else None}
    if best:
        out["model_top1"] = (f"{best['fmt']}:{best['group']} {best['order']}/{best['residency']} "
                             f"splits={best['splits']} pack={best['gqa_pack']} w{best['warps']} "
                             f"u{best['unroll']}")
        out["model_top1_predicted_us"] = round(float(best["pred_us"]), 3)
    return out


if __name__ == "__main__":
    main()
