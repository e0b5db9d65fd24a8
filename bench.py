#!/usr/bin/env python3
"""Decode-step benchmark of the MI355X split-KV decode-attention path.

Workloads (--config selects, 2 is the default and the
one the headline metric is quoted on):

  1  MHA decode: 32 heads (32 KV heads), head dim 128, batch 1, 4096 cached
     tokens, f16 KV head-major contiguous, one split (plan
     f16_hm_c_g1_u2_d128): the reference's CPU-runnable plumbing case.
  2  Llama-3-8B-shaped GQA decode: 32 query heads over 8 KV heads, head dim
     128, batch 1, 32768 cached tokens, K/V ~ N(0,1) from the reference
     generator (runtime/kvf_host.h:51-61, seed 1) with 1% outlier channels x8,
     quantized int8:G=64 on the GPU by the product's quantize/place kernel,
     head-major contiguous; plan int8_hm_c_g4_u2_d128, 32 splits. With
     --fmt f16 the same cache unquantized (plan f16_hm_c_g4_u2_d128).
  3  Paged batched GQA decode: batch 8, lengths uniform in [2048, 8192] (seed
     2), one shared pool of 4096 pages of 16 tokens shuffled with seed 18 and
     handed out in order, token-major int8:64, binary16 query and output,
     through the variable-length extension.
  4  Long-context GQA decode: batch 1, 65536 tokens, int4:G=32 head-major
     contiguous.

One step = one decode-attention call of the plan. Two steps are timed on
every run and reported in config, their outputs checked to agree before
timing: the one-launch step (kvf_launch_fused_variant: the split kernel
merges its splits in its last workgroup per head group) and the drop-in step
the reference's generated kvf_launch_<name> enqueues (split kernel, then the
log-sum-exp merge kernel; runtime/kvf_kernels.cuh:309-320). The headline
value (--step auto) is the faster of the two in this run: they are within a
few per cent of each other and which one wins differs between boxes;
config.entry_point names it, and --step fused / two-launch fixes one.

Timing. The cache is replicated into enough copies that consecutive steps
never find their bytes in the 256 MiB Infinity Cache (the reference flushes
with a memset instead, runtime/kvf_host.h:302-331; a rotation keeps the flush
out of the timed region). The GPU is held behind a spin kernel while the
host enqueues all K steps, so the timed region is the GPU's own back-to-back
rate, not Python's launch rate (config.gpu_waited_for_host says whether the
GPU ever caught up with the host). K defaults to 2000 steps after 500 warm-up
steps: averaged over 400 steps, the same box reads 0.3-0.8 us more per step,
a start-up cost after the spin that more steps amortise, as a serving loop
does. HIP events bracket the K steps and, in a
second pass, the split kernel alone (the roofline's dominant kernel), bound to
its own dispatch. A third pass repeats the second with events created
without the system-scope fence (hipEventDisableSystemFence), which otherwise
ends each timed dispatch with a system-scope release; it is reported beside
the roofline (config.split_kernel_in_step_us_avg_events_without_fence).
config.reference_method_us_median times the step as the reference's harness
does (runtime/kvf_host.h:302-331): one step per rep after a cache flush,
event-timed, median of 100 reps.

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
import types

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
METRIC = ("\u00b5s/decode step + achieved HBM GB/s (% of peak), "
          "GQA32/8 d128 32k int8:64")
CONFIG_DEFAULTS = {  # config -> (fmt, group, n, order, block tokens, splits, waves)
    1: ("f16", 0, 4096, "hm", 0, 1, 4),
    2: ("int8", 64, 32768, "hm", 0, 32, 4),
    3: ("int8", 64, 8192, "tm", 16, 8, 4),
    4: ("int4", 32, 65536, "hm", 0, 32, 8),
}


def parse():
    p = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=2000)
    p.add_argument("--warmup", type=int, default=500)
    p.add_argument("--config", type=int, default=2, choices=sorted(CONFIG_DEFAULTS))
    p.add_argument("--fmt", default=None, choices=["f16", "int8", "int4"])
    p.add_argument("--group", type=int, default=None)
    p.add_argument("--n", type=int, default=None,
                   help="tokens (configs 2 and 4; config 3 draws its lengths)")
    p.add_argument("--order", default=None, choices=["hm", "tm"])
    p.add_argument("--block-tokens", type=int, default=None)
    p.add_argument("--splits", type=int, default=None)
    p.add_argument("--warps", type=int, default=None, help="wavefronts per workgroup (4 or 8)")
    p.add_argument("--unroll", type=int, default=2)
    p.add_argument("--pack", type=int, default=1)
    p.add_argument("--copies", type=int, default=0,
                   help="cache replicas rotated over steps (0: enough for 1 GiB)")
    p.add_argument("--cpu-seconds", type=float, default=12.0,
                   help="CPU baseline budget (0 skips it)")
    p.add_argument("--step", default="auto", choices=["auto", "fused", "two-launch"],
                   help="the step the headline value times: the one-launch kvf_launch_fused_variant, "
                        "the drop-in two-launch step (split kernel + merge kernel), or auto: "
                        "the faster of the two in this run (both are timed either way)")
    p.add_argument("--kv-heads", type=int, default=8, choices=[1, 2, 4, 8],
                   help="KV heads on this GPU, 4 query heads each: 8 is the whole model; 8/P is one "
                        "GPU's share when P GPUs split the heads (no exchange between them)")
    p.add_argument("--varlen-flags", type=int, default=0,
                   help="config 3: VarlenArgs flags (1: longest first)")
    p.add_argument("--json-only", action="store_true")
    a = p.parse_args()
    fmt, group, n, order, bt, splits, waves = CONFIG_DEFAULTS[a.config]
    a.warps = a.warps or waves
    a.fmt = a.fmt or fmt
    a.group = a.group if a.group is not None else group
    a.n = a.n or n
    a.order = a.order or order
    a.block_tokens = a.block_tokens if a.block_tokens is not None else bt
    a.splits = a.splits or splits
    return a


def log(*a, quiet=False):
    if not quiet:
        print(*a, file=sys.stderr, flush=True)


def build_workload(args, R, torch, np):
    """Inputs of the selected config, quantized and placed on the GPU by the
    product's own append kernel, replicated for the cache rotation."""
    host = R.host_lib()
    P = ctypes.c_void_p
    dev = torch.device("cuda:0")
    W = types.SimpleNamespace()
    W.B = 8 if args.config == 3 else 1
    if args.config == 1:  # MHA: every query head has its own KV head
        W.H, W.Hkv, W.D = 32, 32, 128
    else:
        W.H, W.Hkv, W.D = 4 * args.kv_heads, args.kv_heads, 128
    W.fmt = R.FMT_BY_NAME[args.fmt]
    W.group = args.group if W.fmt != R.FMT_F16 else 0
    W.order = R.ORD_HEAD if args.order == "hm" else R.ORD_TOKEN
    W.bt = args.block_tokens
    B, H, Hkv, D = W.B, W.H, W.Hkv, W.D
    if args.config == 3:
        lens = np.empty(B, np.int32)
        host.kvfh_varlen_lengths(B, 2048, 8192, 2, P(lens.ctypes.data))
        W.lens = lens
        W.lens_spec = "uniform(2048, 8192, 2)"
        W.n = int(lens.max())
    else:
        W.lens = None
        W.n = args.n
    n = W.n
    q = np.empty((B, H, D), np.float32)
    K = np.empty((B, Hkv, n, D), np.float32)
    V = np.empty((B, Hkv, n, D), np.float32)
    host.kvfh_make_data(B, H, Hkv, D, n, 1, P(q.ctypes.data), P(K.ctypes.data), P(V.ctypes.data))
    if args.config == 2:
        host.kvfh_inject_outliers(B, Hkv, D, n, 1001, 0.01, 8.0, P(K.ctypes.data), P(V.ctypes.data))
    W.q, W.K, W.V = q, K, V
    rb = R.row_bytes(W.fmt, D)
    mw = D // W.group if W.group else 0
    W.rb, W.mw = rb, mw
    if args.config == 3:
        pool = 4096
        mb = (W.n + W.bt - 1) // W.bt
        tbl = np.empty(B * mb, np.int32)
        used = host.kvfh_pool_table(B, P(lens.ctypes.data), W.bt, pool, 18, mb, P(tbl.ctypes.data))
        if used < 0:
            raise SystemExit("block pool too small")
        rows = pool * Hkv * W.bt
        W.table = torch.from_numpy(np.where(tbl < 0, 0, tbl).astype(np.int32)).to(dev)
        W.max_blocks = mb
    else:
        rows, W.max_blocks = R.rows_alloc(B, Hkv, n, W.bt)
        W.table = None
        if W.bt:
            tbl = np.empty(B * W.max_blocks, np.int32)
            host.kvfh_page_table(B * W.max_blocks, 18, P(tbl.ctypes.data))
            W.table = torch.from_numpy(tbl).to(dev)
    k0 = torch.zeros(rows * rb, dtype=torch.uint8, device=dev)
    v0 = torch.zeros(rows * rb, dtype=torch.uint8, device=dev)
    km0 = torch.zeros(rows * mw, dtype=torch.int32, device=dev) if mw else None
    vm0 = torch.zeros(rows * mw, dtype=torch.int32, device=dev) if mw else None
    for src, dst, dm in ((K, k0, km0), (V, v0, vm0)):
        if args.config == 3:  # each sequence appends only its own tokens into its own pages
            for b in range(B):
                L = int(lens[b])
                x = torch.from_numpy(np.ascontiguousarray(src[b, :, :L])).to(dev)
                R.quantize_place(W.fmt, W.group, D, x, 1, Hkv, L, W.order, W.bt, W.table[b],
                                 W.max_blocks, dst, dm)
        else:
            x = torch.from_numpy(src).to(dev)
            R.quantize_place(W.fmt, W.group, D, x, B, Hkv, n, W.order, W.bt, W.table,
                             W.max_blocks, dst, dm)
        del x
    torch.cuda.synchronize()
    # algorithmic bytes per step (runtime/kvf_driver.cu:51: KV payload + group meta)
    tokens = int(lens.sum()) if args.config == 3 else B * n
    W.alg_bytes = 2 * tokens * Hkv * (rb + mw * 4)
    cache_bytes = 2 * rows * (rb + mw * 4)
    W.copies = args.copies or max(4, math.ceil((1 << 30) / cache_bytes))
    W.caches = [(k0, v0, km0, vm0)]
    for _ in range(W.copies - 1):
        W.caches.append(tuple(t.clone() if t is not None else None for t in (k0, v0, km0, vm0)))
    W.G = H // Hkv if args.pack else 1
    W.vid = R.variant_id(W.fmt, W.order, W.bt > 0, W.G, args.unroll, D)
    W.qd = torch.from_numpy(q).to(dev)
    W.out = torch.zeros((B, H, D), dtype=torch.float32, device=dev)
    if args.config == 3:
        W.q16 = torch.from_numpy(q.astype(np.float16)).to(dev)
        W.out16 = torch.zeros((B, H, D), dtype=torch.float16, device=dev)
        W.lens_d = torch.from_numpy(lens).to(dev)
        W.va = R.VarlenArgs()
        W.va.seq_lens = W.lens_d.data_ptr()
        W.va.q16 = W.q16.data_ptr()
        W.va.out16 = W.out16.data_ptr()
        W.va.flags = args.varlen_flags
    else:
        W.va = None
    if args.config == 2:
        W.data = "synthetic: reference generator seed 1 + 1% outlier channels x8"
        W.workload = (f"GQA{H}/{Hkv} d{D} n{n} B{B} {args.fmt}{':' + str(W.group) if W.group else ''} "
                      f"{args.order}/{'paged:%d' % W.bt if W.bt else 'contiguous'}")
    elif args.config == 3:
        W.data = ("synthetic: reference generator seed 1, lengths U[2048, 8192] seed 2, "
                  "4096-page pool shuffled with seed 18")
        W.workload = (f"GQA{H}/{Hkv} d{D} B{B} lengths {int(lens.min())}..{int(lens.max())} "
                      f"(sum {int(lens.sum())}) {args.fmt}:{W.group} {args.order}/paged:{W.bt} "
                      f"pool 4096, f16 q/out")
    elif args.config == 1:
        W.data = "synthetic: reference generator seed 1"
        W.workload = (f"MHA{H} d{D} n{n} B{B} {args.fmt} "
                      f"{args.order}/{'paged:%d' % W.bt if W.bt else 'contiguous'}")
    else:
        W.data = "synthetic: reference generator seed 1"
        W.workload = (f"GQA{H}/{Hkv} d{D} n{n} B{B} {args.fmt}:{W.group} "
                      f"{args.order}/{'paged:%d' % W.bt if W.bt else 'contiguous'}")
    return W


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; the path shards by "
                          "(batch, kv-head) with no exchange between GPUs"}), flush=True)
        sys.exit(2)
    import numpy as np
    import torch
    from kvforge_amd import runtime as R

    q_ = args.json_only
    R.hip_lib()
    t_prep = time.perf_counter()
    W = build_workload(args, R, torch, np)
    log(f"inputs ready in {time.perf_counter() - t_prep:.1f} s", quiet=q_)
    B, H, Hkv, D, n, S = W.B, W.H, W.Hkv, W.D, W.n, args.splits
    dev = W.out.device
    copies = W.copies
    part_o = torch.zeros((B, H, S, D), dtype=torch.float32, device=dev)
    part_ml = torch.zeros((B, H, S, 2), dtype=torch.float32, device=dev)
    arg_list = [R.make_args(W.qd, k, v, km, vm, W.table, W.out, part_o, part_ml, B, H, Hkv, n, S,
                            args.warps, group=W.group, block_tokens=W.bt, max_blocks=W.max_blocks,
                            D=D)
                for (k, v, km, vm) in W.caches]
    L = R.hip_lib()
    vb = W.vid.encode()
    vid = W.vid
    st = torch.cuda.current_stream()
    sh = ctypes.c_void_p(st.cuda_stream)
    refs = [ctypes.byref(a) for a in arg_list]
    va = ctypes.byref(W.va) if W.va is not None else None
    out_t = W.out16 if W.va is not None else W.out

    if W.va is not None:
        def launch_step(i):
            return L.kvf_launch_varlen_variant(vb, refs[i % copies], va, sh)
    else:
        def launch_step(i):
            return L.kvf_launch_variant(vb, refs[i % copies], sh)

    def step(i):
        e = launch_step(i)
        if e:
            raise R.KvfError(f"decode step of {vid} failed: {e}")

    # correctness guard: the plan's output must match a single-split run
    step(0)
    torch.cuda.synchronize()
    got = out_t.float().clone()
    a1 = R.make_args(W.qd, *W.caches[0], W.table, W.out, None, None, B, H, Hkv, n, 1, 4,
                     group=W.group, block_tokens=W.bt, max_blocks=W.max_blocks, D=D)
    v1 = R.variant_id(W.fmt, W.order, W.bt > 0, W.G, 2, D)
    if W.va is not None:
        R.check(L.kvf_launch_varlen_variant(v1.encode(), ctypes.byref(a1), va, sh), "S=1 step")
    else:
        R.launch(v1, a1)
    torch.cuda.synchronize()
    ref1 = out_t.float()
    rel = float(torch.linalg.vector_norm(got - ref1) / torch.linalg.vector_norm(ref1))
    if not (rel < 2e-3 and bool(torch.isfinite(got).all())):
        raise SystemExit(f"plan {vid} S={S} disagrees with S=1: rel_l2 {rel}")

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    K_ = args.steps

    # fused path: one launch per step, split merge inside the kernel
    G = W.G
    counters = R.fused_counters(B, Hkv if G > 1 else H)
    cptr = ctypes.c_void_p(counters.data_ptr())
    cwords = counters.numel()

    def step_fused(i):
        e = L.kvf_launch_fused_variant(vb, refs[i % copies], va, cptr, cwords, sh)
        if e:
            raise R.KvfError(f"kvf_launch_fused_variant({vid}) failed: {e}")

    # the two merges fold the same partials in different orders: fp32 outputs
    # agree to 1e-5; binary16 outputs (config 3) may round a few elements to
    # neighbouring values, each at most 2^-11 relative
    agree = 1e-5 if W.va is None else 2.0 ** -11
    relf = None
    if S > 1:
        out_t.zero_()
        step_fused(0)
        torch.cuda.synchronize()
        relf = float(torch.linalg.vector_norm(got - out_t.float()) / torch.linalg.vector_norm(got))
        if not (relf < agree and int(counters.abs().sum()) == 0):
            raise SystemExit(f"fused step disagrees with the two-launch step: {relf}")
        for i in range(args.warmup):
            step_fused(i)
        torch.cuda.synchronize()

    # ---- timed region: K decode steps back to back, as a serving loop issues
    # them; the GPU is held by a spin kernel while the host enqueues ---------
    # the spin lasts about 25 ms per 400 steps, longer than the host takes to
    # enqueue them
    spin_cycles = int(1e8 * max(1.0, K_ / 400))
    host_late = {}

    def timed(fn, name):
        e_start = torch.cuda.Event(enable_timing=True)
        e_end = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        w0 = time.perf_counter()
        torch.cuda._sleep(spin_cycles)
        e_start.record(st)
        for i in range(K_):
            fn(i)
        e_end.record(st)
        starved = e_start.query()
        torch.cuda.synchronize()
        w1 = time.perf_counter()
        host_late[name] = bool(starved)
        if starved:
            log("warning: the GPU reached the timed region before the host finished "
                "enqueueing; the step time includes host launch gaps", quiet=q_)
        return e_start.elapsed_time(e_end) / K_, w1 - w0

    step2_ms, wall_2 = timed(step, "two_launch")
    fused_ms, wall_f = timed(step_fused, "fused") if S > 1 else (None, None)
    # auto: whichever of the two entry points ran faster on this GPU (both are
    # product paths; which one wins differs between boxes by a few per cent)
    headline_fused = args.step == "fused" or (args.step == "auto" and fused_ms is not None
                                              and fused_ms < step2_ms)
    if S > 1 and headline_fused:
        step_ms, wall_t = fused_ms, wall_f
        path = "kvf_launch_fused_variant (one launch, in-kernel split merge)"
    else:
        step_ms, wall_t = step2_ms, wall_2
        path = ("kvf_launch_varlen_variant" if W.va is not None else "kvf_launch_variant") + \
            (" (split kernel + merge kernel)" if S > 1 else " (one split: one kernel)")

    # ---- roofline pass: the same K steps again, each with HIP events bound
    # to its split kernel's own dispatch (the duration a kernel trace reports
    # for that kernel inside the step; the merge launch, if any, follows it as
    # in every step) ---------------------------------------------------------
    fused_now = S > 1 and headline_fused
    cnt_arg = cptr if fused_now else None

    def roofline_pass(nofence):
        kev = _KernelEvents(K_, nofence)
        torch.cuda.synchronize()
        torch.cuda._sleep(spin_cycles)
        for i in range(K_):
            e = L.kvf_launch_step_timed(vb, refs[i % copies], va, cnt_arg, cwords if fused_now else 0, sh,
                                        *kev.pair(i))
            if e:
                raise R.KvfError(f"timed step launch failed: {e}")
        torch.cuda.synchronize()
        ms = kev.elapsed_ms()
        kev.close()
        return 1e3 * sum(ms) / K_, 1e3 * statistics.median(ms)

    part_avg_us, part_med_us = roofline_pass(False)
    # the same pass with events created without the system-scope fence: an
    # event with the fence ends its dispatch with a system-scope release, so
    # these read the kernel shorter, closer to its duration in the plain
    # steps; a kernel trace cannot check them (under the profiler every
    # event-bound dispatch runs longer), so the roofline keeps the figure the
    # trace of the pass above reproduces
    nofence_avg_us, _ = roofline_pass(True)

    # persistent step (one launch, workgroups claiming (sequence, head group,
    # split) items from a queue, merge inside): checked against the fused
    # step's output, then timed as the other paths (after the roofline pass,
    # so the passes before it keep their order in a kernel trace). The grid
    # is capped at half the items, so the queue kernel runs and every
    # workgroup claims (uncapped, a step whose items all fit the resident
    # grid runs the static fused grid instead)
    persist_ms = None
    items = S * (Hkv if G > 1 else H) * B
    persist_wgs = max(1, items // 2)
    if S > 1:
        queue = R.persistent_queue()
        qptr = ctypes.c_void_p(queue.data_ptr())

        def step_persistent(i):
            e = L.kvf_launch_persistent_variant(vb, refs[i % copies], va, cptr, cwords, qptr,
                                                queue.numel(), persist_wgs, sh)
            if e:
                raise R.KvfError(f"kvf_launch_persistent_variant({vid}) failed: {e}")

        out_t.zero_()
        step_persistent(0)
        torch.cuda.synchronize()
        relp = float(torch.linalg.vector_norm(got - out_t.float()) / torch.linalg.vector_norm(got))
        if not (relp < agree and int(counters.abs().sum()) == 0 and int(queue.abs().sum()) == 0):
            raise SystemExit(f"persistent step disagrees with the two-launch step: {relp}")
        for i in range(args.warmup):
            step_persistent(i)
        persist_ms = timed(step_persistent, "persistent_queue")[0]

    # the reference's own timing method (runtime/kvf_host.h:302-331): one
    # step of the headline entry point per rep, event-timed, each after a
    # flush, median over the reps. The flush reads 1 GiB, which evicts L2 and
    # the 256 MiB MALL (the reference writes its flush buffer; a read leaves
    # no dirty lines to be written back while the step runs)
    step_ref = step_fused if headline_fused else step
    flush = torch.ones(1 << 28, dtype=torch.float32, device="cuda:0")
    sink = torch.empty((), dtype=torch.float32, device="cuda:0")
    ref_reps = 100
    rev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(ref_reps)]
    torch.cuda.synchronize()
    for i in range(ref_reps):
        torch.sum(flush, dim=0, out=sink)
        rev[i][0].record(st)
        step_ref(i)
        rev[i][1].record(st)
    torch.cuda.synchronize()
    ref_method_us = 1e3 * statistics.median(e0.elapsed_time(e1) for e0, e1 in rev)
    del flush, sink

    alg_bytes = W.alg_bytes
    achieved = alg_bytes / (part_avg_us * 1e-6) / 1e9
    traffic = _traffic_from_profiles(vid, args, W.alg_bytes)
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
        "dtype": "u8" if W.fmt == R.FMT_INT8 else ("u4" if W.fmt == R.FMT_INT4 else "f16"),
        "data": W.data,
        "config": {
            "workload": W.workload,
            "baseline_config": args.config,
            "kv_heads_on_gpu": W.Hkv,
            "plan": f"{vid} splits={S} waves={args.warps}"
                    + (f" varlen_flags={args.varlen_flags}" if W.va is not None and args.varlen_flags else ""),
            "entry_point": path,
            "two_launch_us_per_step": round(step2_ms * 1e3, 3),
            "fused_us_per_step": round(fused_ms * 1e3, 3) if fused_ms is not None else None,
            "fused_vs_two_launch_rel_l2": float(f"{relf:.3g}") if relf is not None else None,
            "persistent_queue_us_per_step": round(persist_ms * 1e3, 3) if persist_ms is not None else None,
            "persistent_queue_workgroups": f"{persist_wgs} for {items} items" if persist_ms is not None else None,
            "alg_bytes_per_step": alg_bytes,
            "step_hbm_gbs": round(alg_bytes / (step_ms * 1e-3) / 1e9, 1),
            "step_frac_of_peak": round(alg_bytes / (step_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "split_kernel_in_step_us_avg": round(part_avg_us, 3),
            "split_kernel_in_step_us_median": round(part_med_us, 3),
            "split_kernel_in_step_us_avg_events_without_fence": round(nofence_avg_us, 3),
            "reference_method_us_median": round(ref_method_us, 3),
            "reference_method": f"one step per rep after a 1 GiB read, event-timed, median of {ref_reps} "
                                "(runtime/kvf_host.h:302-331)",
            "cache_copies_rotated": copies,
            "wall_s_timed_region": round(wall_t, 4),
            "gpu_waited_for_host": host_late,
        },
        "roofline": {
            "bound": "hbm",
            "kernel": "decode_partial",
            "kernel_time": "split kernel inside the decode step: HIP events bound to its own "
                           f"dispatch in {K_} back-to-back steps, average",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "probe_peak": _probe_peak(),
            "frac_of_probe_peak": round(achieved / _probe_peak(), 4) if _probe_peak() else None,
            "traffic": traffic["hbm_bytes_per_launch"] if traffic else None,
            "traffic_source": traffic["source"] if traffic else None,
        },
        "cpu_baseline": None,
    }
    result["config"]["cost_model"] = _cost_model(args, W, S)
    if args.cpu_seconds > 0:
        result["cpu_baseline"] = _cpu_baseline(args, W, step_ms, q_)
    print(json.dumps(result), flush=True)


def _probe_peak():
    """bw_peak_gbs of machines/mi355x.gpu: the best HBM read rate the HIP
    probe measured (kvforge_amd/tools/bw_probe.hip), or None."""
    try:
        with open(os.path.join(ROOT, "machines", "mi355x.gpu")) as f:
            for line in f:
                k, _, v = line.partition("=")
                if k.strip() == "bw_peak_gbs":
                    return float(v)
    except OSError:
        pass
    return None


HIP_EVENT_DISABLE_SYSTEM_FENCE = 0x20000000  # hip_runtime_api.h


class _KernelEvents:
    """n (start, stop) HIP event pairs for binding to kernel dispatches. With
    nofence they are created with hipEventDisableSystemFence through the HIP
    runtime torch has already loaded (the one libkvf_hip.so runs on);
    otherwise they are torch's default timing events."""

    def __init__(self, n, nofence):
        import torch
        self.nofence = nofence
        if not nofence:
            self.ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                       for _ in range(n)]
            for e0, e1 in self.ev:  # torch creates an event at its first record
                e0.record()
                e1.record()
            return
        hip = ctypes.CDLL("libamdhip64.so.7", mode=os.RTLD_NOLOAD)
        hip.hipEventCreateWithFlags.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_uint]
        hip.hipEventCreateWithFlags.restype = ctypes.c_int
        hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
        hip.hipEventElapsedTime.restype = ctypes.c_int
        hip.hipEventDestroy.argtypes = [ctypes.c_void_p]
        hip.hipEventDestroy.restype = ctypes.c_int
        self.hip = hip
        self.ev = []
        for _ in range(n):
            pair = []
            for _ in range(2):
                h = ctypes.c_void_p()
                e = hip.hipEventCreateWithFlags(ctypes.byref(h), HIP_EVENT_DISABLE_SYSTEM_FENCE)
                if e:
                    raise RuntimeError(f"hipEventCreateWithFlags failed: {e}")
                pair.append(h)
            self.ev.append(tuple(pair))

    def pair(self, i):
        e0, e1 = self.ev[i]
        if self.nofence:
            return e0, e1
        return ctypes.c_void_p(e0.cuda_event), ctypes.c_void_p(e1.cuda_event)

    def elapsed_ms(self):
        if not self.nofence:
            return [e0.elapsed_time(e1) for e0, e1 in self.ev]
        out = []
        ms = ctypes.c_float()
        for e0, e1 in self.ev:
            e = self.hip.hipEventElapsedTime(ctypes.byref(ms), e0, e1)
            if e:
                raise RuntimeError(f"hipEventElapsedTime failed: {e}")
            out.append(ms.value)
        return out

    def close(self):
        if self.nofence:
            for pair in self.ev:
                for h in pair:
                    self.hip.hipEventDestroy(h)
        self.ev = []


def _traffic_from_profiles(vid, args, alg_bytes):
    """HBM bytes per launch of the split kernel for this config's benchmarked
    plan, from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE summary
    (profiles/traffic.json, scaled by the copy-kernel calibration recorded
    there), or None if no summary covers this run: another plan, split count,
    wave count or workload size. Profile-derived: the bench run itself does
    not collect counters."""
    config = args.config
    _, _, _, _, _, splits, waves = CONFIG_DEFAULTS[config]
    if args.splits != splits or args.warps != waves:
        return None
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            tab = json.load(f)
    except (OSError, ValueError):
        return None
    ent = tab.get(f"config{config}:{vid}")
    if not ent or ent.get("alg_bytes") != alg_bytes:
        return None
    return {"hbm_bytes_per_launch": ent["hbm_bytes_per_launch"],
            "source": f"profiles/traffic.json config{config}:{vid} (rocprofv3 --pmc FETCH_SIZE x "
                      f"{ent.get('fetch_scale', 2.0)} + WRITE_SIZE x {ent.get('write_scale', 1.0)}, "
                      f"{ent.get('profile', '')})"}


def _cpu_baseline(args, W, step_ms, quiet):
    """Oracle reference_attention (runtime/kvf_host.h:202-234, double precision)
    on the dequantised cache: one core, then every host core this job may use
    (the (sequence, head) pairs spread over threads, identical output)."""
    import numpy as np
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import _oracle as O
    _, kdeq = O.quantize(W.fmt, W.group, W.D, W.K)[::2]
    _, vdeq = O.quantize(W.fmt, W.group, W.D, W.V)[::2]
    threads = int(os.environ.get("OMP_NUM_THREADS") or 0) or (os.cpu_count() or 1)
    threads = max(1, min(threads, os.cpu_count() or 1))
    q = W.q
    if W.lens is not None:  # binary16 query, as the GPU consumes it
        q = q.astype(np.float16).astype(np.float32)
        one_fn = lambda: O.reference_attention_varlen(q, kdeq, vdeq, W.lens)  # noqa: E731
        all_fn = lambda: O.reference_attention_varlen_mt(q, kdeq, vdeq, W.lens, threads)  # noqa: E731
    else:
        one_fn = lambda: O.reference_attention(q, kdeq, vdeq)  # noqa: E731
        all_fn = lambda: O.reference_attention_mt(q, kdeq, vdeq, threads)  # noqa: E731

    def sample(fn, budget):
        times = []
        t_end = time.perf_counter() + budget
        while len(times) < 3 or (time.perf_counter() < t_end and len(times) < 50):
            t0 = time.perf_counter()
            fn()
            times.append(time.perf_counter() - t0)
        return statistics.median(times), len(times)

    one, n1 = sample(one_fn, args.cpu_seconds * 0.7)
    allc, na = sample(all_fn, args.cpu_seconds * 0.3)
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


def _cost_model(args, W, S):
    """The kvf planner's prediction for the benchmarked plan and its own top-1
    plan for the same shape (MI355X machine file and fitted constants), or
    None when the compiler binary is not built. A variable-length batch is
    planned on its own lengths (the same distribution and seed, capacity
    8192 per sequence)."""
    import csv
    import subprocess
    import tempfile
    kvf = os.path.join(ROOT, "kvforge_amd", "bin", "kvf")
    if not os.path.exists(kvf):
        return None
    varlen = getattr(W, "lens_spec", None) if W.lens is not None else None
    n = 8192 if varlen else W.n
    seq = f", seq_lens = {varlen}" if varlen else ""
    # (split counts past the planner's default cap of 64 only when asked for)
    cap = "target max_splits = 256\n\n" if S > 64 else ""
    spec = (f"{cap}decode bench(H: {W.H}, H_kv: {W.Hkv}, d: {W.D}, n: {n}, batch: {W.B}) {{\n"
            f"  Q: query<H, d, f32>\n  K: kvcache<n, d, ?, ?, ?>\n  V: kvcache<n, d, ?, ?, ?>\n"
            f"  O = decode_attn(Q, K, V, scale = auto, splits = ?, gqa_pack = ?{seq})\n}}\n")
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
    want = {"fmt": W.vid.split("_")[0], "group": str(W.group),
            "order": "head_major" if args.order == "hm" else "token_major",
            "residency": "paged" if W.bt else "contiguous", "block_tokens": str(W.bt),
            "splits": str(S), "gqa_pack": str(args.pack), "warps": str(args.warps),
            "unroll": str(args.unroll)}
    mine = next((r for r in rows if all(r[k] == v for k, v in want.items())), None)
    live = [r for r in rows if r["rejected"] == "0"]
    best = min(live, key=lambda r: float(r["pred_us"])) if live else None
    out = {"predicted_us_per_step": round(float(mine["pred_us"]), 3) if mine else None,
           "planned_lengths": f"{W.B} sequences, {varlen}" if varlen else f"{W.B} x {n}"}
    if best:
        out["model_top1"] = (f"{best['fmt']}:{best['group']} {best['order']}/{best['residency']} "
                             f"splits={best['splits']} pack={best['gqa_pack']} w{best['warps']} "
                             f"u{best['unroll']}")
        out["model_top1_predicted_us"] = round(float(best["pred_us"]), 3)
    return out


if __name__ == "__main__":
    main()
