"""Per-phase timeline of one decode step on the GPU, from per-wave clock stamps.

    python kvforge_amd/tools/timeline.py [--config 2] [--order hm|tm] [--steps 60] [--out FILE.md] [--raw FILE.npz]

Builds, under kvforge_amd/_build/timeline/, a copy of the library that holds
only the benchmarked plan of the chosen bench.py config, with s_memrealtime
stamps (the 100 MHz constant clock, 10 ns) written by lane 0 of every wave at
fixed points of the split kernel, and a one-launch step
(kvf_launch_fused_variant) that takes the stamp buffer from the KVF_DBG
variable. The copy is made by inserting the stamps at named places of the
kernel source; nothing else changes, so the instrumented step runs the same
code as the product's between the stamps. It then times the step back to back
(HIP events around the steps, as bench.py does), runs it once more per step
with the stamps, and reports, over the steps after the first five:

  per wave      start, first tile consumed, main loop left, drain done,
                wave combine barrier passed, combine arithmetic done,
                partials stored (write-through complete), arrival counted;
  per merging   merge entered and merge stored (the last workgroup of each
  workgroup     head group);
  per step      the span from the first wave's start to the last merge store,
                and the step time less that span: the part of a step spent
                outside any wave (dispatch, wave launch, end of kernel).

The same is done for an empty full-chip grid (one workgroup of 256 threads
per CU, each wave stamping only its start and its end), whose step time
against its span splits a kernel's fixed cost into the waves' own time and the
time around them. The output is a markdown table (--out), the raw stamps
optionally an npz (--raw).

Measurement tool: nothing in the product loads the instrumented library.
"""
import argparse
import ctypes
import os
import shutil
import subprocess
import sys
import types

HERE = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.dirname(HERE)
ROOT = os.path.dirname(PKG)
sys.path.insert(0, ROOT)
BUILD = os.path.join(PKG, "_build", "timeline")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = ["-std=c++17", "-O3", "--offload-arch=gfx950", "-fPIC", "-Xclang", "-target-feature",
         "-Xclang", "-packed-fp32-ops", "-mllvm", "-amdgpu-mfma-vgpr-form",
         "-mllvm", "-amdgpu-atomic-optimizer-strategy=None"]

# (stamp slot, name): per wave unless noted
PHASES = [(0, "wave start"), (1, "first tile consumed"), (2, "main loop left"), (9, "drain done"),
          (3, "wave combine barrier passed"), (10, "combine arithmetic done"),
          (4, "partials stored (write-through complete)"), (5, "arrival counted (atomic returned)")]
MERGE = [(6, "merge entered"), (11, "merge stored")]

_STAMP = ('{ unsigned long long t_; asm volatile("s_memrealtime %0\\n\\ts_waitcnt lgkmcnt(0)" : "=s"(t_)'
          ' : "v"(DEP) : "memory"); TS(IDX, t_); }')


def _stamp(idx, dep):
    return _STAMP.replace("IDX", str(idx)).replace("DEP", dep)


def _patches():
    """(file, anchor, replacement) edits that insert the stamps."""
    tsdef = ('  auto TS = [&](int i_, unsigned long long v_) __attribute__((always_inline)) {\n'
             '    if (x.dbg && lane == 0)\n'
             '      x.dbg[((size_t)(blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z)) * WPB +\n'
             '             (threadIdx.x >> 6)) * 16 + i_] = v_;\n'
             '  };\n')
    return [
        ("kvf_ext.hpp", "  bool dry_merge = false;\n",
         "  bool dry_merge = false;\n  unsigned long long *dbg = nullptr;\n"),
        ("kvf_runtime.hip", "  x.counters = counters;\n  return fx(*a, x, Launch{}, st);",
         "  x.counters = counters;\n"
         "  if (const char *e = std::getenv(\"KVF_DBG\")) x.dbg = (unsigned long long *)std::strtoull(e, nullptr, 10);\n"
         "  return fx(*a, x, Launch{}, st);"),
        ("kvf_kernels.hpp", "  constexpr int nw = WPB; // equals a.warps, checked at launch\n",
         "  constexpr int nw = WPB; // equals a.warps, checked at launch\n" + tsdef +
         "  " + _stamp(0, "lane") + "\n"
         # slot 7: where the wave runs (XCC_ID in the high word, HW_ID: CU, SIMD, wave slot)
         "  TS(7, ((unsigned long long)__builtin_amdgcn_s_getreg(0x1814) << 32) |\n"
         "        (unsigned)__builtin_amdgcn_s_getreg(0xF804));\n"),
        ("kvf_kernels.hpp", "        compute(ring(Ui), k, mask_tag);\n        ++k;\n      });\n    }",
         "        compute(ring(Ui), k, mask_tag);\n        if (k == 0) " + _stamp(1, "acc[0][0][0]") +
         "\n        ++k;\n      });\n    }"),
        ("kvf_kernels.hpp", "  // drain: the tiles still in flight, masked (a full tile computes the same)\n",
         "  " + _stamp(2, "acc[0][0][0]") + "\n"
         "  // drain: the tiles still in flight, masked (a full tile computes the same)\n"),
        ("kvf_kernels.hpp", "  // ---- wave result: per head (m_run, l, m_true) and O[head][D] ---------------\n",
         "  " + _stamp(9, "acc[0][0][0]") + "\n"
         "  // ---- wave result: per head (m_run, l, m_true) and O[head][D] ---------------\n"),
        ("kvf_kernels.hpp", "  // every LDS read of an output element is issued before any is used: the\n",
         "  " + _stamp(3, "lane") + "\n"
         "  // every LDS read of an output element is issued before any is used: the\n"),
        ("kvf_kernels.hpp",
         "    const int hq = G > 1 ? hkv * G + hh : hb;\n    const long long head = (long long)b * a.H + hq;\n",
         "    const int hq = G > 1 ? hkv * G + hh : hb;\n    const long long head = (long long)b * a.H + hq;\n"
         "    if (idx0 + nthreads >= G * D) " + _stamp(10, "O") + "\n"),
        ("kvf_kernels.hpp",
         "    asm volatile(\"s_waitcnt vmcnt(0)\" ::: \"memory\");\n    __syncthreads();\n"
         "    if (threadIdx.x == 0)\n"
         "      s_last = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==\n"
         "               (unsigned)(a.splits - 1);\n    __syncthreads();\n    const bool last = s_last != 0;\n",
         "    asm volatile(\"s_waitcnt vmcnt(0)\" ::: \"memory\");\n    " + _stamp(4, "lane") + "\n"
         "    __syncthreads();\n"
         "    if (threadIdx.x == 0) {\n"
         "      const unsigned old_ = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);\n"
         "      s_last = old_ == (unsigned)(a.splits - 1);\n      " + _stamp(5, "old_") + "\n    }\n"
         "    __syncthreads();\n    const bool last = s_last != 0;\n"
         "    if (last) " + _stamp(6, "lane") + "\n"),
        ("kvf_kernels.hpp",
         "    if (last && threadIdx.x == 0) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);\n",
         "    if (last) { asm volatile(\"s_waitcnt vmcnt(0)\" ::: \"memory\"); " + _stamp(11, "lane") + " }\n"
         "    if (last && threadIdx.x == 0) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);\n"),
    ]


EMPTY_SRC = r'''
#include <hip/hip_runtime.h>
__global__ void __launch_bounds__(256) stamp_only(unsigned long long *dbg) {
  unsigned long long t0, t1;
  asm volatile("s_memrealtime %0\n\ts_waitcnt lgkmcnt(0)" : "=s"(t0) :: "memory");
  asm volatile("s_memrealtime %0\n\ts_waitcnt lgkmcnt(0)" : "=s"(t1) :: "memory");
  if (dbg && (threadIdx.x & 63) == 0) {
    const size_t w = (size_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    dbg[w * 2] = t0;
    dbg[w * 2 + 1] = t1;
  }
}
extern "C" hipError_t timeline_empty(int wgs, unsigned long long *dbg, hipStream_t st) {
  hipLaunchKernelGGL(stamp_only, dim3(wgs), dim3(256), 0, st, dbg);
  return hipGetLastError();
}
'''


def build(vid, inst):
    """The instrumented library holding plan `vid` (instantiated as `inst`)
    and the empty stamping kernel; returns their paths."""
    csrc = os.path.join(BUILD, "csrc")
    os.makedirs(csrc, exist_ok=True)
    src = os.path.join(PKG, "csrc")
    files = {f: open(os.path.join(src, f)).read()
             for f in ("kvf_kernels.hpp", "kvf_ext.hpp", "kvf_runtime.hip", "kvf_merge.hip")}
    for f, old, new in _patches():
        if files[f].count(old) != 1:
            raise SystemExit(f"timeline: the stamp anchor in {f} is gone: {old[:60]!r}")
        files[f] = files[f].replace(old, new)
    for f, text in files.items():
        with open(os.path.join(csrc, f), "w") as fh:
            fh.write(text)
    with open(os.path.join(csrc, "timeline_plan.hip"), "w") as fh:
        fh.write('#include "kvf_kernels.hpp"\n'
                 f"template hipError_t kvf::launch<{inst}>(const kvf::Args &, hipStream_t);\n"
                 f"template hipError_t kvf::gfx950::launch_ext<{inst}>(const kvf::Args &, "
                 "const kvf::gfx950::Ext &, const kvf::gfx950::Launch &, hipStream_t);\n"
                 "void kvf_register_all(kvf::Registry &r) {\n"
                 f'  r.add("{vid}", &kvf::launch<{inst}>, &kvf::gfx950::launch_ext<{inst}>);\n}}\n')
    with open(os.path.join(csrc, "timeline_empty.hip"), "w") as fh:
        fh.write(EMPTY_SRC)
    objs = []
    for name in ("kvf_runtime", "kvf_merge", "timeline_plan"):
        o = os.path.join(BUILD, name + ".o")
        # kernel-argument preloading as the library's build has it
        extra = ["-mllvm", "-amdgpu-kernarg-preload-count=" + ("10" if name == "kvf_merge" else "14")]
        subprocess.run([HIPCC] + FLAGS + extra + ["-I" + csrc, "-I" + os.path.join(ROOT, "include"), "-c",
                                                  os.path.join(csrc, name + ".hip"), "-o", o], check=True)
        objs.append(o)
    lib = os.path.join(BUILD, "libkvf_timeline.so")
    subprocess.run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", lib] + objs, check=True)
    empty = os.path.join(BUILD, "libkvf_timeline_empty.so")
    subprocess.run([HIPCC] + FLAGS + ["-shared", "-o", empty, os.path.join(csrc, "timeline_empty.hip")], check=True)
    return lib, empty


def _inst(vid):
    fmt, order, res, g, u, d = vid.split("_")
    F = {"f16": "kvf::FMT_F16", "int8": "kvf::FMT_INT8", "int4": "kvf::FMT_INT4"}[fmt]
    O = "kvf::ORD_HEAD" if order == "hm" else "kvf::ORD_TOKEN"
    return f"{F}, {d[1:]}, {g[1:]}, {u[1:]}, {O}, {'true' if res == 'p' else 'false'}"


def _pct(x, q):
    import numpy as np
    x = x[~np.isnan(x)]
    return float(np.percentile(x, q)) if len(x) else float("nan")


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--config", type=int, default=2, choices=[2, 3, 4])
    ap.add_argument("--order", default=None, choices=["hm", "tm"],
                    help="KV order instead of the config's (the same data, placed the other way)")
    ap.add_argument("--steps", type=int, default=60)
    ap.add_argument("--out", default=None)
    ap.add_argument("--raw", default=None)
    a0 = ap.parse_args()
    import numpy as np
    import torch
    import bench
    from kvforge_amd import runtime as R

    fmt, group, n, order, bt, splits, waves = bench.CONFIG_DEFAULTS[a0.config]
    order = a0.order or order
    args = types.SimpleNamespace(config=a0.config, fmt=fmt, group=group, n=n, order=order, block_tokens=bt,
                                 copies=0, unroll=2, pack=1, splits=splits, warps=waves, kv_heads=8,
                                 varlen_flags=0)
    print(f"building the instrumented library ({bench.CONFIG_DEFAULTS[a0.config]})", flush=True)
    R.hip_lib()  # (bench's data path runs the product's quantizer)
    W = bench.build_workload(args, R, torch, np)
    lib_path, empty_path = build(W.vid, _inst(W.vid))
    L = ctypes.CDLL(lib_path)
    P, Z = ctypes.c_void_p, ctypes.c_size_t
    L.kvf_launch_fused_variant.restype = ctypes.c_int
    L.kvf_launch_fused_variant.argtypes = [ctypes.c_char_p, ctypes.POINTER(R.Args),
                                           ctypes.POINTER(R.VarlenArgs), P, Z, P]
    E = ctypes.CDLL(empty_path)
    E.timeline_empty.restype = ctypes.c_int
    E.timeline_empty.argtypes = [ctypes.c_int, P, P]

    dev = torch.device("cuda:0")
    S = splits
    po = torch.zeros((W.B, W.H, S, W.D), dtype=torch.float32, device=dev)
    pm = torch.zeros((W.B, W.H, S, 2), dtype=torch.float32, device=dev)
    arg_list = [R.make_args(W.qd, k, v, km, vm, W.table, W.out, po, pm, W.B, W.H, W.Hkv, W.n, S, waves,
                            group=W.group, block_tokens=W.bt, max_blocks=W.max_blocks, D=W.D)
                for (k, v, km, vm) in W.caches]
    counters = R.fused_counters(W.B, W.Hkv)
    va = ctypes.byref(W.va) if W.va is not None else None
    sh = R.stream_handle()
    nwaves = S * W.Hkv * W.B * waves
    per = nwaves * 16
    dbg = torch.zeros(per * a0.steps, dtype=torch.int64, device=dev)

    def launch(i, stamps):
        if stamps:
            os.environ["KVF_DBG"] = str(dbg.data_ptr() + i * per * 8)
        else:
            os.environ.pop("KVF_DBG", None)
        a = arg_list[i % len(arg_list)]
        e = L.kvf_launch_fused_variant(W.vid.encode(), ctypes.byref(a), va, P(counters.data_ptr()),
                                       counters.numel(), sh)
        if e:
            raise R.KvfError(f"instrumented step failed: {e}")

    def timed(fn, k):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        torch.cuda._sleep(int(2e8))
        e0.record()
        for i in range(k):
            fn(i)
        e1.record()
        torch.cuda.synchronize()
        return 1e3 * e0.elapsed_time(e1) / k  # us per step

    for i in range(50):
        launch(i, False)
    step_plain = timed(lambda i: launch(i, False), 500)
    step_stamped = timed(lambda i: launch(i, True), a0.steps)
    t = dbg.cpu().numpy().reshape(a0.steps, nwaves, 16).astype(np.int64)[5:]
    t0 = t[:, :, 0].min(1, keepdims=True)

    def rel(c):
        return np.where(t[:, :, c] > 0, (t[:, :, c] - t0) * 10.0 / 1000.0, np.nan)

    rows = []
    for c, name in PHASES:
        x = rel(c)
        rows.append((name, "every wave", _pct(x, 10), _pct(x, 50), _pct(x, 90), float(np.nanmean(np.nanmax(x, 1)))))
    merging = ~np.isnan(rel(6))
    for c, name in MERGE:
        x = np.where(merging, rel(c), np.nan)
        rows.append((name, "merging workgroups", _pct(x, 10), _pct(x, 50), _pct(x, 90),
                     float(np.nanmean(np.nanmax(x, 1)))))
    span = float(np.nanmean(np.nanmax(np.where(merging, rel(11), np.nan), 1)))

    # the empty grid: one 4-wave workgroup per CU
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    edbg = torch.zeros(cus * 4 * 2 * 40, dtype=torch.int64, device=dev)
    empty = lambda i: E.timeline_empty(cus, None, sh)  # noqa: E731
    for i in range(50):
        empty(i)
    empty_step = timed(empty, 2000)
    for i in range(40):
        E.timeline_empty(cus, P(edbg.data_ptr() + i * cus * 4 * 2 * 8), sh)
    torch.cuda.synchronize()
    et = edbg.cpu().numpy().reshape(40, cus * 4, 2).astype(np.int64)[5:]
    espan = float(np.mean((et[:, :, 1].max(1) - et[:, :, 0].min(1)) * 10.0 / 1000.0))
    estart = float(np.mean((np.percentile(et[:, :, 0], 90, axis=1) - et[:, :, 0].min(1)) * 10.0 / 1000.0))

    lines = [f"# Timeline of one decode step: {W.workload}, plan {W.vid} splits={S} waves={waves}", "",
             "Command (repository root on the GPU box):", "",
             f"    python3 kvforge_amd/tools/timeline.py --config {a0.config} --steps {a0.steps}"
             + (f" --order {a0.order}" if a0.order else "")
             + (f" --out {a0.out}" if a0.out else ""), "",
             "One-launch step (kvf_launch_fused_variant), per-wave s_memrealtime stamps (10 ns), times "
             "in us after the step's first wave started, over the steps after the first five; "
             "`max` is the average over steps of the step's latest stamp.", "",
             "| Point | Over | p10 | median | p90 | max |", "|---|---|---|---|---|---|"]
    for name, over, p10, med, p90, mx in rows:
        lines.append(f"| {name} | {over} | {p10:.2f} | {med:.2f} | {p90:.2f} | {mx:.2f} |")
    lines += ["",
              f"- Step time, back to back without stamps: **{step_plain:.2f} us**; with stamps "
              f"{step_stamped:.2f} us.",
              f"- First wave start to last merge store (stamped steps): **{span:.2f} us**; the rest of the "
              f"stamped step, {step_stamped - span:.2f} us, is spent outside every wave (dispatch, wave launch, "
              f"end of kernel).",
              f"- Empty grid ({cus} workgroups of 4 waves, each wave stamping its start and end), back to back: "
              f"**{empty_step:.2f} us** per kernel; first wave start to last wave end {espan:.2f} us "
              f"(90 % of the waves started within {estart:.2f} us), so {empty_step - espan:.2f} us of an empty "
              f"kernel's step lies outside its waves.", ""]
    text = "\n".join(lines)
    print(text, flush=True)
    if a0.out:
        with open(a0.out, "w") as fh:
            fh.write(text + "\n")
    if a0.raw:
        # t[step][wave][slot]: wave w of workgroup (split, head group, sequence)
        # = w // waves in (x, y, z) grid order; slot 7 holds XCC_ID << 32 | HW_ID
        np.savez_compressed(a0.raw, t=t, empty=et, grid=np.array([S, W.Hkv, W.B, waves]))


if __name__ == "__main__":
    main()
