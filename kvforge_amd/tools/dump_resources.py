"""Register, scratch and LDS use of every gfx950 split kernel, for the CDNA
cost model's occupancy terms (the reference reads the same facts out of its
CUDA binary with tools/dump_resources.py; here hipcc's resource-usage remarks
report them for the code objects this repository builds).

    python kvforge_amd/tools/dump_resources.py [--jobs 8] [--out machines/resources_gfx950.csv]

Compiles every explicit-instantiation source under kvforge_amd/csrc/gen with
-Rpass-analysis=kernel-resource-usage (objects go to a temporary directory)
and writes one CSV row per decode_partial instantiation:

    fmt,d,group,g,u,ord,paged,waves,vgpr,agpr,sgpr,scratch,occupancy

fmt/ord use the kernels' numbering (f16 0, int8 1, int4 2; head-major 0,
token-major 1); `group` is the quantisation group the kernel is built for (the
head dimension for f16), `g` the GQA pack, `u` the unroll knob, `waves` the
wavefronts per workgroup; `occupancy` is the compiler's waves per SIMD.
"""
import argparse
import concurrent.futures as cf
import glob
import os
import re
import subprocess
import sys
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.dirname(HERE)
ROOT = os.path.dirname(PKG)
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = ["-std=c++17", "-O3", "--offload-arch=gfx950", "-fPIC", "-Xclang", "-target-feature",
         "-Xclang", "-packed-fp32-ops", "-mllvm", "-amdgpu-mfma-vgpr-form",
         "-I" + os.path.join(ROOT, "include"),
         "-I" + os.path.join(PKG, "csrc"), "-Rpass-analysis=kernel-resource-usage"]
NAME = re.compile(r"decode_partialILi(\d+)ELi(\d+)ELi(\d+)ELi(\d+)ELi(\d+)ELi(\d+)ELb(\d)ELi(\d+)E")
REMARK = re.compile(r"remark: (.*?) \[-Rpass-analysis")


def remarks(src, tmp):
    obj = os.path.join(tmp, os.path.basename(src) + ".o")
    p = subprocess.run([HIPCC, *FLAGS, "-c", src, "-o", obj], capture_output=True, text=True)
    if p.returncode != 0:
        raise RuntimeError(f"{src}: {p.stderr[-2000:]}")
    rows, cur = [], None
    for line in p.stderr.splitlines():
        m = REMARK.search(line)
        if not m:
            continue
        text = m.group(1)
        if text.startswith("Function Name:"):
            cur = {"name": text.split(":", 1)[1].strip()}
            rows.append(cur)
        elif cur is not None and ":" in text:
            k, v = text.split(":", 1)
            cur[k.strip()] = v.strip()
    return rows


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=8)
    ap.add_argument("--out", default=os.path.join(ROOT, "machines", "resources_gfx950.csv"))
    args = ap.parse_args()
    srcs = sorted(glob.glob(os.path.join(PKG, "csrc", "gen", "kvf_inst_*.hip")))
    if not srcs:
        sys.exit("no instantiation sources under kvforge_amd/csrc/gen")
    table = {}
    with tempfile.TemporaryDirectory() as tmp, cf.ThreadPoolExecutor(args.jobs) as pool:
        for rows in pool.map(lambda s: remarks(s, tmp), srcs):
            for r in rows:
                m = NAME.search(r["name"])
                if not m:
                    continue
                fmt, d, group, g, u, ord_, paged, waves = (int(x) for x in m.groups())
                table[(fmt, d, group, g, u, ord_, paged, waves)] = (
                    int(r["VGPRs"]), int(r["AGPRs"]), int(r["TotalSGPRs"]),
                    int(r["ScratchSize [bytes/lane]"]), int(r["Occupancy [waves/SIMD]"]))
    with open(args.out, "w") as f:
        f.write("fmt,d,group,g,u,ord,paged,waves,vgpr,agpr,sgpr,scratch,occupancy\n")
        for k in sorted(table):
            f.write(",".join(str(x) for x in (*k, *table[k])) + "\n")
    print(f"wrote {len(table)} kernels to {args.out}")


if __name__ == "__main__":
    main()
