"""Register, scratch and LDS use of every gfx950 split kernel, for the CDNA
cost model's occupancy terms (the reference reads the same facts out of its
CUDA binary with tools/dump_resources.py; here hipcc's resource-usage remarks
report them for the code objects this repository builds).

    python kvforge_amd/tools/dump_resources.py [--jobs 8] [--out machines/resources_gfx950.csv]

Compiles every explicit-instantiation source under kvforge_amd/csrc/gen with
-Rpass-analysis=kernel-resource-usage (objects go to a temporary directory)
and writes one CSV row per decode_partial instantiation:

    fmt,d,group,g,u,ord,paged,waves,vgpr,agpr,sgpr,scratch,occupancy,valu,mfma,lds,salu

fmt/ord use the kernels' numbering (f16 0, int8 1, int4 2; head-major 0,
token-major 1); `group` is the quantisation group the kernel is built for (the
head dimension for f16), `g` the GQA pack, `u` the unroll knob, `waves` the
wavefronts per workgroup; `occupancy` is the compiler's waves per SIMD.

valu, mfma, lds, salu: instructions per 32-token tile of the kernel's main
loop, counted in the gfx950 assembly of the same compile (-S): the loop is
the one holding the most MFMAs in its own blocks (the main loop comes in a
masked and an unmasked copy, one for chunks that start inside a tile; the
unmasked one, with fewer vector instructions, is taken); its blocks hold the
tile's compute once per unrolled step, so the counts are divided by (MFMAs
in the loop / MFMAs per tile). MFMAs per
tile follow from the kernel's column geometry: COLS = g x (d / group) query
columns (g for f16), two passes when COLS > 16, hi and lo in one MFMA when
COLS <= 8, and per pass and binary16 half 2 x d/32 QK steps plus d/16 PV
steps. `lds` counts ds_* instructions (the cross-row shuffles), `salu` s_*.
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
         "-mllvm", "-amdgpu-atomic-optimizer-strategy=None", "-mllvm", "-amdgpu-kernarg-preload-count=14",
         "-I" + os.path.join(ROOT, "include"),
         "-I" + os.path.join(PKG, "csrc"), "-Rpass-analysis=kernel-resource-usage"]
NAME = re.compile(r"decode_partialILi(\d+)ELi(\d+)ELi(\d+)ELi(\d+)ELi(\d+)ELi(\d+)ELb(\d)ELi(\d+)E")
REMARK = re.compile(r"remark: (.*?) \[-Rpass-analysis")


LABEL = re.compile(r"^(_Z\w+):")
BLOCK = re.compile(r"^(\.LBB\d+_\d+):(.*)")
BB = re.compile(r"^; (%bb\.\d+):(.*)")
IN_LOOP = re.compile(r"Header=BB(\d+_\d+) Depth=\d+")


def mfma_per_tile(fmt, d, group, g):
    cols = g * (d // group if fmt != 0 else 1)
    passes = 2 if cols > 16 else 1
    nq = 1 if cols <= 8 else 2
    return (2 * (d // 32) + d // 16) * nq * passes


def loop_mix(lines):
    """Instruction mix of the loop with the most MFMAs in its own blocks (the
    fewest vector instructions breaking a tie). A
    block (a `.LBB` label or an unlabelled `; %bb.N:` fall-through) counts for
    the innermost loop holding it, as the assembler's comments on the block's
    first lines name it ("Loop Header: Depth=d" for a header, "in Loop:
    Header=BBx_y" for the others)."""
    blocks, notes, order = {}, {}, []
    cur, head = None, False
    for line in lines:
        m = BLOCK.match(line) or BB.match(line)
        if m:
            cur = m.group(1)
            blocks[cur], notes[cur], head = [], m.group(2), True
            order.append(cur)
            continue
        t = line.strip()
        if cur is None or not t:
            continue
        if t[0] == ";":
            if head:
                notes[cur] += " " + t
            continue
        head = False
        if t[0] != ".":
            blocks[cur].append(t.split()[0])
    loops = {}
    for b in order:
        if "Loop Header: Depth=" in notes[b]:
            owner = "BB" + b[len(".LBB"):] if b.startswith(".LBB") else b
        else:
            h = IN_LOOP.search(notes[b])
            owner = "BB" + h.group(1) if h else None
        if owner:
            loops.setdefault(owner, []).extend(blocks[b])
    if not loops:
        return None
    # of several loops with that many MFMAs (the main loop's masked and
    # unmasked copies), the one with the fewest vector ALU instructions: the
    # unmasked copy, which every chunk starting on a tile boundary runs
    ops = max(loops.values(), key=lambda o: (sum(x.startswith("v_mfma") for x in o),
                                             -sum(x.startswith("v_") for x in o)))
    mix = {"mfma": 0, "valu": 0, "lds": 0, "salu": 0}
    for op in ops:
        if op.startswith("v_mfma"):
            mix["mfma"] += 1
        elif op.startswith("v_"):
            mix["valu"] += 1
        elif op.startswith("ds_"):
            mix["lds"] += 1
        elif op.startswith("s_"):
            mix["salu"] += 1
    return mix


def kernel_mixes(asm):
    """{mangled decode_partial name: loop mix} of one assembly file."""
    out, name, lines = {}, None, []
    for line in asm.splitlines():
        if name is None:
            m = LABEL.match(line)
            if m and NAME.search(m.group(1)):
                name, lines = m.group(1), []
        elif line.startswith(".Lfunc_end"):
            out[name] = loop_mix(lines)
            name = None
        else:
            lines.append(line)
    return out


def remarks(src, tmp):
    asm = os.path.join(tmp, os.path.basename(src) + ".s")
    p = subprocess.run([HIPCC, *FLAGS, "--cuda-device-only", "-S", src, "-o", asm], capture_output=True,
                       text=True)
    if p.returncode != 0:
        raise RuntimeError(f"{src}: {p.stderr[-2000:]}")
    with open(asm) as fh:
        mixes = kernel_mixes(fh.read())
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
    for r in rows:
        r["mix"] = mixes.get(r["name"])
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
                mix = r["mix"]
                if not mix or mix["mfma"] == 0:
                    sys.exit(f"no MFMA loop found in {r['name']}")
                copies = mix["mfma"] / mfma_per_tile(fmt, d, group, g)
                if copies != int(copies):
                    sys.exit(f"{r['name']}: {mix['mfma']} loop MFMAs is no whole number of tiles")
                per_tile = tuple(round(mix[k] / copies, 1) for k in ("valu", "mfma", "lds", "salu"))
                table[(fmt, d, group, g, u, ord_, paged, waves)] = (
                    int(r["VGPRs"]), int(r["AGPRs"]), int(r["TotalSGPRs"]),
                    int(r["ScratchSize [bytes/lane]"]), int(r["Occupancy [waves/SIMD]"]), *per_tile)
    with open(args.out, "w") as f:
        f.write("fmt,d,group,g,u,ord,paged,waves,vgpr,agpr,sgpr,scratch,occupancy,valu,mfma,lds,salu\n")
        for k in sorted(table):
            f.write(",".join(str(x) for x in (*k, *table[k])) + "\n")
    print(f"wrote {len(table)} kernels to {args.out}")


if __name__ == "__main__":
    main()
