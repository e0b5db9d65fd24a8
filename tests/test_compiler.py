"""The kvf compiler (kvforge_amd/bin/kvf) against the reference's own outputs.

Golden data (tests/golden/compiler, copied by tests/golden/make_fixtures.py):
plans.csv of the four edge shapes (results/edge/*), the full prediction table
of the reference's RTX 5060 sweep under its fitted constants, and the
constants plus the report that calibrating on that sweep produced. Front-end
behaviour follows the reference's tests/smoke.ps1: the semantic checks and
the nine rejection messages. Where the reference compiler has been built
from its sources (oracle/_ref/kvf_ref), further programs are compared with it
byte for byte.
"""
import gzip
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
KVF = os.path.join(ROOT, "kvforge_amd", "bin", "kvf")
REF = os.path.join(ROOT, "oracle", "_ref", "kvf_ref")
GOLD = os.path.join(ROOT, "tests", "golden", "compiler")
GEN = os.path.join(ROOT, "kvforge_amd", "csrc", "gen")


@pytest.fixture(scope="module", autouse=True)
def _built():
    subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "kvforge_amd"), KVF], check=True)


def kvf(*args, cwd=None, exe=KVF):
    return subprocess.run([exe, *args], cwd=cwd, capture_output=True, text=True)


def spec(name, H, Hkv, d, n, batch=1, fmt="?", order="?", res="?", splits="?", pack="?",
         targets=()):
    lines = list(targets)
    lines.append(f"decode {name}(H: {H}, H_kv: {Hkv}, d: {d}, n: {n}, batch: {batch}) {{")
    lines.append("  Q: query<H, d, f32>")
    lines.append(f"  K: kvcache<n, d, {fmt}, {order}, {res}>")
    lines.append(f"  V: kvcache<n, d, {fmt}, {order}, {res}>")
    lines.append(f"  O = decode_attn(Q, K, V, scale = auto, splits = {splits}, gqa_pack = {pack})")
    lines.append("}")
    return "\n".join(lines) + "\n"


def write(tmp_path, name, text):
    p = tmp_path / name
    p.write_text(text)
    return str(p)


def machine(name):
    return os.path.join(GOLD, name)


# ---------------------------------------------------------------- golden plans
# the reference's tests/edge/*.kv shapes (rtx5060 machine, lossy formats on)
EDGE = {
    "edge_g8_n3333": (16, 2, 64, 3333, 3),
    "edge_n129": (32, 8, 128, 129, 1),
    "edge_odd_n": (12, 4, 128, 1001, 2),
    "edge_short": (8, 8, 64, 100, 1),
}


@pytest.mark.parametrize("name", sorted(EDGE))
def test_edge_plans_csv_matches_reference(tmp_path, name):
    H, Hkv, d, n, b = EDGE[name]
    src = write(tmp_path, f"{name}.kv", spec(
        name, H, Hkv, d, n, b,
        targets=[f'target machine = "{machine("rtx5060-laptop.gpu")}"',
                 "target include_quantized = 1"]))
    r = kvf("plan", src, "--out", str(tmp_path / "out"), "--top", "3")
    assert r.returncode == 0, r.stderr
    got = (tmp_path / "out" / "plans.csv").read_bytes()
    want = open(os.path.join(GOLD, f"{name}_plans.csv"), "rb").read()
    assert got == want


def test_predict_matches_reference_table(tmp_path):
    sweep = tmp_path / "sweep.csv"
    sweep.write_bytes(gzip.open(os.path.join(GOLD, "sweep_rtx5060-laptop.csv.gz")).read())
    out = tmp_path / "pred.csv"
    r = kvf("predict", "--sweep", str(sweep), "--machine", machine("rtx5060-laptop.gpu"),
            "--calib", os.path.join(GOLD, "constants_rtx5060.cal"), "--out", str(out))
    assert r.returncode == 0, r.stderr
    want = gzip.open(os.path.join(GOLD, "predicted_full_rtx5060-laptop.csv.gz")).read()
    assert out.read_bytes() == want


def test_calibrate_reproduces_reference_constants(tmp_path):
    sweep = tmp_path / "sweep.csv"
    sweep.write_bytes(gzip.open(os.path.join(GOLD, "sweep_rtx5060-laptop.csv.gz")).read())
    cal = tmp_path / "fit.cal"
    r = kvf("calibrate", "--sweep", str(sweep), "--machine", machine("rtx5060-laptop.gpu"),
            "--out", str(cal))
    assert r.returncode == 0, r.stderr
    assert cal.read_text() == open(os.path.join(GOLD, "constants_rtx5060.cal")).read()
    # the printed report (fitted constants, then metrics on the fitted and the
    # held-out shapes) is the reference's too
    want = open(os.path.join(GOLD, "calibrate_rtx5060.txt"), encoding="utf-8-sig").read()
    assert r.stdout == want.replace("\r\n", "\n")


# ---------------------------------------------------------------- front end
GEN_HDR = f'target machine = "{os.path.join(GOLD, "generic-gpu.gpu")}"'


def test_pinned_splits_honoured_with_pack_free(tmp_path):
    src = write(tmp_path, "p.kv", spec("served_gqa", 32, 8, 128, 8192, 8, fmt="f16",
                                       splits=4, targets=[GEN_HDR]))
    r = kvf("plan", src, "--out", str(tmp_path / "o"), "--top", "400")
    assert r.returncode == 0, r.stderr
    assert "splits=4" in r.stdout and "splits=1 " not in r.stdout and "splits=8" not in r.stdout
    rows = (tmp_path / "o" / "plans.csv").read_text().splitlines()[1:]
    assert rows and all(row.split(",")[11] == "4" for row in rows)
    assert {row.split(",")[12] for row in rows} == {"0", "1"}


def test_accuracy_limit_keeps_int4_out(tmp_path):
    src = write(tmp_path, "l.kv", spec("llama3_8b", 32, 8, 128, 32768, targets=[GEN_HDR]))
    r = kvf("plan", src, "--out", str(tmp_path / "o"), "--max-err", "0.02", "--top", "3")
    assert r.returncode == 0, r.stderr
    chosen = [ln for ln in r.stdout.splitlines() if ln.strip().startswith("format:")][0]
    assert "int8" in chosen


def test_lossy_formats_excluded_by_default(tmp_path):
    src = write(tmp_path, "p.kv", spec("served_gqa", 32, 8, 128, 8192, 8, fmt="f16",
                                       splits=4, targets=[GEN_HDR]))
    r = kvf("plan", src, "--out", str(tmp_path / "o"), "--top", "3")
    assert r.returncode == 0 and "lossy formats excluded" in r.stdout


def _body(H, Hkv, d, kfmt="f16", vfmt=None, kshape="n, d", extra="", v="V"):
    vfmt = vfmt or kfmt
    return (f"decode bad(H: {H}, H_kv: {Hkv}, d: {d}, n: 1024) {{ Q: query<H, d, f32> "
            f"K: kvcache<{kshape}, {kfmt}> V: kvcache<n, d, {vfmt}> "
            f"O = decode_attn(Q, K, {v}{extra}) }}")


TM = "token_major, contiguous"
REJECT = [
    ("h_multiple", GEN_HDR + "\n" + _body(30, 8, 128, f"f16, {TM}"), "multiple of H_kv"),
    ("typo_key", "target bw_peek_gbs = 40\n" + _body(8, 8, 128, f"f16, {TM}"), "unknown machine key"),
    ("format_name", GEN_HDR + "\n" + _body(8, 8, 128, f"fp16, {TM}"), "unknown KV format"),
    ("cache_shape", GEN_HDR + "\n" + _body(8, 8, 128, f"f16, {TM}", kshape="n, 64"), "cache shape"),
    ("free_mismatch", GEN_HDR + "\n" + _body(8, 8, 128, f"f16, {TM}", vfmt="?, ?, ?"),
     "both pin a format"),
    ("undeclared", GEN_HDR + "\n" + _body(8, 8, 128, f"f16, {TM}", v="W"), "not declared"),
    ("head_dim", GEN_HDR + "\n" + _body(8, 8, 96, f"f16, {TM}"), "d = 64 or d = 128"),
    ("group_divides", GEN_HDR + "\n" + _body(8, 8, 64, f"int8:128, {TM}"), "divide d"),
    ("pack_group", GEN_HDR + "\n" + _body(24, 8, 128, f"f16, {TM}", extra=", gqa_pack = true"),
     "gqa_pack = true needs"),
]


@pytest.mark.parametrize("case,text,needle", REJECT, ids=[c[0] for c in REJECT])
def test_rejections(tmp_path, case, text, needle):
    r = kvf("plan", write(tmp_path, f"{case}.kv", text), "--out", str(tmp_path / "o"))
    assert r.returncode != 0
    assert needle in r.stderr, r.stderr


def test_syntax_errors_name_the_position(tmp_path):
    r = kvf("plan", write(tmp_path, "s.kv", "decode x(H: 8, H_kv: 8, d: 128 n: 4) {}"))
    assert r.returncode == 1 and "parse:1:" in r.stderr
    r = kvf("plan", write(tmp_path, "t.kv", "decode x(H: 8, H_kv: 8, d: 128, n: 4) { Q: query<H, d, f32> $ }"))
    assert r.returncode == 1 and "lex:1:" in r.stderr


def test_machine_files_load():
    for f in ("generic-gpu.gpu", "rtx5060-laptop.gpu", "rtx4060-laptop.gpu"):
        r = kvf("machine", machine(f))
        assert r.returncode == 0 and "cost model     = warp" in r.stdout
    r = kvf("machine", os.path.join(ROOT, "machines", "mi355x.gpu"))
    assert r.returncode == 0 and "cost model     = cdna" in r.stdout and "sms = 256" in r.stdout


# ---------------------------------------------------------------- against the built reference
REF_PROGRAMS = {
    "llama3_gate": (spec("llama3_8b", 32, 8, 128, 32768, targets=[GEN_HDR, "target max_rel_err = 0.02"]), []),
    "mha_budget": (spec("mha_4k", 32, 32, 128, 4096, targets=[GEN_HDR, "target max_rel_err = 0.1"]), []),
    "pinned": (spec("baseline_fp16", 32, 8, 128, 32768, fmt="f16", order="token_major", res="contiguous",
                    splits=1, pack="false", targets=[GEN_HDR]), []),
    "paged_long": (spec("long_ctx", 32, 8, 128, 65536, fmt="int4:32", order="head_major", res="paged:16",
                        targets=[f'target machine = "{machine("rtx4060-laptop.gpu")}"',
                                 "target max_splits = 256"]), []),
    "overrides": (spec("tweak", 64, 8, 64, 20000, 3, targets=[GEN_HDR, "target sms = 20",
                                                               "target include_quantized = 1"]),
                  ["--calib", os.path.join(GOLD, "constants_rtx5060.cal")]),
}


@pytest.mark.skipif(not os.path.exists(REF), reason="reference compiler not built (oracle/_ref)")
@pytest.mark.parametrize("name", sorted(REF_PROGRAMS))
def test_plans_csv_matches_built_reference(tmp_path, name):
    text, extra = REF_PROGRAMS[name]
    src = write(tmp_path, f"{name}.kv", text)
    a = kvf("plan", src, "--out", str(tmp_path / "ours"), *extra)
    b = kvf("plan", src, "--out", str(tmp_path / "ref"), *extra, exe=REF)
    assert a.returncode == 0 and b.returncode == 0, (a.stderr, b.stderr)
    assert (tmp_path / "ours" / "plans.csv").read_bytes() == (tmp_path / "ref" / "plans.csv").read_bytes()
    hdr_ours = (tmp_path / "ours" / "plan_info.h").read_text()
    hdr_ref = (tmp_path / "ref" / "plan_info.h").read_text()
    assert hdr_ours == hdr_ref


# ---------------------------------------------------------------- code generation
def test_emit_dispatch_reproduces_library_sources(tmp_path):
    r = kvf("emit-dispatch", "--out", str(tmp_path), "--d", "128,64", "--g", "1,2,4,8")
    assert r.returncode == 0, r.stderr
    ours = sorted(os.listdir(tmp_path))
    assert ours == sorted(os.listdir(GEN))
    for f in ours:
        assert (tmp_path / f).read_text() == open(os.path.join(GEN, f)).read(), f


def test_plan_emits_hip_launcher(tmp_path):
    src = write(tmp_path, "ns.kv", spec(
        "north_star", 32, 8, 128, 32768, fmt="int8:64", order="head_major", res="contiguous",
        targets=[f'target machine = "{os.path.join(ROOT, "machines", "mi355x.gpu")}"']))
    r = kvf("plan", src, "--out", str(tmp_path / "o"))
    assert r.returncode == 0, r.stderr
    tu = (tmp_path / "o" / "decode_north_star.hip").read_text()
    assert 'extern "C" hipError_t kvf_launch_north_star(const kvf::Args *in, hipStream_t st)' in tu
    assert 'extern "C" const char *kvf_plan_north_star()' in tu
    assert "a.group_shift = 6;" in tu and "kvf::launch<kvf::FMT_INT8, 128," in tu
    assert "cuda" not in tu.lower()
    plan = [ln for ln in tu.splitlines() if ln.startswith("// plan: ")][0][len("// plan: "):]
    assert f'return "{plan}";' in tu


HIPCC = "/opt/rocm/bin/hipcc"


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not installed")
def test_generated_launcher_compiles_for_gfx950(tmp_path):
    src = write(tmp_path, "pg.kv", spec(
        "paged_tm", 32, 8, 128, 8192, 8, fmt="int4:32", order="token_major", res="paged:16",
        targets=[f'target machine = "{os.path.join(ROOT, "machines", "mi355x.gpu")}"']))
    r = kvf("plan", src, "--out", str(tmp_path / "o"))
    assert r.returncode == 0, r.stderr
    obj = tmp_path / "o" / "tu.o"
    c = subprocess.run([HIPCC, "-std=c++17", "-O3", "--offload-arch=gfx950", "-fPIC",
                        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
                        "-I", os.path.join(ROOT, "include"),
                        "-I", os.path.join(ROOT, "kvforge_amd", "csrc"),
                        "-c", str(tmp_path / "o" / "decode_paged_tm.hip"), "-o", str(obj)],
                       capture_output=True, text=True)
    assert c.returncode == 0, c.stderr[-2000:]
    syms = subprocess.run(["nm", str(obj)], capture_output=True, text=True).stdout
    assert " T kvf_launch_paged_tm" in syms and " T kvf_plan_paged_tm" in syms


# ------------------------------------------------- MI355X model against its sweep
def _evaluate(tmp_path, *extra):
    sweep = tmp_path / "sweep.csv"
    with gzip.open(os.path.join(ROOT, "kvforge_amd", "model", "sweep_mi355x.csv.gz"), "rb") as f:
        sweep.write_bytes(f.read())
    r = kvf("evaluate", "--sweep", str(sweep), "--machine", os.path.join(ROOT, "machines", "mi355x.gpu"),
            "--calib", os.path.join(ROOT, "kvforge_amd", "model", "constants_mi355x.cal"), *extra)
    assert r.returncode == 0, r.stderr
    return r.stdout


def _block(text, header):
    out = text.split(header, 1)[1]
    return out.split("\n\n", 1)[0]


def test_mi355x_model_top1_against_measured_sweep(tmp_path):
    # the committed constants against the committed MI355X sweep (every plan of
    # 12 uniform shapes timed on the GPU with the kernels of the same commit):
    # with every format allowed the model's top-1 is on average within 4 % of
    # the measured best and never 9 % away (the worst is the 14 us MHA d64
    # batch-2 shape at 8.0 %, where unroll 4 is ranked above unroll 2; the next
    # two are 7.5 and 5.9 %); among f16 and int8 plans the mean is 0.6 % and the
    # worst 2.3 %; and the north star's int8:64 pick is the measured best (the
    # north star asks for 10 %)
    text = _evaluate(tmp_path, "--which", "all")
    blk = _block(text, "no accuracy limit")
    regret_max = float(blk.split("regret max")[1].split("%")[0])
    regret_mean = float(blk.split("regret mean")[1].split("%")[0])
    assert regret_mean < 4.0 and regret_max < 9.0, blk
    worst = sorted(float(ln.split("regret=")[1].split("%")[0]) for ln in blk.splitlines() if "regret=" in ln)
    assert worst[-2] < 8.0, blk
    blk8 = _block(text, "accuracy limit 0.02")
    assert float(blk8.split("regret mean")[1].split("%")[0]) < 1.5, blk8
    assert float(blk8.split("regret max")[1].split("%")[0]) < 7.0, blk8
    # issue-bound int4 plans: the model picks 8 waves where the sweep measured them fastest
    ns = [ln for ln in blk.splitlines() if "H32_Hkv8_d128_n65536_b1" in ln][0]
    assert "int4:" in ns and " w8 " in ns, ns
    text8 = _evaluate(tmp_path, "--which", "all", "--only", "int8:64")
    ns8 = [ln for ln in text8.splitlines() if "H32_Hkv8_d128_n32768_b1" in ln][0]
    assert float(ns8.split("regret=")[1].split("%")[0]) < 1.0, ns8
    assert "splits=32 pack w4" in ns8, ns8


def test_mi355x_model_on_the_mixed_shape_sweep(tmp_path):
    # the mixed-shape sweep (every plan of the log-uniform GQA 64/8 B16 batch,
    # of GQA-4 d64 B4 and of config 3's paged batch, timed on the GPU with
    # their own per-sequence lengths): the committed constants pick config 3's
    # measured best; every f16 and int8 pick is the measured best, and with
    # int4 allowed the worst is the log-uniform batch's int4:128 pick with
    # unroll 4 ranked above unroll 2 (10.8 %)
    sweep = tmp_path / "mixed.csv"
    with gzip.open(os.path.join(ROOT, "kvforge_amd", "model", "sweep_mixed_mi355x.csv.gz"), "rb") as f:
        sweep.write_bytes(f.read())
    r = kvf("evaluate", "--sweep", str(sweep), "--machine", os.path.join(ROOT, "machines", "mi355x.gpu"),
            "--calib", os.path.join(ROOT, "kvforge_amd", "model", "constants_mi355x.cal"), "--which", "all")
    assert r.returncode == 0, r.stderr
    for header in ("lossless only", "accuracy limit", "no accuracy limit"):
        blk = _block(r.stdout, header)
        lines = [ln for ln in blk.splitlines() if "regret=" in ln]
        assert len(lines) == (2 if header == "lossless only" else 3), blk
        bound = 11.0 if header == "no accuracy limit" else 1.0
        for ln in lines:
            assert float(ln.split("regret=")[1].split("%")[0]) < bound, ln
        c3 = [ln for ln in lines if "_b8_uniform-2048-8192-2" in ln]
        if c3:
            assert "regret=0%" in c3[0] and "token_major/paged:16 | splits=8 pack" in c3[0], c3[0]


def test_mi355x_model_on_the_head_share_sweep(tmp_path):
    # every plan (splits up to 256) of one GPU's share of GQA 32/8 d128 at 32k
    # tokens when 2, 4 or 8 GPUs split the KV heads, timed on the GPU: the
    # committed constants stay within 6 % of the measured best in every
    # accuracy class, and pick a split count that fills the chip as the
    # measured best does (64 for 4 KV heads, 128 for 2, 128 or 256 for 1: the
    # one-head share measures best at 128 in f16 and at 256 in int8 and int4)
    sweep = tmp_path / "shares.csv"
    with gzip.open(os.path.join(ROOT, "kvforge_amd", "model", "sweep_shares_mi355x.csv.gz"), "rb") as f:
        sweep.write_bytes(f.read())
    r = kvf("evaluate", "--sweep", str(sweep), "--machine", os.path.join(ROOT, "machines", "mi355x.gpu"),
            "--calib", os.path.join(ROOT, "kvforge_amd", "model", "constants_mi355x.cal"), "--which", "all")
    assert r.returncode == 0, r.stderr
    want = {"H16_Hkv4": (64,), "H8_Hkv2": (128,), "H4_Hkv1": (128, 256)}
    for header in ("lossless only", "accuracy limit", "no accuracy limit"):
        lines = [ln for ln in _block(r.stdout, header).splitlines() if "regret=" in ln]
        assert len(lines) == 3, header
        for ln in lines:
            assert float(ln.split("regret=")[1].split("%")[0]) < 6.0, ln
            shape = ln.split()[0].rsplit("_d128", 1)[0]
            assert any(f"splits={w} " in ln for w in want[shape]), ln


# ------------------------------------- extension: f16 query and per-sequence lengths
def _ext_program(dtype="f16", seq="true"):
    return (f'target machine = "{os.path.join(ROOT, "machines", "mi355x.gpu")}"\n'
            "decode pool(H: 32, H_kv: 8, d: 128, n: 8192, batch: 8) {\n"
            f"  Q: query<H, d, {dtype}>\n"
            "  K: kvcache<n, d, int8:64, token_major, paged:16>\n"
            "  V: kvcache<n, d, int8:64, token_major, paged:16>\n"
            f"  O = decode_attn(Q, K, V, scale = auto, splits = 8, gqa_pack = true, seq_lens = {seq})\n"
            "}\n")


def test_f16_query_and_seq_lens_emit_varlen_launcher(tmp_path):
    r = kvf("plan", write(tmp_path, "pool.kv", _ext_program()), "--out", str(tmp_path / "o"))
    assert r.returncode == 0, r.stderr
    tu = (tmp_path / "o" / "decode_pool.hip").read_text()
    assert ('extern "C" hipError_t kvf_launch_varlen_pool(const kvf::Args *in, '
            'const kvf_varlen_args_t *va, hipStream_t st)') in tu
    assert "if (!va->seq_lens) return hipErrorInvalidValue;" in tu
    assert "if (!va->q16 || !va->out16) return hipErrorInvalidValue;" in tu
    assert "x.seq_lens = va->seq_lens;" in tu and "x.out16 = static_cast<_Float16 *>(va->out16);" in tu
    assert "kvf::gfx950::launch_ext<kvf::FMT_INT8, 128, 4, " in tu
    # the reference's launcher stays, unchanged
    assert 'extern "C" hipError_t kvf_launch_pool(const kvf::Args *in, hipStream_t st)' in tu
    hdr = (tmp_path / "o" / "plan_info.h").read_text()
    assert "#define KVF_LAUNCH_VARLEN kvf_launch_varlen_pool" in hdr
    assert "#define KVF_SEQ_LENS 1" in hdr and "#define KVF_Q_F16 1" in hdr
    ir = (tmp_path / "o" / "ir.txt").read_text()
    assert "tensor<32x128xf16>" in ir and "seq_lens = true" in ir
    # lengths alone keep the fp32 query: no binary16 checks, no q16/out16
    r = kvf("plan", write(tmp_path, "p32.kv", _ext_program("f32")), "--out", str(tmp_path / "o32"))
    assert r.returncode == 0, r.stderr
    tu32 = (tmp_path / "o32" / "decode_pool.hip").read_text()
    assert "kvf_launch_varlen_pool" in tu32 and "va->q16" not in tu32
    # a program without the extension emits exactly the reference's entry points
    r = kvf("plan", write(tmp_path, "plain.kv", _ext_program("f32", "false")), "--out", str(tmp_path / "op"))
    assert r.returncode == 0, r.stderr
    assert "varlen" not in (tmp_path / "op" / "decode_pool.hip").read_text()
    assert "KVF_LAUNCH_VARLEN" not in (tmp_path / "op" / "plan_info.h").read_text()


@pytest.mark.parametrize("text,needle", [
    (_ext_program("bf16"), "only f32 or f16 queries"),
    (_ext_program("f16", "maybe"), "expected true, false, uniform(lo, hi, seed) or loguniform"),
    (_ext_program("f16", "loguniform(0, 8192, 1)"), "integers 1 <= lo <= hi"),
    (_ext_program("f16", "uniform(4096, 2048, 1)"), "integers 1 <= lo <= hi"),
    (_ext_program("f16", "uniform(2048, 9000, 2)"), "exceeds n = 8192"),
    (_ext_program("f16", "loguniform(1024, 8192)"), "expected ','"),
])
def test_extension_rejections(tmp_path, text, needle):
    r = kvf("plan", write(tmp_path, "bad.kv", text), "--out", str(tmp_path / "o"))
    assert r.returncode != 0 and needle in r.stderr, r.stderr


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not installed")
def test_generated_varlen_launcher_compiles_for_gfx950(tmp_path):
    r = kvf("plan", write(tmp_path, "pool.kv", _ext_program()), "--out", str(tmp_path / "o"))
    assert r.returncode == 0, r.stderr
    c = subprocess.run([HIPCC, "-std=c++17", "-O1", "--offload-arch=gfx950", "-c",
                        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
                        "-I", os.path.join(ROOT, "include"), "-I", os.path.join(ROOT, "kvforge_amd", "csrc"),
                        str(tmp_path / "o" / "decode_pool.hip"), "-o", str(tmp_path / "pool.o")],
                       capture_output=True, text=True)
    assert c.returncode == 0, c.stderr[-2000:]


# ------------------------------------------- extension: length distributions
def _dist_program(name, batch, n, seq, fmt="f16", order="head_major", res="contiguous", splits="?",
                  pack="true"):
    return (f'target machine = "{os.path.join(ROOT, "machines", "mi355x.gpu")}"\n'
            f'target calib = "{os.path.join(ROOT, "kvforge_amd", "model", "constants_mi355x.cal")}"\n'
            f"decode {name}(H: 64, H_kv: 8, d: 128, n: {n}, batch: {batch}) {{\n"
            "  Q: query<H, d, f32>\n"
            f"  K: kvcache<n, d, {fmt}, {order}, {res}>\n"
            f"  V: kvcache<n, d, {fmt}, {order}, {res}>\n"
            f"  O = decode_attn(Q, K, V, scale = auto, splits = {splits}, gqa_pack = {pack}, seq_lens = {seq})\n"
            "}\n")


def _plans(tmp_path, name, text):
    r = kvf("plan", write(tmp_path, f"{name}.kv", text), "--all", "--out", str(tmp_path / name))
    assert r.returncode == 0, r.stderr
    lines = (tmp_path / name / "plans.csv").read_text().splitlines()
    head = lines[0].split(",")
    return [dict(zip(head, ln.split(","))) for ln in lines[1:]], (tmp_path / name / "ir.txt").read_text()


def test_length_distributions_draw_the_oracles_lengths(tmp_path):
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    import _oracle as O
    lens = O.lengths_loguniform(16, 1024, 131072, 5)
    rows, ir = _plans(tmp_path, "lu", _dist_program("lu", 16, 131072, "loguniform(1024, 131072, 5)"))
    assert f"seq_lens = loguniform:1024:131072:5 ({int(lens.sum())} tokens, longest {int(lens.max())})" in ir
    assert rows and all(r["seq_lens"] == "loguniform:1024:131072:5" for r in rows)
    lens = O.varlen_lengths(8, 2048, 8192, 2)
    _, ir = _plans(tmp_path, "un", _dist_program("un", 8, 8192, "uniform(2048, 8192, 2)"))
    assert f"seq_lens = uniform:2048:8192:2 ({int(lens.sum())} tokens, longest {int(lens.max())})" in ir
    # without a distribution the plans.csv keeps the reference's columns
    rows, _ = _plans(tmp_path, "pl", _dist_program("pl", 8, 8192, "true"))
    assert "seq_lens" not in rows[0]


def _pred(rows, splits):
    r = [r for r in rows if r["splits"] == str(splits)]
    assert len(r) == 1
    return r[0]


def test_cost_model_counts_every_sequence_and_the_longest(tmp_path):
    # equal lengths reduce to the plain program exactly
    eq, _ = _plans(tmp_path, "eq", _dist_program("eq", 16, 4096, "uniform(4096, 4096, 1)", splits=8))
    pl, _ = _plans(tmp_path, "pl", _dist_program("pl", 16, 4096, "true", splits=8))
    assert [(r["warps"], r["unroll"], r["pred_us"]) for r in eq] == \
           [(r["warps"], r["unroll"], r["pred_us"]) for r in pl]
    # bytes from the sum of the lengths: f16, packed, K and V, 8 KV heads of
    # 128 dims at 2 bytes (pred_gbs * pred_us is the streamed byte count)
    lu, _ = _plans(tmp_path, "lu", _dist_program("lu", 16, 131072, "loguniform(1024, 131072, 5)", splits=1))
    r = lu[0]
    streamed = float(r["pred_gbs"]) * float(r["pred_us"]) * 1e3
    assert abs(streamed / (2 * 264493 * 8 * 128 * 2) - 1) < 1e-4, streamed
    # one split: the longest sequence (90876 tokens) bounds the step, which
    # then costs far more than the same tokens spread evenly
    ev, _ = _plans(tmp_path, "ev", _dist_program("ev", 16, 131072, "uniform(16531, 16531, 1)", splits=1))
    best = lambda rows: min(float(x["pred_us"]) for x in rows)
    assert best(lu) > 3.0 * best(ev), (best(lu), best(ev))
    # with the splits free the planner splits the skewed batch further
    free_lu, _ = _plans(tmp_path, "flu", _dist_program("flu", 16, 131072, "loguniform(1024, 131072, 5)"))
    free_ev, _ = _plans(tmp_path, "fev", _dist_program("fev", 16, 131072, "uniform(16531, 16531, 1)"))
    assert int(free_lu[0]["splits"]) > int(free_ev[0]["splits"]), (free_lu[0], free_ev[0])


def test_skewed_lengths_dispatch_longest_first(tmp_path):
    # a program whose longest sequence is over twice the mean length emits a
    # varlen launcher that always runs longest first; otherwise the caller's
    # flag decides
    src = _dist_program("lu", 16, 131072, "loguniform(1024, 131072, 5)")
    r = kvf("plan", write(tmp_path, "lu.kv", src), "--out", str(tmp_path / "lu"))
    assert r.returncode == 0, r.stderr
    tu = (tmp_path / "lu" / "decode_lu.hip").read_text()
    assert "x.longest_first = true; // longest 90876 > 2 x mean 16530" in tu
    src = _dist_program("un", 8, 8192, "uniform(2048, 8192, 2)")
    r = kvf("plan", write(tmp_path, "un.kv", src), "--out", str(tmp_path / "un"))
    assert r.returncode == 0, r.stderr
    tu = (tmp_path / "un" / "decode_un.hip").read_text()
    assert "x.longest_first = (va->flags & KVF_VARLEN_LONGEST_FIRST) != 0;" in tu


def test_sweep_rows_with_lengths_are_costed_on_them(tmp_path):
    rows, _ = _plans(tmp_path, "lu", _dist_program("lu", 16, 131072, "loguniform(1024, 131072, 5)",
                                                   fmt="int8:64", order="token_major", res="paged:16"))
    pick = rows[:3]
    cols = ["name", "H", "H_kv", "d", "n", "batch", "fmt", "group", "order", "residency", "block_tokens",
            "splits", "gqa_pack", "warps", "unroll"]
    lines = [",".join(cols + ["t_us", "verified", "seq_lens"])]
    for r in pick:
        lines.append(",".join([r[c] for c in cols] + ["100.0", "1", r["seq_lens"]]))
    sweep = write(tmp_path, "sweep.csv", "\n".join(lines) + "\n")
    out = tmp_path / "pred.csv"
    p = kvf("predict", "--sweep", sweep, "--machine", os.path.join(ROOT, "machines", "mi355x.gpu"),
            "--calib", os.path.join(ROOT, "kvforge_amd", "model", "constants_mi355x.cal"), "--out", str(out))
    assert p.returncode == 0, p.stderr
    got = out.read_text().splitlines()[1:]
    assert len(got) == 3
    for r, g in zip(pick, got):
        f = g.split(",")
        assert f[0] == "H64_Hkv8_d128_n131072_b16_loguniform-1024-131072-5"
        assert abs(float(f[11]) / float(r["pred_us"]) - 1) < 1e-5, (f, r["pred_us"])
