"""GPU parity of the decode-attention path, through the C-ABI.

Bar (the reference's own, bench/sweep.cu:194-197 and runtime/kvf_driver.cu:52):
relative L2 error against the double-precision attention over the same
dequantised cache below 2e-3; for f16 caches also max-abs <= 2e-3. The
cache itself (codes, scales, paged placement) must be bit-exact.
"""
import itertools
import math
import sys
import types

import numpy as np
import pytest
import torch

import _oracle as O
from _cases import Case, build, reference, run, args, vid
from kvforge_amd import runtime as R

pytestmark = pytest.mark.gpu

REL_TOL = 2e-3
ABS_TOL_F16 = 2e-3
# Tight bounds on the benchmarked plans, beside the reference's 2e-3 bar: the
# reference's own kernels reach 2.4e-6 (int8) and 2.4e-6 (int4) over its
# sweep (results/sweep_rtx5060-laptop.csv, err_ref); these plans measure
# 1.1e-6 (int8:64 with outlier channels, 32k), 2.5e-6 (int4:32, 64k) and
# ~3e-7 (f16), so a tenfold loss of precision fails here.
TIGHT = {R.FMT_INT8: 1e-5, R.FMT_INT4: 2e-5, R.FMT_F16: 5e-6}


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    R.hip_lib()


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def check(b, got, what):
    ref = reference(b)
    err = O.rel_l2(got, ref)
    mx = float(np.max(np.abs(got - ref)))
    say(f"  {b.case.tag()} {what}: rel_l2={err:.3g} max_abs={mx:.3g}")
    assert np.all(np.isfinite(got)), what
    assert err < REL_TOL, (what, err)
    if b.case.fmt == R.FMT_F16:
        assert mx <= ABS_TOL_F16, (what, mx)
    return err


def test_registry_has_reference_ids():
    ids = set(R.variants())
    for v in ["f16_hm_c_g1_u2_d128", "int8_hm_c_g4_u2_d128", "int4_tm_p_g8_u4_d64",
              "int8_tm_p_g4_u4_d128"]:
        assert v in ids
    assert len(ids) == 3 * 2 * 2 * 2 * 4 * 2


def test_config1_mha_f16_plumbing():
    # MHA, B1, 32 heads, d128, n4096, f16 head-major, S=1
    b = build(Case(1, 32, 32, 128, 4096, R.FMT_F16, 0, R.ORD_HEAD, 0))
    check(b, run(b, 1, pack=False), "S=1")
    check(b, run(b, 8, pack=False, unroll=4, warps=8), "S=8")


@pytest.mark.parametrize("fmt,group", [(R.FMT_F16, 0), (R.FMT_INT8, 64), (R.FMT_INT4, 32)])
@pytest.mark.parametrize("order", [R.ORD_HEAD, R.ORD_TOKEN])
@pytest.mark.parametrize("bt", [0, 16])
def test_twelve_variants(fmt, group, order, bt):
    b = build(Case(2, 32, 8, 128, 1000, fmt, group, order, bt, seed=3))
    for pack in (True, False):
        for splits in (1, 4):
            check(b, run(b, splits, pack=pack, unroll=2 if splits == 1 else 4,
                         warps=4 if pack else 8), f"pack={pack} S={splits}")


@pytest.mark.parametrize("fmt,group", [(R.FMT_INT8, 128), (R.FMT_INT4, 64), (R.FMT_INT4, 128),
                                       (R.FMT_INT8, 32)])
def test_other_groups(fmt, group):
    b = build(Case(1, 16, 4, 128, 700, fmt, group, R.ORD_HEAD, 0, seed=4))
    check(b, run(b, 3), "S=3")


@pytest.mark.parametrize("fmt,group", [(R.FMT_F16, 0), (R.FMT_INT8, 64), (R.FMT_INT4, 32),
                                       (R.FMT_INT4, 64)])
@pytest.mark.parametrize("bt", [0, 32])
def test_d64(fmt, group, bt):
    b = build(Case(2, 16, 2, 64, 777, fmt, group, R.ORD_TOKEN if bt else R.ORD_HEAD, bt, seed=5))
    check(b, run(b, 2), "S=2")
    check(b, run(b, 1, pack=False), "S=1 unpacked")


# tests/edge/*.kv of the reference: shapes that stress chunking and packing
EDGE = [
    ("edge_short", 1, 8, 8, 64, 100),
    ("edge_n129", 1, 32, 8, 128, 129),
    ("edge_odd_n", 2, 12, 4, 128, 1001),
    ("edge_g8_n3333", 3, 16, 2, 64, 3333),
]


@pytest.mark.parametrize("name,B,H,Hkv,D,n", EDGE)
def test_edge_shapes(name, B, H, Hkv, D, n):
    g = H // Hkv
    for fmt, group in ((R.FMT_F16, 0), (R.FMT_INT8, 64), (R.FMT_INT4, 32)):
        for order, bt in ((R.ORD_HEAD, 0), (R.ORD_TOKEN, 64)):
            b = build(Case(B, H, Hkv, D, n, fmt, group, order, bt, seed=7))
            for splits in (1, 2, 64):
                check(b, run(b, splits, pack=g in (2, 4, 8)), f"{name} S={splits}")


def test_empty_splits_and_partials():
    # n < splits * 2: some splits own no token and must report (-inf, 0, 0)
    c = Case(1, 8, 2, 128, 40, R.FMT_INT8, 64, R.ORD_HEAD, 0, seed=9)
    b = build(c)
    S = 32
    a = args(b, S, 4, partial_buffers=True)
    R.launch_partial(vid(b, True, 2), a)
    torch.cuda.synchronize()
    po, pm = (t.cpu().numpy() for t in a._keep)
    o_ref, lse_ref, m_ref = O.reference_partials(b.q_host, b.kdeq, b.vdeq, S)
    m, L = pm[..., 0].astype(np.float64), pm[..., 1].astype(np.float64)
    empty = np.isneginf(m_ref)
    assert np.any(empty)
    assert np.all(np.isneginf(m[empty])) and np.all(L[empty] == 0) and np.all(po[empty] == 0)
    full = ~empty
    assert np.max(np.abs(m[full] - m_ref[full])) < 1e-4
    lse = m + np.log2(np.where(L > 0, L, 1))
    assert np.max(np.abs(lse[full] - lse_ref[full])) < 1e-4
    # normalised partials: the reference's relative bar; V enters PV as
    # binary16 dequantised values, so single entries of a 2-token split can
    # differ by up to a binary16 rounding of |v| (< 2^-11 * 4 here)
    on = po[full] / L[full][:, None]
    assert O.rel_l2(on.astype(np.float32), o_ref[full]) < REL_TOL
    assert np.max(np.abs(on - o_ref[full])) < 2.0 ** -11 * 4
    # the merge of these partials equals the unsplit reference
    out = torch.zeros_like(b.out)
    a.out = out.data_ptr()
    R.launch_merge(128, a)
    torch.cuda.synchronize()
    check(b, out.cpu().numpy(), "merge")


def test_merge_split_counts():
    # the merge folds the splits 32 at a time with a running max, and past one
    # chunk runs 2, 4 or 8 slices side by side: split counts around and past
    # one chunk and each slice count (with more than 8 chunks a slice folds
    # several), for both head dimensions, and one where the last splits own
    # no token
    for D, n in ((128, 3000), (64, 2500)):
        b = build(Case(2, 8, 2, D, n, R.FMT_INT8, 32, R.ORD_HEAD, 0, seed=11))
        for splits in (31, 33, 97, 200, 300):
            check(b, run(b, splits), f"D={D} S={splits}")
    b = build(Case(1, 4, 4, 128, 150, R.FMT_F16, 0, R.ORD_HEAD, 0, seed=12))
    check(b, run(b, 100, pack=False), "n=150 S=100")
    b = build(Case(1, 4, 1, 128, 9000, R.FMT_INT8, 64, R.ORD_HEAD, 0, seed=13))
    check(b, run(b, 256), "one KV head, S=256")


def test_north_star_int8_32k():
    # GQA 32/8, d128, n32768, int8:64 with 1% outlier
    # channels x8, head-major contiguous, splits swept
    b = build(Case(1, 32, 8, 128, 32768, R.FMT_INT8, 64, R.ORD_HEAD, 0, seed=1, outliers=True))
    for splits in (1, 2, 4, 8, 16, 64):
        for unroll, warps in ((2, 4), (4, 8)):
            err = check(b, run(b, splits, unroll=unroll, warps=warps), f"S={splits} u{unroll} w{warps}")
            assert err < TIGHT[R.FMT_INT8], (splits, unroll, warps, err)
    # the plan bench.py times for the headline metric: 32 splits, 4 waves, u2
    err = check(b, run(b, 32, unroll=2, warps=4), "benchmarked plan S=32 u2 w4")
    assert err < TIGHT[R.FMT_INT8], err
    # against exact fp32 attention the error is the quantizer's, as the
    # oracle's own dequantised reference shows
    exact = O.reference_attention(b.q_host, b.K, b.V)
    err_exact = O.rel_l2(run(b, 64), exact)
    err_quant = O.rel_l2(reference(b), exact)
    say(f"  err_exact int8:64 with outliers = {err_exact:.4g} (quantizer alone {err_quant:.4g})")
    assert abs(err_exact - err_quant) < 0.02 * err_quant


def test_north_star_f16_32k():
    b = build(Case(1, 32, 8, 128, 32768, R.FMT_F16, 0, R.ORD_HEAD, 0, seed=1))
    for splits in (1, 64):
        check(b, run(b, splits), f"S={splits}")
    err = check(b, run(b, 32, unroll=2, warps=4), "S=32 u2 w4")
    assert err < TIGHT[R.FMT_F16], err


def test_long_context_int4_64k():
    # n65536, int4:32, head-major contiguous, splits 8..256
    b = build(Case(1, 32, 8, 128, 65536, R.FMT_INT4, 32, R.ORD_HEAD, 0, seed=1))
    for splits in (8, 16, 64, 128, 256):
        for warps in (4, 8):
            err = check(b, run(b, splits, warps=warps), f"S={splits} w{warps}")
            assert err < TIGHT[R.FMT_INT4], (splits, warps, err)
    # the plan bench.py --config 4 times: 32 splits, 8 waves, u2
    err = check(b, run(b, 32, unroll=2, warps=8), "benchmarked plan S=32 u2 w8")
    assert err < TIGHT[R.FMT_INT4], err


def test_int8_eight_packed_heads_accuracy():
    # int8:64 with eight heads per workgroup has 16 accumulator columns, so a
    # softmax weight's hi and lo halves share one accumulator; its lo half
    # used to be a binary16 subnormal (3.7e-6 to 3.9e-6 here), it measures
    # about 6e-7 now
    b = build(Case(1, 64, 8, 128, 8192, R.FMT_INT8, 64, R.ORD_HEAD, 0, seed=1))
    for splits in (1, 8):
        err = check(b, run(b, splits), f"G8 S={splits}")
        assert err < 2.5e-6, (splits, err)


def _scaled_case(fmt, group, H, Hkv, n, q_peak=None, v_scale=None, seed=5):
    """A case at the edge of the binary16 operands' range: q_peak sets one
    query dimension so that max |q * scale * log2 e| reaches it, v_scale
    multiplies V so that the largest quantization scale of a V group reaches
    it (levels = 255 for int8, 15 for int4)."""
    D = 128
    q, K, V = O.make_data(1, H, Hkv, D, n, seed)
    scale_log2 = math.log2(math.e) / math.sqrt(D)
    if q_peak is not None:
        q[:, :, 7] *= q_peak / (np.abs(q[:, :, 7]).max() * scale_log2)
    if v_scale is not None:
        levels = 255 if fmt == R.FMT_INT8 else 15
        g = V.reshape(-1, D // group, group)
        V *= v_scale / ((g.max(axis=2) - g.min(axis=2)).max() / levels)
    return build(Case(1, H, Hkv, D, n, fmt, group, R.ORD_HEAD, 0, seed=seed), data=(q, K, V))


@pytest.mark.parametrize("fmt,group,H", [(R.FMT_INT8, 64, 64), (R.FMT_INT8, 64, 32), (R.FMT_INT4, 32, 32)])
def test_input_range_limits(fmt, group, H):
    # the query limit of the quantized kernels, |q * scale * log2 e| < 1023,
    # taken to 900 in one dimension (a nearly one-hot softmax)
    b = _scaled_case(fmt, group, H, 8, 2048, q_peak=900.0)
    for splits in (1, 8):
        check(b, run(b, splits), f"q peak 900 S={splits}")
    del b
    # V group scales near their limit: 12 where hi and lo weights share an
    # accumulator (eight packed int8:64 heads, limit 16), 200 elsewhere
    # (limit 256); the query stays as drawn, so the running max lags and
    # weights reach up to 2^8 (2^12 in the former)
    b = _scaled_case(fmt, group, H, 8, 2048, v_scale=12.0 if H == 64 else 200.0)
    for splits in (1, 8):
        check(b, run(b, splits), f"V scale at the limit S={splits}")


@pytest.mark.parametrize("order", [R.ORD_HEAD, R.ORD_TOKEN])
def test_paged_page_ids_reloaded(order):
    # a wave keeps the page ids of its next 32 tiles in one register (one
    # sub-tile per lane) and reloads them every 32 tiles: n = 32768 in pages
    # of 16 tokens with one split gives each of 4 waves 256 tiles, so the
    # reload runs 7 times per wave; with 3 splits the ranges start mid-page
    b = build(Case(1, 32, 8, 128, 32768, R.FMT_INT8, 64, order, 16, seed=5))
    for splits, warps in ((1, 4), (3, 4), (1, 8)):
        check(b, run(b, splits, unroll=2, warps=warps), f"S={splits} w{warps}")
    # the same through the per-sequence-length path, whose splits take every
    # S-th tile (and read their page ids before the length): 256 tiles per
    # wave at S = 1, tiles 3 apart at S = 3
    lens_d = torch.tensor([32768], dtype=torch.int32, device="cuda:0")
    for splits in (1, 3):
        b.out.fill_(float("nan"))
        R.launch_varlen(vid(b, True, 2), args(b, splits, 4), lens_d)
        torch.cuda.synchronize()
        check(b, b.out.cpu().numpy(), f"varlen S={splits}")


def _pool_case(B, lo, hi, pool):
    """Variable lengths from a shared, shuffled block pool, paged:16
    token-major, int8:64, binary16 query/output, each sequence appending only
    its own tokens into its own pages; the pooled cache is checked byte for
    byte against the oracle's quantizer through the page table."""
    H, Hkv, D, bt = 32, 8, 128, 16
    lens = O.varlen_lengths(B, lo, hi, 2)
    n_max = int(lens.max())
    q, K, V = O.make_data(B, H, Hkv, D, n_max, 1)
    q16 = q.astype(np.float16)
    kd, km, kdeq = O.quantize(R.FMT_INT8, 64, D, K)
    vd, vm, vdeq = O.quantize(R.FMT_INT8, 64, D, V)
    table, mb = O.pool_table(lens, bt, pool, 18)
    dev = torch.device("cuda:0")
    tbl = torch.from_numpy(np.where(table < 0, 0, table).astype(np.int32)).to(dev)
    rows = pool * Hkv * bt
    kc = torch.zeros(rows * D, dtype=torch.uint8, device=dev)
    vc = torch.zeros(rows * D, dtype=torch.uint8, device=dev)
    kmc = torch.zeros(rows * 2, dtype=torch.int32, device=dev)
    vmc = torch.zeros(rows * 2, dtype=torch.int32, device=dev)
    for bb in range(B):
        L = int(lens[bb])
        for src, dst, dm in ((K, kc, kmc), (V, vc, vmc)):
            x = torch.from_numpy(np.ascontiguousarray(src[bb, :, :L])).to(dev)
            R.quantize_place(R.FMT_INT8, 64, D, x, 1, Hkv, L, R.ORD_TOKEN, bt, tbl[bb], mb,
                             dst, dm)
    torch.cuda.synchronize()
    # every (sequence, head, token < len) row sits where row_of puts it
    for codes, metas, dev_c, dev_m in ((kd, km, kc, kmc), (vd, vm, vc, vmc)):
        cc = dev_c.cpu().numpy().reshape(rows, D)
        mm = dev_m.cpu().numpy().view(np.uint32).reshape(rows, 2)
        codes = codes.reshape(B, Hkv, n_max, D)
        metas = metas.reshape(B, Hkv, n_max, 2, 2).view(np.uint32).reshape(B, Hkv, n_max, 2)
        for bb in range(B):
            t = np.arange(int(lens[bb]))
            for h in range(Hkv):
                prow = table[bb, t >> 4].astype(np.int64) * Hkv * bt + (t & (bt - 1)) * Hkv + h
                assert np.array_equal(cc[prow], codes[bb, h, :t.size]), ("codes", bb, h)
                assert np.array_equal(mm[prow], metas[bb, h, :t.size]), ("meta", bb, h)
    c = types.SimpleNamespace(B=B, H=H, Hkv=Hkv, D=D, lens=lens, n_max=n_max, mb=mb, tbl=tbl,
                              kc=kc, vc=vc, kmc=kmc, vmc=vmc)
    c.q16d = torch.from_numpy(q16).to(dev)
    c.out16 = torch.zeros((B, H, D), dtype=torch.float16, device=dev)
    c.qdummy = torch.zeros((B, H, D), dtype=torch.float32, device=dev)
    c.outdummy = torch.zeros((B, H, D), dtype=torch.float32, device=dev)
    c.lens_d = torch.from_numpy(lens).to(dev)
    c.ref = O.reference_attention_varlen_mt(q16.astype(np.float32), kdeq, vdeq, lens, 8)
    return c


def _pool_args(c, splits, warps, po=None, pm=None):
    dev = c.q16d.device
    if po is None and splits > 1:
        po = torch.full((c.B, c.H, splits, c.D), float("nan"), device=dev)
        pm = torch.full((c.B, c.H, splits, 2), float("nan"), device=dev)
    a = R.make_args(c.qdummy, c.kc, c.vc, c.kmc, c.vmc, c.tbl, c.outdummy, po, pm, c.B, c.H,
                    c.Hkv, c.n_max, splits, warps, group=64, block_tokens=16, max_blocks=c.mb,
                    D=c.D)
    a._keep = (po, pm)
    return a


def _pool_check(c, what):
    torch.cuda.synchronize()
    got = c.out16.float().cpu().numpy()
    err = O.rel_l2(got, c.ref)
    say(f"  pool B{c.B} lens {c.lens.min()}..{c.lens.max()} {what}: rel_l2={err:.3g}")
    assert np.all(np.isfinite(got))
    assert err < REL_TOL, (what, err)


def test_varlen_pool_f16_qo():
    # BASELINE configs[2] scaled down: B4, lengths 200..900, a 512-page pool
    c = _pool_case(4, 200, 900, 512)
    for splits in (1, 8):
        c.out16.fill_(float("nan"))
        R.launch_varlen("int8_tm_p_g4_u2_d128", _pool_args(c, splits, 4), c.lens_d,
                        q16=c.q16d, out16=c.out16)
        _pool_check(c, f"S={splits}")
    # the same step through the library kvf planned from kvforge_amd/plans/config3.kv
    # (its launcher fixes splits = 8 and the plan's waves and shifts)
    plan = R.plan_lib("config3").kvf_plan_config3().decode()
    assert plan.startswith("int8:64 | token_major/paged:16 | splits=8 pack"), plan
    dev = c.q16d.device
    po = torch.full((c.B, c.H, 8, c.D), float("nan"), device=dev)
    pm = torch.full((c.B, c.H, 8, 2), float("nan"), device=dev)
    c.out16.fill_(float("nan"))
    R.launch_plan_varlen("config3", _pool_args(c, 1, 8, po, pm), c.lens_d, q16=c.q16d,
                         out16=c.out16)
    _pool_check(c, f"planned config3 ({plan})")


def test_config3_full_size():
    # BASELINE configs[2] at its stated size, the plan bench.py --config 3
    # times: B8, lengths U[2048, 8192] (seed 2), a 4096-page pool shuffled
    # with seed 18, paged:16 token-major int8:64, f16 q/out, 8 splits, 4 waves
    c = _pool_case(8, 2048, 8192, 4096)
    for splits, warps in ((8, 4), (1, 4), (16, 8)):
        c.out16.fill_(float("nan"))
        R.launch_varlen("int8_tm_p_g4_u2_d128", _pool_args(c, splits, warps), c.lens_d,
                        q16=c.q16d, out16=c.out16)
        _pool_check(c, f"S={splits} w{warps}")
    # the one-launch step on the same workload
    counters = R.fused_counters(c.B, c.Hkv)
    c.out16.fill_(float("nan"))
    R.launch_fused("int8_tm_p_g4_u2_d128", _pool_args(c, 8, 4), counters,
                   varlen=(c.lens_d, c.q16d, c.out16))
    _pool_check(c, "fused S=8 w4")
    assert int(counters.abs().sum()) == 0
    # and through the planned library (splits fixed by the plan)
    dev = c.q16d.device
    po = torch.full((c.B, c.H, 8, c.D), float("nan"), device=dev)
    pm = torch.full((c.B, c.H, 8, 2), float("nan"), device=dev)
    c.out16.fill_(float("nan"))
    R.launch_plan_varlen("config3", _pool_args(c, 1, 8, po, pm), c.lens_d, q16=c.q16d,
                         out16=c.out16)
    _pool_check(c, "planned config3")


VARLEN_CASES = [
    # (B, H, Hkv, D, n, fmt, group, order, bt, lengths, splits)
    (5, 8, 2, 128, 700, R.FMT_F16, 0, R.ORD_HEAD, 0, [0, 1, 33, 700, 64], (2, 3, 8, 40)),
    (9, 8, 2, 128, 900, R.FMT_INT8, 64, R.ORD_TOKEN, 16, [900] + [1] * 7 + [32], (2, 3)),
    (3, 8, 2, 64, 300, R.FMT_INT4, 32, R.ORD_HEAD, 32, [0, 0, 0], (4,)),
    (1, 32, 8, 128, 3000, R.FMT_INT8, 64, R.ORD_HEAD, 0, [2999], (2, 7, 64)),
    (64, 4, 2, 64, 200, R.FMT_INT8, 32, R.ORD_TOKEN, 0, "random", (2, 5)),
    (65, 4, 1, 64, 120, R.FMT_INT4, 64, R.ORD_TOKEN, 16, "random", (3,)),
]


@pytest.mark.parametrize("case", VARLEN_CASES, ids=lambda c: f"B{c[0]}_{R.FMT_NAMES[c[5]]}")
def test_varlen_edge_lengths(case):
    # per-sequence lengths: empty and one-token sequences, lengths at and
    # around a tile, one long sequence beside many short ones, a batch of
    # empty sequences, batches of 64 and 65, and tokens past each length
    # that must not be read. The partial buffers start as NaN, so a merge
    # that read a slot no workgroup wrote would show.
    B, H, Hkv, D, n, fmt, group, order, bt, lens, split_list = case
    if isinstance(lens, str):
        rng = np.random.default_rng(B)
        lens = rng.integers(0, n + 1, size=B)
        lens[::7] = 0
        lens[1] = n
    lens = np.asarray(lens, dtype=np.int32)
    b = build(Case(B, H, Hkv, D, n, fmt, group, order, bt, seed=21))
    ref = O.reference_attention_varlen(b.q_host, b.kdeq, b.vdeq, lens)
    lens_d = torch.from_numpy(lens).to("cuda:0")
    # each case also longest first (ties, empty sequences; ignored past 64 sequences)
    for splits in split_list:
        for (pack, unroll, warps), flags in itertools.product(((True, 2, 4), (False, 4, 8)),
                                                              (0, R.VARLEN_LONGEST_FIRST)):
            b.out.fill_(float("nan"))
            a = args(b, splits, warps)
            R.launch_varlen(vid(b, pack, unroll), a, lens_d, flags=flags)
            torch.cuda.synchronize()
            got = b.out.cpu().numpy()
            err = O.rel_l2(got, ref) if np.any(ref) else float(np.max(np.abs(got)))
            say(f"  {b.case.tag()} lens {lens.min()}..{lens.max()} S={splits} pack={pack} flags={flags}: "
                f"err={err:.3g}")
            assert np.all(np.isfinite(got))
            assert np.all(got[lens == 0] == 0)
            assert err < REL_TOL
    # the fused step, longest first
    splits = max(split_list)
    if splits > 1:
        counters = R.fused_counters(B, Hkv)
        b.out.fill_(float("nan"))
        R.launch_fused(vid(b, True, 2), args(b, splits, 4), counters, varlen=(lens_d, None, None),
                       flags=R.VARLEN_LONGEST_FIRST)
        torch.cuda.synchronize()
        got = b.out.cpu().numpy()
        err = O.rel_l2(got, ref) if np.any(ref) else float(np.max(np.abs(got)))
        say(f"  {b.case.tag()} fused longest first S={splits}: err={err:.3g}")
        assert np.all(np.isfinite(got)) and np.all(got[lens == 0] == 0)
        assert err < REL_TOL and int(counters.abs().sum()) == 0


def test_bad_arguments_are_rejected():
    b = build(Case(1, 8, 2, 128, 64, R.FMT_INT8, 64, R.ORD_HEAD, 0), check_cache=False)
    a = args(b, 1, 4)
    a.warps = 3
    assert R.hip_lib().kvf_launch_variant(b"int8_hm_c_g4_u2_d128", a, None) == R.HIP_ERROR_INVALID_VALUE
    a.warps = 4
    assert R.hip_lib().kvf_launch_variant(b"int8_hm_c_g4_u2_d96", a, None) == R.HIP_ERROR_NOT_FOUND
    a.group_shift = 4
    assert R.hip_lib().kvf_launch_variant(b"int8_hm_c_g4_u2_d128", a, None) == R.HIP_ERROR_INVALID_VALUE


@pytest.mark.parametrize("fmt,group,order,bt,G", [
    (R.FMT_INT8, 64, R.ORD_HEAD, 0, 4), (R.FMT_F16, 0, R.ORD_TOKEN, 16, 4),
    (R.FMT_INT4, 32, R.ORD_HEAD, 32, 8), (R.FMT_INT8, 128, R.ORD_TOKEN, 0, 1)])
def test_fused_merge_matches_two_launch(fmt, group, order, bt, G):
    # one-launch step (last workgroup merges) against the two-launch step
    H = 32 if G in (1, 4) else 16
    Hkv = H // 4 if G == 1 else H // G
    b = build(Case(2, H, Hkv, 128, 1500, fmt, group, order, bt, seed=11))
    counters = R.fused_counters(2, Hkv if G > 1 else H)
    # (past 32 splits the last workgroup folds the splits in chunks of 32, one
    # memory round trip per chunk: an even and an odd chunk count, several
    # chunks, and a chunk that ends past the split count)
    for splits, warps, unroll in ((8, 4, 2), (13, 8, 4), (64, 4, 4), (97, 4, 2), (200, 4, 2)):
        two = run(b, splits, pack=G > 1, unroll=unroll, warps=warps)
        b.out.fill_(float("nan"))
        a = args(b, splits, warps)
        # the first call runs on another query, so its partials differ from the
        # second call's: a merge that read a stale partial from the first call
        # (same buffers, counters left at zero) would not match the two-launch
        # step
        q_saved = b.q.clone()
        b.q.mul_(-0.5)
        R.launch_fused(vid(b, G > 1, unroll), a, counters)
        torch.cuda.synchronize()
        b.q.copy_(q_saved)
        R.launch_fused(vid(b, G > 1, unroll), a, counters)
        torch.cuda.synchronize()
        fused = b.out.cpu().numpy()
        assert int(counters.abs().sum()) == 0
        check(b, fused, f"fused S={splits} w{warps} u{unroll}")
        assert np.max(np.abs(fused - two)) <= 1e-5 * max(1.0, float(np.max(np.abs(two))))


@pytest.mark.parametrize("fmt,group", [(R.FMT_F16, 0), (R.FMT_INT8, 64), (R.FMT_INT4, 32)])
@pytest.mark.parametrize("order", [R.ORD_HEAD, R.ORD_TOKEN])
@pytest.mark.parametrize("bt", [0, 16])
@pytest.mark.parametrize("D", [64, 128])
def test_every_registered_variant(fmt, group, order, bt, D):
    # every (G, U) of this bucket and head dimension, both wave counts,
    # split and unsplit: all 192 registered ids run once across the cases
    ids = set(R.variants())
    for G in (1, 2, 4, 8):
        H = 6 if G == 1 else 2 * G
        b = build(Case(1, H, 2, D, 333, fmt, group, order, bt, seed=11 + G))
        for i, U in enumerate((2, 4)):
            assert vid(b, G > 1, U) in ids
            splits, warps = ((1, 8), (5, 4))[i] if G % 2 == 0 else ((3, 4), (1, 8))[i]
            check(b, run(b, splits, pack=G > 1, unroll=U, warps=warps), f"G={G} U={U} S={splits} W={warps}")


@pytest.mark.parametrize("fmt,group,order,bt", [
    (R.FMT_INT8, 64, R.ORD_HEAD, 0), (R.FMT_INT4, 32, R.ORD_TOKEN, 0),
    (R.FMT_INT8, 128, R.ORD_TOKEN, 16), (R.FMT_F16, 0, R.ORD_HEAD, 64)])
def test_append_tokens_equals_whole_cache_placement(fmt, group, order, bt):
    # appending a cache one token per sequence and step, each sequence at its
    # own position, gives the bytes the oracle's quantize + place give for the
    # whole cache; a position past the layout writes nothing
    B, Hkv, D, n = 3, 2, 128, 40
    _, K, _ = O.make_data(B, 2 * Hkv, Hkv, D, n, 21)
    kd, km, _ = O.quantize(fmt, group, D, K)
    pkd, pkm, table, mb = O.place(B, Hkv, n, fmt, group, D, order, bt, kd, km)
    dev = torch.device("cuda:0")
    rows, _ = R.rows_alloc(B, Hkv, n, bt)
    mw = D // group if fmt != R.FMT_F16 else 0
    data = torch.zeros(rows * R.row_bytes(fmt, D), dtype=torch.uint8, device=dev)
    meta = torch.zeros(rows * mw, dtype=torch.int32, device=dev) if mw else None
    tbl = torch.from_numpy(table.astype(np.int32)).to(dev) if bt else None
    Kt = torch.from_numpy(K.reshape(B, Hkv, n, D))
    offs = [0, 7, 23]
    for step in range(n + 1):
        # the last step's positions all lie outside the layout, which holds
        # max_blocks * block_tokens tokens per sequence when paged
        past = mb * bt if bt else n
        pos = [(step + o) % n for o in offs] if step < n else [past, -1, 1 << 20]
        x = Kt[torch.arange(B), :, torch.tensor([min(p, n - 1) for p in pos])].contiguous().to(dev)
        pt = torch.tensor(pos, dtype=torch.int32, device=dev)
        R.append_tokens(fmt, group, D, x, B, Hkv, n, pt, order, bt, tbl, mb, data, meta)
    torch.cuda.synchronize()
    assert np.array_equal(data.cpu().numpy(), pkd.ravel()), "codes differ"
    if mw:
        assert np.array_equal(meta.cpu().numpy().view(np.uint32), pkm.ravel()), "meta differs"
