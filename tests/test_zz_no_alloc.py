"""The entry point that allocates nothing (kvf_launch_fused_variant_noalloc),
through the C-ABI, against the existing one-launch entry point
kvf_launch_fused_variant with caller-owned counters and partials, and
against the oracle's double-precision attention (the reference's bar,
rel_l2 < 2e-3, runtime/kvf_driver.cu:52): two calls in a row on the same
device scratch, the second with a smaller input, then the first shape again.
(The rejection of steps too large for the scratch happens before any device
call and is tested on the CPU, in test_abi.py.)"""
import ctypes
import sys

import numpy as np
import pytest
import torch

import _oracle as O
from _cases import Case, build, reference, args, vid
from kvforge_amd import runtime as R

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    R.hip_lib()


def _noalloc(vid_, a, va=None):
    L = R.hip_lib()
    return L.kvf_launch_fused_variant_noalloc(vid_.encode(), ctypes.byref(a),
                                              ctypes.byref(va) if va is not None else None,
                                              R.stream_handle())


def _both(b, splits, warps, unroll):
    c = b.case
    v = vid(b, True, unroll)
    # existing entry point: caller-owned counters and partial buffers
    counters = R.fused_counters(c.B, c.Hkv)
    b.out.fill_(float("nan"))
    R.launch_fused(v, args(b, splits, warps), counters)
    torch.cuda.synchronize()
    want = b.out.cpu().numpy()
    # the new one: no workspace, Args::part_o / part_ml left null
    b.out.fill_(float("nan"))
    a = args(b, 1, warps)
    a.splits = splits
    a.part_o = None
    a.part_ml = None
    assert _noalloc(v, a) == R.HIP_SUCCESS
    torch.cuda.synchronize()
    got = b.out.cpu().numpy()
    err = O.rel_l2(got, reference(b))
    print(f"  {c.tag()} S={splits} w{warps} u{unroll}: rel_l2={err:.3g} "
          f"max|noalloc-fused|={float(np.max(np.abs(got - want))):.3g}", flush=True)
    sys.stdout.flush()
    assert np.all(np.isfinite(got))
    assert err < 2e-3
    # same kernels, same arithmetic: equal to rounding of the merge order
    assert np.max(np.abs(got - want)) <= 1e-5 * max(1.0, float(np.max(np.abs(want))))
    return got


def test_noalloc_matches_fused_entry_point_twice():
    big = build(Case(2, 32, 8, 128, 3000, R.FMT_INT8, 64, R.ORD_HEAD, 0, seed=31))
    small = build(Case(1, 16, 4, 128, 700, R.FMT_INT4, 32, R.ORD_TOKEN, 16, seed=32))
    _both(big, 16, 4, 2)
    # second call: a smaller step on the same scratch (the first call's
    # partials are still there; a stale read would not match)
    _both(small, 8, 8, 4)
    # and the first shape again after the smaller one
    _both(big, 32, 4, 2)


def test_noalloc_varlen_f16():
    # variable lengths with binary16 query and output through the same entry
    B, H, Hkv, D = 3, 32, 8, 128
    b = build(Case(B, H, Hkv, D, 900, R.FMT_INT8, 64, R.ORD_TOKEN, 16, seed=33))
    lens = np.array([900, 17, 333], np.int32)
    lens_d = torch.from_numpy(lens).to("cuda:0")
    q16 = b.q.half()
    out16 = torch.full((B, H, D), float("nan"), dtype=torch.float16, device="cuda:0")
    va = R.VarlenArgs()
    va.seq_lens = lens_d.data_ptr()
    va.q16 = q16.data_ptr()
    va.out16 = out16.data_ptr()
    a = args(b, 1, 4)
    a.splits = 8
    a.part_o = None
    a.part_ml = None
    assert _noalloc("int8_tm_p_g4_u2_d128", a, va) == R.HIP_SUCCESS
    torch.cuda.synchronize()
    got = out16.float().cpu().numpy()
    ref = O.reference_attention_varlen(q16.float().cpu().numpy(), b.kdeq, b.vdeq, lens)
    err = O.rel_l2(got, ref)
    print(f"  varlen f16 q/out S=8: rel_l2={err:.3g}", flush=True)
    assert np.all(np.isfinite(got)) and err < 2e-3


def test_noalloc_allocates_nothing_and_replays_in_a_graph():
    # after one call (the per-device and per-variant set-up), further calls
    # leave the device's free memory unchanged, and the step captured into a
    # HIP graph (one kernel node: the kernel returns its counters to zero
    # itself, so no memset is recorded) replays with the eager result, on two
    # different queries and back, with eager work between the replays
    b = build(Case(1, 32, 8, 128, 4096, R.FMT_INT8, 64, R.ORD_HEAD, 0, seed=34))
    v = vid(b, True, 2)
    a = args(b, 1, 4)
    a.splits = 32
    a.part_o = None
    a.part_ml = None
    assert _noalloc(v, a) == R.HIP_SUCCESS
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info()[0]
    for _ in range(3):
        assert _noalloc(v, a) == R.HIP_SUCCESS
    torch.cuda.synchronize()
    assert torch.cuda.mem_get_info()[0] == free0
    q0 = b.q.clone()
    eager = []
    for scale in (1.0, -0.5):
        b.q.copy_(q0 * scale)
        b.out.fill_(float("nan"))
        assert _noalloc(v, a) == R.HIP_SUCCESS
        torch.cuda.synchronize()
        eager.append(b.out.clone())
    b.q.copy_(q0)
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    with torch.cuda.graph(g, stream=s):
        assert _noalloc(v, a) == R.HIP_SUCCESS
    torch.cuda.synchronize()
    for r, scale in enumerate((1.0, -0.5, 1.0, -0.5)):
        b.q.copy_(q0 * scale)
        b.out.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        want = eager[0 if scale == 1.0 else 1]
        assert torch.equal(b.out, want), f"replay {r}"
    b.q.copy_(q0)
    b.out.fill_(float("nan"))
    g.replay()
    torch.cuda.synchronize()
    err = O.rel_l2(b.out.cpu().numpy(), reference(b))
    print(f"  graph replay of the no-alloc step: rel_l2={err:.3g}", flush=True)
    assert err < 2e-3
