"""The persistent step (kvf_launch_persistent_variant) through the C-ABI.

Workgroups claim (sequence, head group, split) items from a queue in device
memory. Every item is computed as in the static grid, so the outputs must
equal the static steps' bit for bit: the fused step's with merge counters,
the two-launch step's without. Grids far smaller than the item count make
every workgroup claim many items; each step runs twice on the same buffers
with different queries (a stale partial or a queue left non-zero by the first
call would show), and the queue and counters must be zero afterwards.
"""
import ctypes
import sys

import numpy as np
import pytest
import torch

import _oracle as O
from _cases import Case, build, reference, args, vid, run
from kvforge_amd import runtime as R

pytestmark = pytest.mark.gpu

REL_TOL = 2e-3


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    R.hip_lib()


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _twice(b, launch):
    # the first call on another query; the second is the one kept
    q_saved = b.q.clone()
    b.q.mul_(-0.5)
    launch()
    torch.cuda.synchronize()
    b.q.copy_(q_saved)
    b.out.fill_(float("nan"))
    launch()
    torch.cuda.synchronize()
    return b.out.cpu().numpy()


CASES = [
    # fmt, group, order, block tokens, G, H, Hkv, splits, warps, unroll
    (R.FMT_INT8, 64, R.ORD_HEAD, 0, 4, 32, 8, 8, 4, 2),
    (R.FMT_F16, 0, R.ORD_TOKEN, 16, 4, 32, 8, 13, 8, 2),
    (R.FMT_INT4, 32, R.ORD_HEAD, 32, 8, 16, 2, 64, 4, 2),
    (R.FMT_INT8, 128, R.ORD_TOKEN, 0, 1, 32, 8, 8, 4, 2),
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"{R.FMT_NAMES[c[0]]}{c[1] or ''}_G{c[4]}_S{c[7]}")
def test_persistent_equals_static_steps(case):
    fmt, group, order, bt, G, H, Hkv, splits, warps, unroll = case
    b = build(Case(2, H, Hkv, 128, 1500, fmt, group, order, bt, seed=31))
    v = vid(b, G > 1, unroll)
    nhg = 2 * (Hkv if G > 1 else H)
    counters = R.fused_counters(2, nhg // 2)
    queue = R.persistent_queue()
    # the static steps
    two = _twice(b, lambda: R.launch(v, args(b, splits, warps)))
    fused = _twice(b, lambda: R.launch_fused(v, args(b, splits, warps), counters))
    assert int(counters.abs().sum()) == 0
    err = O.rel_l2(two, reference(b))
    say(f"  {b.case.tag()} {v} S={splits} items={nhg * splits}: two-launch rel_l2={err:.3g}")
    assert err < REL_TOL
    for wgs in (0, 1, 7, 50):
        got = _twice(b, lambda: R.launch_persistent(v, args(b, splits, warps), queue, counters=counters,
                                                    workgroups=wgs))
        assert int(queue.abs().sum()) == 0 and int(counters.abs().sum()) == 0
        assert np.array_equal(got, fused), f"persistent fused, {wgs} workgroups"
        got = _twice(b, lambda: R.launch_persistent(v, args(b, splits, warps), queue, workgroups=wgs))
        assert int(queue.abs().sum()) == 0
        assert np.array_equal(got, two), f"persistent + merge kernel, {wgs} workgroups"
        say(f"    {wgs or 'all resident'} workgroups: equal to the fused and two-launch steps")
    # one split: the items write the output directly
    one = run(b, 1, pack=G > 1, unroll=unroll, warps=warps)
    got = _twice(b, lambda: R.launch_persistent(v, args(b, 1, warps), queue, workgroups=3))
    assert int(queue.abs().sum()) == 0
    assert np.array_equal(got, one)


def test_persistent_varlen_longest_first():
    # per-sequence lengths with empty and one-token sequences, in index order
    # and longest first, on a grid of 5 workgroups
    B, H, Hkv, D, n = 6, 32, 8, 128, 2000
    lens = np.array([1500, 0, 1, 2000, 33, 700], dtype=np.int32)
    b = build(Case(B, H, Hkv, D, n, R.FMT_INT8, 64, R.ORD_TOKEN, 16, seed=33))
    ref = O.reference_attention_varlen(b.q_host, b.kdeq, b.vdeq, lens)
    lens_d = torch.from_numpy(lens).to("cuda:0")
    v = vid(b, True, 2)
    counters = R.fused_counters(B, Hkv)
    queue = R.persistent_queue()
    for flags in (0, R.VARLEN_LONGEST_FIRST):
        fused = _twice(b, lambda: R.launch_fused(v, args(b, 8, 4), counters, varlen=(lens_d, None, None),
                                                 flags=flags))
        got = _twice(b, lambda: R.launch_persistent(v, args(b, 8, 4), queue, counters=counters,
                                                    varlen=(lens_d, None, None), workgroups=5, flags=flags))
        err = O.rel_l2(got, ref)
        say(f"  varlen B{B} flags={flags}: rel_l2={err:.3g}")
        assert np.all(got[lens == 0] == 0) and err < REL_TOL
        assert np.array_equal(got, fused)
        assert int(queue.abs().sum()) == 0 and int(counters.abs().sum()) == 0


def test_persistent_rejects_bad_arguments():
    b = build(Case(1, 8, 2, 128, 64, R.FMT_INT8, 64, R.ORD_HEAD, 0), check_cache=False)
    a = args(b, 2, 4)
    L = R.hip_lib()
    queue = R.persistent_queue()
    qp = ctypes.c_void_p(queue.data_ptr())
    vid_ = b"int8_hm_c_g4_u2_d128"
    qw = R.QUEUE_WORDS
    assert L.kvf_launch_persistent_variant(vid_, ctypes.byref(a), None, None, 0, None, 0, 0, None) == \
        R.HIP_ERROR_INVALID_VALUE
    assert L.kvf_launch_persistent_variant(vid_, ctypes.byref(a), None, None, 0, qp, qw, -1, None) == \
        R.HIP_ERROR_INVALID_VALUE
    # a queue shorter than KVF_QUEUE_WORDS
    assert L.kvf_launch_persistent_variant(vid_, ctypes.byref(a), None, None, 0, qp, qw - 1, 0, None) == \
        R.HIP_ERROR_INVALID_VALUE
    assert L.kvf_launch_persistent_variant(b"int8_hm_c_g4_u2_d96", ctypes.byref(a), None, None, 0, qp, qw,
                                           0, None) == R.HIP_ERROR_NOT_FOUND
    # the persistent kernels are built for unroll 2
    assert L.kvf_launch_persistent_variant(b"int8_hm_c_g4_u4_d128", ctypes.byref(a), None, None, 0, qp, qw,
                                           1, None) == R.HIP_ERROR_INVALID_VALUE
