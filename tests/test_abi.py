"""The C-ABI library loads without a GPU and exports every function that
include/*.h declares with C linkage; Args keeps the reference's layout
(runtime/kvf_kernels.cuh:29-46: 9 pointers, 9 ints, 1 float). No kernel is
launched here."""
import ctypes
import os
import re

import pytest

from kvforge_amd import runtime as R

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INCLUDE = os.path.join(ROOT, "include")


def _c_functions(path):
    """Names of the functions declared inside the header's extern "C" block."""
    text = open(path).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    names = []
    for block in re.findall(r'extern "C" \{(.*?)\n\}', text, flags=re.S):
        for m in re.finditer(r"\b([A-Za-z_][A-Za-z0-9_]*)\s*\(", block):
            name = m.group(1)
            if name.startswith("kvf_"):
                names.append(name)
    return names


def test_header_declares_entry_points():
    names = _c_functions(os.path.join(INCLUDE, "kvf_abi.h"))
    for must in ("kvf_launch_variant", "kvf_launch_merge", "kvf_quantize_place", "kvf_append_tokens",
                 "kvf_variant_count", "kvf_variant_id"):
        assert must in names
    assert len(names) == len(set(names))


@pytest.mark.skipif(not os.path.exists(R.HIP_LIB), reason="libkvf_hip.so not built")
def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(R.HIP_LIB)
    missing = []
    for h in sorted(os.listdir(INCLUDE)):
        if h.endswith(".h"):
            for name in _c_functions(os.path.join(INCLUDE, h)):
                if not hasattr(lib, name):
                    missing.append(f"{h}:{name}")
    assert not missing, missing


@pytest.mark.skipif(not os.path.exists(R.HIP_LIB), reason="libkvf_hip.so not built")
def test_registry_is_populated_without_a_gpu():
    # the registry is filled by static code; listing it touches no device
    lib = R.hip_lib()
    n = lib.kvf_variant_count()
    ids = {lib.kvf_variant_id(i).decode() for i in range(n)}
    # the reference's gen/ tables hold 144 ids (12 buckets x G{1,4,8} x U{2,4}
    # x D{64,128}); G=2 is added because plan enumeration packs g=2 groups
    # (src/plan.cpp:37-86) and would otherwise name a variant nobody compiled
    assert n == 192 and len(ids) == 192
    for fmt in ("f16", "int8", "int4"):
        for o in ("hm", "tm"):
            for r in ("c", "p"):
                for g in (1, 2, 4, 8):
                    for u in (2, 4):
                        for d in (64, 128):
                            assert f"{fmt}_{o}_{r}_g{g}_u{u}_d{d}" in ids
    assert lib.kvf_version().decode()


def test_args_layout_matches_reference():
    a = R.Args
    names = [f[0] for f in a._fields_]
    assert names == ["q", "k", "v", "k_meta", "v_meta", "block_table", "out", "part_o",
                     "part_ml", "B", "H", "Hkv", "n", "splits", "warps", "group_shift",
                     "block_shift", "max_blocks", "scale_log2"]
    p = ctypes.sizeof(ctypes.c_void_p)
    assert a.B.offset == 9 * p
    assert a.scale_log2.offset == 9 * p + 9 * 4
    assert ctypes.sizeof(a) == 9 * p + 9 * 4 + 4


def test_planned_program_library_exports_its_entry_points():
    # kvforge_amd/plans/config3.kv, planned and built by `make -C kvforge_amd`:
    # the reference's two entry points plus the variable-length one; the plan
    # string is host data, readable without a GPU
    L = R.plan_lib("config3")
    for sym in ("kvf_launch_config3", "kvf_launch_varlen_config3", "kvf_plan_config3"):
        assert hasattr(L, sym), sym
    plan = L.kvf_plan_config3().decode()
    assert plan.startswith("int8:64 | token_major/paged:16 | splits=8 pack w"), plan
    # the north-star program: the reference's entry points only, and the
    # plan the sweep measured fastest for that shape among int8:64 plans
    N = R.plan_lib("northstar")
    for sym in ("kvf_launch_northstar", "kvf_plan_northstar"):
        assert hasattr(N, sym), sym
    assert not hasattr(N, "kvf_launch_varlen_northstar")
    assert N.kvf_plan_northstar().decode() == "int8:64 | head_major/contiguous | splits=32 pack w4 u2"
    # each program has its single-plan driver
    for name in ("config3", "northstar"):
        assert os.access(os.path.join(ROOT, "kvforge_amd", "plans", f"kvf_driver_{name}"), os.X_OK), name


@pytest.mark.skipif(not os.path.exists(R.HIP_LIB), reason="libkvf_hip.so not built")
def test_sized_buffers_are_checked_before_any_device_call():
    # ABI version 2: the fused, persistent and timed-step entry points take
    # the sizes of their counter and queue buffers and reject buffers that
    # are too small, before touching the device (a caller sized to the
    # version-1 contract, one word per head group, gets hipErrorInvalidValue
    # instead of out-of-bounds atomics)
    lib = R.hip_lib()
    assert lib.kvf_abi_version() == R.ABI_VERSION == 2
    text = open(os.path.join(INCLUDE, "kvf_abi.h")).read()
    assert "#define KVF_ABI_VERSION 2" in text
    assert "#define KVF_QUEUE_WORDS (2 * KVF_COUNTER_STRIDE)" in text
    assert "ABI 2" in lib.kvf_version().decode()
    a = R.Args()
    a.B, a.H, a.Hkv, a.n, a.splits, a.warps, a.group_shift = 2, 32, 8, 4096, 32, 4, 6
    buf = ctypes.create_string_buffer(4 * 4096)  # host memory: never dereferenced
    p = ctypes.cast(buf, ctypes.c_void_p)
    need = 2 * 8 * R.COUNTER_STRIDE  # B x head groups (pack 4: Hkv) x stride
    for vid, groups in ((b"int8_hm_c_g4_u2_d128", 8), (b"int8_hm_c_g1_u2_d128", 32)):
        need = 2 * groups * R.COUNTER_STRIDE
        for words in (0, 2 * groups, need - 1):
            assert lib.kvf_launch_fused_variant(vid, ctypes.byref(a), None, p, words,
                                                None) == R.HIP_ERROR_INVALID_VALUE, (vid, words)
            assert lib.kvf_launch_step_timed(vid, ctypes.byref(a), None, p, words, None, p,
                                             p) == R.HIP_ERROR_INVALID_VALUE, (vid, words)
            assert lib.kvf_launch_persistent_variant(vid, ctypes.byref(a), None, p, words, p,
                                                     R.QUEUE_WORDS, 0,
                                                     None) == R.HIP_ERROR_INVALID_VALUE, (vid, words)
    # no counters at all is not a fused step either
    assert lib.kvf_launch_fused_variant(b"int8_hm_c_g4_u2_d128", ctypes.byref(a), None, None, 0,
                                        None) == R.HIP_ERROR_INVALID_VALUE


@pytest.mark.skipif(not os.path.exists(R.HIP_LIB), reason="libkvf_hip.so not built")
def test_noalloc_entry_rejects_steps_beyond_its_scratch():
    # kvf_launch_fused_variant_noalloc checks the step's counters and partials
    # against its fixed device scratch (KVF_SCRATCH_BYTES) before touching the
    # device: 64 sequences x 32 heads x 32 splits x 130 floats is 34 MB
    lib = R.hip_lib()
    a = R.Args()
    a.B, a.H, a.Hkv, a.n, a.splits, a.warps, a.group_shift = 64, 32, 8, 4096, 32, 4, 6
    assert lib.kvf_launch_fused_variant_noalloc(b"int8_hm_c_g4_u2_d128", ctypes.byref(a), None,
                                                None) == R.HIP_ERROR_INVALID_VALUE
    # an unknown id is not found, also before any device call
    assert lib.kvf_launch_fused_variant_noalloc(b"int8_hm_c_g4_u2_d96", ctypes.byref(a), None,
                                                None) == R.HIP_ERROR_NOT_FOUND
    text = open(os.path.join(INCLUDE, "kvf_abi.h")).read()
    assert "#define KVF_SCRATCH_BYTES (16u << 20)" in text
