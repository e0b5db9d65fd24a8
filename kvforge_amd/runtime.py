"""Python face of the C-ABI in include/kvf_abi.h (libkvf_hip.so).

This mirrors how the reference's own Python side binds the boundary
(bench/wsl/compare.py:42-45 builds kvf::Args with ctypes: 9 pointers, 9 ints,
1 float): the same structure, loaded through ctypes, with torch used only to
own device memory and streams. There is no fallback: if the HIP library is
missing, importing the runtime raises.
"""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
HIP_LIB = os.path.join(HERE, "libkvf_hip.so")
HOST_LIB = os.path.join(HERE, "libkvf_hostdata.so")

FMT_F16, FMT_INT8, FMT_INT4 = 0, 1, 2
ORD_HEAD, ORD_TOKEN = 0, 1
FMT_NAMES = {FMT_F16: "f16", FMT_INT8: "int8", FMT_INT4: "int4"}
FMT_BY_NAME = {v: k for k, v in FMT_NAMES.items()}

ABI_VERSION = 2  # KVF_ABI_VERSION of include/kvf_abi.h

HIP_SUCCESS = 0
HIP_ERROR_INVALID_VALUE = 1
HIP_ERROR_NOT_FOUND = 500


class KvfError(RuntimeError):
    pass


class Args(ctypes.Structure):
    """kvf::Args, field for field (runtime/kvf_kernels.cuh:29-46)."""
    _fields_ = [
        ("q", ctypes.c_void_p), ("k", ctypes.c_void_p), ("v", ctypes.c_void_p),
        ("k_meta", ctypes.c_void_p), ("v_meta", ctypes.c_void_p),
        ("block_table", ctypes.c_void_p), ("out", ctypes.c_void_p),
        ("part_o", ctypes.c_void_p), ("part_ml", ctypes.c_void_p),
        ("B", ctypes.c_int), ("H", ctypes.c_int), ("Hkv", ctypes.c_int), ("n", ctypes.c_int),
        ("splits", ctypes.c_int), ("warps", ctypes.c_int), ("group_shift", ctypes.c_int),
        ("block_shift", ctypes.c_int), ("max_blocks", ctypes.c_int),
        ("scale_log2", ctypes.c_float),
    ]


class VarlenArgs(ctypes.Structure):
    """kvf::VarlenArgs (the additive variable-length / f16 q-out extension)."""
    _fields_ = [("seq_lens", ctypes.c_void_p), ("q16", ctypes.c_void_p),
                ("out16", ctypes.c_void_p), ("flags", ctypes.c_int)]


VARLEN_LONGEST_FIRST = 1


_hip = None
_host = None


def hip_lib():
    """Load libkvf_hip.so; raise if it is not built (no silent fallback)."""
    global _hip
    if _hip is not None:
        return _hip
    if not os.path.exists(HIP_LIB):
        raise KvfError(f"{HIP_LIB} is missing: run __graft_entry__.build() "
                       "(or make -C kvforge_amd) first")
    L = ctypes.CDLL(HIP_LIB)
    P = ctypes.c_void_p
    I = ctypes.c_int
    L.kvf_launch_variant.restype = I
    L.kvf_launch_variant.argtypes = [ctypes.c_char_p, ctypes.POINTER(Args), P]
    L.kvf_launch_varlen_variant.restype = I
    L.kvf_launch_varlen_variant.argtypes = [ctypes.c_char_p, ctypes.POINTER(Args),
                                            ctypes.POINTER(VarlenArgs), P]
    L.kvf_launch_fused_variant.restype = I
    Z = ctypes.c_size_t
    L.kvf_launch_fused_variant.argtypes = [ctypes.c_char_p, ctypes.POINTER(Args),
                                           ctypes.POINTER(VarlenArgs), P, Z, P]
    L.kvf_launch_persistent_variant.restype = I
    L.kvf_launch_persistent_variant.argtypes = [ctypes.c_char_p, ctypes.POINTER(Args),
                                                ctypes.POINTER(VarlenArgs), P, Z, P, Z, I, P]
    L.kvf_launch_fused_variant_noalloc.restype = I
    L.kvf_launch_fused_variant_noalloc.argtypes = [ctypes.c_char_p, ctypes.POINTER(Args),
                                                   ctypes.POINTER(VarlenArgs), P]
    L.kvf_launch_partial_variant.restype = I
    L.kvf_launch_partial_variant.argtypes = [ctypes.c_char_p, ctypes.POINTER(Args), P]
    L.kvf_launch_partial_variant_timed.restype = I
    L.kvf_launch_partial_variant_timed.argtypes = [ctypes.c_char_p, ctypes.POINTER(Args), P, P, P]
    L.kvf_launch_partial_varlen_variant_timed.restype = I
    L.kvf_launch_partial_varlen_variant_timed.argtypes = [ctypes.c_char_p, ctypes.POINTER(Args),
                                                         ctypes.POINTER(VarlenArgs), P, P, P]
    L.kvf_launch_step_timed.restype = I
    L.kvf_launch_step_timed.argtypes = [ctypes.c_char_p, ctypes.POINTER(Args),
                                        ctypes.POINTER(VarlenArgs), P, Z, P, P, P]
    L.kvf_launch_merge.restype = I
    L.kvf_launch_merge.argtypes = [I, ctypes.POINTER(Args), P]
    L.kvf_variant_count.restype = I
    L.kvf_variant_count.argtypes = []
    L.kvf_variant_id.restype = ctypes.c_char_p
    L.kvf_variant_id.argtypes = [I]
    L.kvf_quantize_place.restype = I
    L.kvf_quantize_place.argtypes = [I, I, I, P, I, I, I, I, I, P, I, P, P, P]
    L.kvf_append_tokens.restype = I
    L.kvf_append_tokens.argtypes = [I, I, I, P, I, I, I, P, I, I, P, I, P, P, P]
    L.kvf_version.restype = ctypes.c_char_p
    L.kvf_version.argtypes = []
    L.kvf_abi_version.restype = I
    L.kvf_abi_version.argtypes = []
    if L.kvf_abi_version() != ABI_VERSION:
        raise KvfError(f"{HIP_LIB} has C ABI version {L.kvf_abi_version()}, this binding "
                       f"expects {ABI_VERSION}: rebuild the library")
    _hip = L
    return L


def host_lib():
    global _host
    if _host is not None:
        return _host
    if not os.path.exists(HOST_LIB):
        raise KvfError(f"{HOST_LIB} is missing: run __graft_entry__.build() first")
    L = ctypes.CDLL(HOST_LIB)
    P, I, U = ctypes.c_void_p, ctypes.c_int, ctypes.c_uint64
    L.kvfh_make_data.argtypes = [I, I, I, I, I, U, P, P, P]
    L.kvfh_page_table.argtypes = [ctypes.c_longlong, U, P]
    L.kvfh_inject_outliers.restype = I
    L.kvfh_inject_outliers.argtypes = [I, I, I, I, U, ctypes.c_double, ctypes.c_float, P, P]
    L.kvfh_varlen_lengths.argtypes = [I, I, I, U, P]
    L.kvfh_pool_table.restype = I
    L.kvfh_pool_table.argtypes = [I, P, I, I, U, I, P]
    _host = L
    return L


def check(err, what="kvf call"):
    if err != HIP_SUCCESS:
        raise KvfError(f"{what} failed with hipError {err}")


def variant_id(fmt, order, paged, pack, unroll, d):
    """src/codegen.cpp:59-65: "{fmt}_{hm|tm}_{c|p}_g{G}_u{U}_d{D}"."""
    f = FMT_NAMES[fmt] if isinstance(fmt, int) else fmt
    return f"{f}_{'hm' if order == ORD_HEAD else 'tm'}_{'p' if paged else 'c'}_g{pack}_u{unroll}_d{d}"


def variants():
    L = hip_lib()
    return [L.kvf_variant_id(i).decode() for i in range(L.kvf_variant_count())]


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _words(t):
    """Size in 32-bit words of a counter or queue buffer (0 for None)."""
    return 0 if t is None else t.numel() * t.element_size() // 4


def make_args(q, k, v, k_meta, v_meta, table, out, part_o, part_ml, B, H, Hkv, n,
              splits, warps, group=0, block_tokens=0, max_blocks=0, scale_log2=None, D=128):
    """Build Args the way runtime/kvf_host.h:273-294 does."""
    import math
    a = Args()
    a.q, a.k, a.v = (t.data_ptr() if t is not None else None for t in (q, k, v))
    a.k_meta = k_meta.data_ptr() if k_meta is not None else None
    a.v_meta = v_meta.data_ptr() if v_meta is not None else None
    a.block_table = table.data_ptr() if table is not None else None
    a.out = out.data_ptr() if out is not None else None
    a.part_o = part_o.data_ptr() if part_o is not None else None
    a.part_ml = part_ml.data_ptr() if part_ml is not None else None
    a.B, a.H, a.Hkv, a.n = B, H, Hkv, n
    a.splits, a.warps = splits, warps
    a.group_shift = int(round(math.log2(group))) if group else 0
    a.block_shift = int(round(math.log2(block_tokens))) if block_tokens else 0
    a.max_blocks = max_blocks
    if scale_log2 is None:
        import numpy as np
        scale_log2 = float(np.float32(np.float32(1.0) / np.sqrt(np.float32(D)))
                           * np.float32(1.4426950408889634))
    a.scale_log2 = scale_log2
    return a


def stream_handle(stream=None):
    import torch
    s = stream if stream is not None else torch.cuda.current_stream()
    return ctypes.c_void_p(s.cuda_stream)


def launch(vid, args, stream=None):
    err = hip_lib().kvf_launch_variant(vid.encode(), ctypes.byref(args), stream_handle(stream))
    check(err, f"kvf_launch_variant({vid})")


def launch_partial(vid, args, stream=None):
    err = hip_lib().kvf_launch_partial_variant(vid.encode(), ctypes.byref(args),
                                               stream_handle(stream))
    check(err, f"kvf_launch_partial_variant({vid})")


COUNTER_STRIDE = 32  # KVF_COUNTER_STRIDE: unsigned ints per merge counter
QUEUE_WORDS = 2 * COUNTER_STRIDE  # KVF_QUEUE_WORDS


def fused_counters(B, head_groups, device="cuda:0"):
    """Zeroed merge counters for kvf_launch_fused_variant: one 128-byte line
    per (sequence, head group)."""
    import torch
    return torch.zeros(B * head_groups * COUNTER_STRIDE, dtype=torch.int32, device=device)


def _varlen_args(seq_lens, q16=None, out16=None, flags=0):
    va = VarlenArgs()
    va.seq_lens = seq_lens.data_ptr() if seq_lens is not None else None
    va.q16 = q16.data_ptr() if q16 is not None else None
    va.out16 = out16.data_ptr() if out16 is not None else None
    va.flags = flags
    return va


def launch_fused(vid, args, counters, varlen=None, stream=None, flags=0):
    """One-launch decode step (split kernel + in-kernel merge); `counters`
    from fused_counters(), left zero afterwards."""
    va = None
    if varlen is not None:
        va = ctypes.byref(_varlen_args(*varlen, flags=flags))
    err = hip_lib().kvf_launch_fused_variant(vid.encode(), ctypes.byref(args), va,
                                             _ptr(counters), _words(counters),
                                             stream_handle(stream))
    check(err, f"kvf_launch_fused_variant({vid})")


def persistent_queue(device="cuda:0"):
    """Zeroed work queue for kvf_launch_persistent_variant (claim counter and
    done counter, one 128-byte line each), left zero by every call."""
    import torch
    return torch.zeros(QUEUE_WORDS, dtype=torch.int32, device=device)


def launch_persistent(vid, args, queue, counters=None, varlen=None, workgroups=0, stream=None, flags=0):
    """Persistent decode step: workgroups claim (sequence, head group, split)
    items from `queue` (persistent_queue()); with `counters`
    (fused_counters()) the merge runs inside the launch, without them the
    merge kernel follows. `workgroups` caps the grid (0: all resident)."""
    va = None
    if varlen is not None:
        va = ctypes.byref(_varlen_args(*varlen, flags=flags))
    err = hip_lib().kvf_launch_persistent_variant(vid.encode(), ctypes.byref(args), va,
                                                  _ptr(counters), _words(counters),
                                                  _ptr(queue), _words(queue), workgroups,
                                                  stream_handle(stream))
    check(err, f"kvf_launch_persistent_variant({vid})")


def launch_merge(d, args, stream=None):
    check(hip_lib().kvf_launch_merge(d, ctypes.byref(args), stream_handle(stream)),
          "kvf_launch_merge")


def launch_varlen(vid, args, seq_lens, q16=None, out16=None, stream=None, flags=0):
    """kvf_launch_varlen_variant; flags: VARLEN_LONGEST_FIRST or 0."""
    va = _varlen_args(seq_lens, q16, out16, flags)
    err = hip_lib().kvf_launch_varlen_variant(vid.encode(), ctypes.byref(args),
                                              ctypes.byref(va), stream_handle(stream))
    check(err, f"kvf_launch_varlen_variant({vid})")


_plans = {}


def plan_lib(name):
    """Load kvforge_amd/plans/libkvf_plan_<name>.so, the library `kvf plan`
    emitted for plans/<name>.kv (kvf_launch_<name>, kvf_plan_<name>, and
    kvf_launch_varlen_<name> when the program declares an f16 query or
    seq_lens); raise if it is not built."""
    if name in _plans:
        return _plans[name]
    path = os.path.join(HERE, "plans", f"libkvf_plan_{name}.so")
    if not os.path.exists(path):
        raise KvfError(f"{path} is missing: run __graft_entry__.build() (or make -C kvforge_amd) first")
    hip_lib()  # the plan library links against it
    L = ctypes.CDLL(path)
    getattr(L, f"kvf_launch_{name}").restype = ctypes.c_int
    getattr(L, f"kvf_launch_{name}").argtypes = [ctypes.POINTER(Args), ctypes.c_void_p]
    getattr(L, f"kvf_plan_{name}").restype = ctypes.c_char_p
    getattr(L, f"kvf_plan_{name}").argtypes = []
    if hasattr(L, f"kvf_launch_varlen_{name}"):
        fn = getattr(L, f"kvf_launch_varlen_{name}")
        fn.restype = ctypes.c_int
        fn.argtypes = [ctypes.POINTER(Args), ctypes.POINTER(VarlenArgs), ctypes.c_void_p]
    _plans[name] = L
    return L


def launch_plan_varlen(name, args, seq_lens, q16=None, out16=None, stream=None, flags=0):
    """kvf_launch_varlen_<name> of a planned program's library."""
    va = _varlen_args(seq_lens, q16, out16, flags)
    err = getattr(plan_lib(name), f"kvf_launch_varlen_{name}")(ctypes.byref(args), ctypes.byref(va),
                                                                stream_handle(stream))
    check(err, f"kvf_launch_varlen_{name}")


def quantize_place(fmt, group, d, x, B, Hkv, n, order, block_tokens, table, max_blocks,
                   data, meta, stream=None):
    """GPU KV append: fp32 logical rows -> codes + (scale, zero) in the layout."""
    err = hip_lib().kvf_quantize_place(
        fmt, group, d, _ptr(x), B, Hkv, n, order, block_tokens, _ptr(table), max_blocks,
        _ptr(data), _ptr(meta), stream_handle(stream))
    check(err, "kvf_quantize_place")


def append_tokens(fmt, group, d, x, B, Hkv, n, positions, order, block_tokens, table,
                  max_blocks, data, meta, stream=None):
    """GPU KV append of one token per sequence: x [B][Hkv][d] fp32 rows go to
    token positions[b] of each sequence, quantized exactly as quantize_place."""
    err = hip_lib().kvf_append_tokens(
        fmt, group, d, _ptr(x), B, Hkv, n, _ptr(positions), order, block_tokens, _ptr(table),
        max_blocks, _ptr(data), _ptr(meta), stream_handle(stream))
    check(err, "kvf_append_tokens")


def row_bytes(fmt, d):
    return d * {FMT_F16: 16, FMT_INT8: 8, FMT_INT4: 4}[fmt] // 8


def rows_alloc(B, Hkv, n, block_tokens):
    if not block_tokens:
        return B * Hkv * n, 0
    mb = (n + block_tokens - 1) // block_tokens
    return B * mb * Hkv * block_tokens, mb
