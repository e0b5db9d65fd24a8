"""CPU checks of the measurement tools under kvforge_amd/tools: the per-wave
timeline's stamp anchors still name one place each in the kernel sources, and
the resource table's loop selection takes the unmasked copy of the main loop."""
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
TOOLS = os.path.join(ROOT, "kvforge_amd", "tools")
sys.path.insert(0, TOOLS)

import dump_resources  # noqa: E402
import timeline  # noqa: E402


def test_timeline_stamp_anchors_name_one_place_each():
    src = os.path.join(ROOT, "kvforge_amd", "csrc")
    texts = {f: open(os.path.join(src, f)).read()
             for f in ("kvf_kernels.hpp", "kvf_ext.hpp", "kvf_runtime.hip", "kvf_merge.hip")}
    patches = timeline._patches()
    assert len(patches) >= 10
    for f, old, new in patches:
        assert texts[f].count(old) == 1, (f, old[:80])
        assert new.count(old.strip().split("\n")[0].strip()) >= 1, (f, old[:80])


def test_timeline_instantiates_the_benchmarked_plans():
    assert timeline._inst("int8_hm_c_g4_u2_d128") == "kvf::FMT_INT8, 128, 4, 2, kvf::ORD_HEAD, false"
    assert timeline._inst("int8_tm_p_g4_u2_d128") == "kvf::FMT_INT8, 128, 4, 2, kvf::ORD_TOKEN, true"
    assert timeline._inst("int4_hm_c_g4_u2_d128") == "kvf::FMT_INT4, 128, 4, 2, kvf::ORD_HEAD, false"


def _asm(loops):
    """A kernel body in the assembler's layout: each loop is a header block and
    one more block inside it, holding the given instructions."""
    lines, n = [], 0
    for body in loops:
        hdr = f".LBB0_{n}"
        lines.append(f"{hdr}: ; Loop Header: Depth=1")
        lines += [f"\t{op} v0, v1" for op in body[: len(body) // 2]]
        lines.append(f".LBB0_{n + 1}: ;   in Loop: Header=BB0_{n} Depth=1")
        lines += [f"\t{op} v0, v1" for op in body[len(body) // 2:]]
        n += 2
    return lines


def test_loop_mix_takes_the_unmasked_copy():
    # two loops with the same MFMA count: the masked copy carries extra
    # vector instructions (selects), the unmasked one is what chunks that
    # start on a tile boundary run
    masked = ["v_mfma_f32_16x16x32_f16"] * 8 + ["v_cndmask_b32"] * 40 + ["v_add_f32"] * 100
    unmasked = ["v_mfma_f32_16x16x32_f16"] * 8 + ["v_add_f32"] * 100 + ["s_add_u32"] * 6
    for order in ((masked, unmasked), (unmasked, masked)):
        mix = dump_resources.loop_mix(_asm(order))
        assert mix["mfma"] == 8 and mix["valu"] == 100 and mix["salu"] == 6, mix
    # a loop with more MFMAs wins regardless of its vector count
    bigger = ["v_mfma_f32_16x16x32_f16"] * 16 + ["v_add_f32"] * 400
    mix = dump_resources.loop_mix(_asm((unmasked, bigger)))
    assert mix["mfma"] == 16 and mix["valu"] == 400, mix


def test_mfma_per_tile_follows_the_column_geometry():
    # f16 d128 (COLS = g): 2 x 4 QK steps + 8 PV steps per pass and half
    assert dump_resources.mfma_per_tile(0, 128, 0, 4) == 16
    # int8:64 d128 g4: COLS = 8, hi and lo in one MFMA
    assert dump_resources.mfma_per_tile(1, 128, 64, 4) == 16
    # int4:32 d128 g4: COLS = 16, hi and lo in separate MFMAs
    assert dump_resources.mfma_per_tile(2, 128, 32, 4) == 32
    # int4:32 d128 g8: COLS = 32, two passes
    assert dump_resources.mfma_per_tile(2, 128, 32, 8) == 64
