"""MFMA results are never read through a branch sooner than the compiler's own in-block rule.

The fp16 and bf16-split attention kernels read their score accumulators with VALU right after the
QK^T chain, and one path to that read goes through the branch that skips the causal masking, where
the compiler adds no wait states. mfma_result_fence covers it. This test builds the device
assembly of every MFMA kernel source, takes the compiler's own minimum distance per opcode inside a
block as the rule, and checks every dependent read reached through a branch against it. The same
scan of attention.hip with the fence emptied must find the short reads (so the scan can see them).
"""

import shutil
from pathlib import Path

import pytest

from tests import mfma_hazards
from tessery_amd import _build

CSRC = _build.PACKAGE / "csrc"
MFMA_SOURCES = ("attention.hip", "qkv4.hip", "linear4.hip", "dense.hip")
ALL_SOURCES = MFMA_SOURCES + ("norm_rope.hip", "model.hip", "util.hip", "noalloc.hip")

pytestmark = pytest.mark.skipif(shutil.which("hipcc") is None and
                                not Path("/opt/rocm/bin/hipcc").exists(),
                                reason="hipcc is needed to build the device assembly")


@pytest.fixture(scope="module")
def assembly(tmp_path_factory):
    """gfx950 assembly of every device source, built once for the scans below."""
    out = tmp_path_factory.mktemp("asm")
    return {s: mfma_hazards.device_assembly(CSRC / s, out / (s + ".s")) for s in ALL_SOURCES}


def test_no_mfma_result_read_early_through_a_branch(assembly):
    rule, cross, short = mfma_hazards.scan([assembly[s] for s in MFMA_SOURCES])
    assert "v_mfma_f32_16x16x32_f16" in rule and "v_mfma_f32_16x16x32_bf16" in rule
    assert len(cross) > 50  # the attention kernels' score reads behind the masking branch
    assert short == [], short[:5]


def test_scan_finds_the_score_read_without_the_fence(tmp_path):
    src = tmp_path / "csrc"
    shutil.copytree(CSRC, src)
    text = (src / "attention.hip").read_text()
    fenced = text.count('asm volatile("s_nop 7\\n\\ts_nop 3"')
    assert fenced == 2
    text = text.replace('asm volatile("s_nop 7\\n\\ts_nop 3"', 'asm volatile(""')
    (src / "attention.hip").write_text(text)
    asm = mfma_hazards.device_assembly(src / "attention.hip", tmp_path / "attention.s")
    _, _, short = mfma_hazards.scan([asm])
    assert any(op == "v_mfma_f32_16x16x32_f16" and t.startswith("v_max_f32")
               for op, _, _, _, _, t in short)


def test_inline_asm_reads_no_fresh_valu_result(assembly):
    """Every inline asm vector memory instruction comes at least 5 wait states after any VALU
    write of its SGPR base (the persistent attention loop restores spilled SGPRs with v_readlane
    right before the table loads), and every inline asm VALU instruction at least one after a
    transcendental whose result it reads, on every path."""
    assert mfma_hazards.inline_asm_hazards(list(assembly.values())) == []


def test_inline_asm_scan_sees_short_distances():
    """A v_readlane restoring a spilled SGPR base right before an asm table load (the pattern of
    the memory fault that made the wait states in the asm helpers necessary: the load took a stale
    base address), and a v_rsq result read by the asm split with no wait state between; with the
    helpers' wait states in the asm statements, neither is reported."""
    def listing(nop_vmem, nop_valu):
        return "\n".join([
            "_Zk:",
            "\tv_readlane_b32 s8, v127, 4",
            "\tv_readlane_b32 s9, v127, 5",
            "\t;;#ASMSTART",
            *(["\ts_nop 4"] if nop_vmem else []),
            "\tglobal_load_dwordx4 v[2:5], v11, s[8:9] offset:0",
            "\t;;#ASMEND",
            "\tv_rsq_f32_e32 v6, v6",
            "\t;;#ASMSTART",
            *(["\ts_nop 0"] if nop_valu else []),
            "\tv_fma_mixlo_f16 v7, v8, v6, 0",
            "\t;;#ASMEND",
            "\ts_endpgm",
            ".Lfunc_end0:"])
    found = mfma_hazards.inline_asm_hazards([listing(False, False)])
    assert [(t.split()[0], waited, w.split()[0]) for _, t, waited, w in found] == [
        ("global_load_dwordx4", 0, "v_readlane_b32"), ("v_fma_mixlo_f16", 0, "v_rsq_f32_e32")]
    assert mfma_hazards.inline_asm_hazards([listing(True, True)]) == []


def test_inline_asm_scan_sees_an_mfma_reading_an_asm_result():
    """An MFMA reading a V fragment that an asm v_mov_b64 copied the instruction before: the
    compiler adds no wait state after an asm statement, so the statement carries its own two."""
    def listing(nop):
        return "\n".join([
            "_Zk:",
            "\t;;#ASMSTART",
            "\tv_mov_b64 v[100:101], v[98:99]",
            *(["\ts_nop 1"] if nop else []),
            "\t;;#ASMEND",
            "\tv_mfma_f32_16x16x32_f16 v[62:65], v[98:101], v[72:75], v[62:65]",
            "\ts_endpgm",
            ".Lfunc_end0:"])
    found = mfma_hazards.inline_asm_hazards([listing(False)])
    assert [(t.split()[0], waited, w.split()[0]) for _, t, waited, w in found] == [
        ("v_mfma_f32_16x16x32_f16", 0, "v_mov_b64")]
    assert mfma_hazards.inline_asm_hazards([listing(True)]) == []


def test_no_instruction_touches_a_register_an_asm_load_is_filling(assembly):
    """The table, q and activation loads issued as inline asm are invisible to the compiler's wait
    placement: no instruction may read or overwrite their destination registers (as a spill, a
    copy or a reuse for another value) before a vmcnt wait has retired them, on any path."""
    assert mfma_hazards.asm_load_reuse(list(assembly.values())) == []


def test_asm_load_scan_sees_an_early_read():
    listing = "\n".join([
        "_Zk:",
        "\t;;#ASMSTART",
        "\tglobal_load_dwordx4 v[6:9], v1, s[2:3] offset:0",
        "\t;;#ASMEND",
        "\tglobal_load_dword v20, v[2:3], off",
        "\ts_waitcnt vmcnt({n})",
        "\tv_add_f32_e32 v10, v6, v7",
        "\ts_endpgm",
        ".Lfunc_end0:"])
    assert mfma_hazards.asm_load_reuse([listing.format(n=1)]) == []
    assert mfma_hazards.asm_load_reuse([listing.format(n=2)]) == [("_Zk", "v_add_f32_e32 v10, v6, v7")]


def test_no_kernel_uses_scratch(assembly):
    """Every kernel keeps its arrays in registers: a helper lambda that the compiler does not
    inline takes the accumulator arrays it captures by reference into scratch memory (qkv4_f16
    ran six times slower so, with no spill reported)."""
    import re

    sizes = {s: [int(n) for n in re.findall(r"^\s*\.amdhsa_private_segment_fixed_size (\d+)",
                                            assembly[s], re.M)] for s in ALL_SOURCES}
    assert sum(map(len, sizes.values())) > 40  # every kernel of the library
    assert {s: v for s, v in sizes.items() if any(v)} == {}
