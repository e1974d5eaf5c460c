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

pytestmark = pytest.mark.skipif(shutil.which("hipcc") is None and
                                not Path("/opt/rocm/bin/hipcc").exists(),
                                reason="hipcc is needed to build the device assembly")


def test_no_mfma_result_read_early_through_a_branch(tmp_path):
    listings = [mfma_hazards.device_assembly(CSRC / s, tmp_path / (s + ".s")) for s in MFMA_SOURCES]
    rule, cross, short = mfma_hazards.scan(listings)
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
