"""The LDS-read check of the DMA kernels' assembly (CPU: hipcc cross-compiles).

check_lds_reads.scan_kernel on planted instruction sequences, then the check
over the product sources: no vector instruction may touch the destination of
an inline-asm ds_read before an lgkmcnt wait covers it.
"""

from __future__ import annotations

import shutil
import sys
from pathlib import Path

import pytest

PKG = Path(__file__).resolve().parent.parent / "vllm-triton-fixed-point-reductions_amd"
sys.path.insert(0, str(PKG))
import check_lds_reads as C  # noqa: E402


def _scan(text: str) -> list[str]:
    return C.scan_kernel(text.strip().splitlines())


def test_use_before_wait_is_reported():
    hits = _scan("""
        ds_read_b128 v[0:3], v10
        v_mov_b32_e32 v20, v1
        s_waitcnt lgkmcnt(0)
        v_mov_b32_e32 v21, v2
    """)
    assert len(hits) == 1 and "v_mov_b32_e32 v20, v1" in hits[0]


def test_partial_wait_covers_the_older_reads_only():
    text = """
        ds_read_b128 v[0:3], v10
        ds_read_b128 v[4:7], v10 offset:16
        s_waitcnt lgkmcnt(1)
        v_mfma_f32_16x16x32_bf16 v[20:23], v[0:3], v[8:11], 0
        v_accvgpr_write_b32 a5, v6
    """
    hits = _scan(text)
    assert len(hits) == 1 and "a5, v6" in hits[0]


def test_writes_count_in_order_and_unrelated_registers_pass():
    hits = _scan("""
        ds_read_b128 v[0:3], v10
        ds_write_b16 v11, v12
        s_waitcnt lgkmcnt(1)
        v_add_u32_e32 v30, v0, v31
        v_add_u32_e32 v32, v33, v34
    """)
    assert hits == []


def test_no_fall_through_after_an_unconditional_branch():
    hits = _scan("""
        ds_read_b128 v[0:3], v10
        s_branch .LBB0_2
    .LBB0_1:
        v_mov_b32_e32 v20, v1
    """)
    assert hits == []


@pytest.mark.skipif(shutil.which("hipcc") is None and not Path("/opt/rocm/bin/hipcc").exists(),
                    reason="hipcc not available")
def test_product_dma_kernels_have_no_early_lds_uses(capsys):
    assert C.main([]) == 0, capsys.readouterr().out
