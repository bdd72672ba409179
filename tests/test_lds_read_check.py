"""The generated-assembly checks of the kernels (CPU: hipcc cross-compiles).

check_lds_reads.scan_kernel and scan_mfma_reads on planted instruction
sequences, then both checks over the product sources: no vector instruction
may touch the destination of an inline-asm ds_read before an lgkmcnt wait
covers it, and no inline-asm instruction may name an MFMA's destination
registers fewer than MFMA_WAIT_STATES wait states after it.
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


def test_lds_address_that_is_a_pending_destination_is_reported():
    # two reads in one asm statement whose outputs are not early-clobber:
    # the compiler may make the first read's destination the second's
    # address, which the first read overwrites if it lands first
    hits = _scan("""
        ds_read_u16 v1, v0
        ds_read_b32 v0, v1
        s_waitcnt lgkmcnt(0)
    """)
    assert len(hits) == 1 and "ds_read_b32 v0, v1" in hits[0]
    # a write's data register counts as well; distinct registers pass
    assert len(_scan("""
        ds_read_b32 v1, v0
        ds_write_b32 v2, v1
    """)) == 1
    assert _scan("""
        ds_read_u16 v1, v0
        ds_read_b32 v2, v3
        s_waitcnt lgkmcnt(0)
    """) == []


def test_no_fall_through_after_an_unconditional_branch():
    hits = _scan("""
        ds_read_b128 v[0:3], v10
        s_branch .LBB0_2
    .LBB0_1:
        v_mov_b32_e32 v20, v1
    """)
    assert hits == []


def _mfma(text: str) -> list[str]:
    return C.scan_mfma_reads(text.strip("\n").splitlines())


MFMA = "v_mfma_f32_16x16x32_bf16 v[34:37], v[18:21], v[84:87], v[34:37]"
ASM_MAX = ";;#ASMSTART\nv_maximum3_f32 v84, |v34|, |v35|, |v36|\n;;#ASMEND"


def test_asm_read_right_after_an_mfma_is_reported():
    hits = _mfma(f"{MFMA}\n{ASM_MAX}")
    assert len(hits) == 1 and "0 wait states" in hits[0]


def test_nops_and_instructions_count_as_wait_states():
    # s_nop N gives N + 1: 8 + 8 + 1 + 1 = 18 wait states is one short
    between = "s_nop 7\ns_nop 7\nv_add_u32_e32 v1, v2, v3\ns_add_i32 s0, s0, 1"
    assert len(_mfma(f"{MFMA}\n{between}\n{ASM_MAX}")) == 1
    assert _mfma(f"{MFMA}\n{between}\ns_nop 0\n{ASM_MAX}") == []


def test_loop_back_edge_is_followed():
    hits = _mfma(f""".LBB0_1:
{ASM_MAX}
v_add_u32_e32 v1, v2, v3
{MFMA}
s_cbranch_scc1 .LBB0_1""")
    assert len(hits) == 1 and "1 wait states" in hits[0]


def test_compiler_generated_use_ends_the_trace():
    # the compiler keeps the wait states before its own read of v34..v36 (or
    # write of them): the MFMA's write has landed by then
    uses = "s_nop 7\nv_mul_f32_e32 v34, v34, v41\nv_mul_f32_e32 v35, v35, v41\nv_mul_f32_e32 v36, v36, v41"
    assert _mfma(f"{MFMA}\n{uses}\n{ASM_MAX}") == []


@pytest.mark.skipif(shutil.which("hipcc") is None and not Path("/opt/rocm/bin/hipcc").exists(),
                    reason="hipcc not available")
def test_product_kernels_have_no_early_lds_or_mfma_uses(capsys):
    assert C.main([]) == 0, capsys.readouterr().out
