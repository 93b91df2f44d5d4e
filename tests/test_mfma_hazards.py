"""MFMA result hazards in the compiled kernels (CPU-only: hipcc -S, no GPU).

An instruction that reads or overwrites an MFMA's destination registers fewer
than 8 wait states after the MFMA sees a stale register. The compiler pads
inside a basic block, but a branch between the MFMA and the read has produced
reads 3-7 wait states later (the metric kernel's doc-tail mask once did, and
a test score came out 0.024 low). flash_maxsim_amd.hazard_check walks every
control-flow path; these tests pin the checker on small listings, then run it
over every kernel of the library.
"""

from __future__ import annotations

import pytest

from flash_maxsim_amd.build import _hipcc
from flash_maxsim_amd.hazard_check import check_asm, check_sources


def _have_hipcc() -> bool:
    try:
        _hipcc()
        return True
    except RuntimeError:
        return False


HEAD = "kern:\n"


def test_read_after_branch_flagged():
    asm = HEAD + """
	v_mfma_f32_16x16x32_f16 v[38:41], v[0:3], v[4:7], v[38:41]
	s_cbranch_vccnz .LBB0_2
	v_mov_b32_e32 v50, 0
	v_mov_b32_e32 v50, 0
	v_mov_b32_e32 v50, 0
	v_mov_b32_e32 v50, 0
	v_mov_b32_e32 v50, 0
	v_mov_b32_e32 v50, 0
	v_mov_b32_e32 v50, 0
	v_mov_b32_e32 v50, 0
.LBB0_2:
	v_maximum3_f32 v1, v1, v38, v39
	s_endpgm
"""
    f = check_asm(asm)
    assert len(f) == 1 and f[0].kind == "RAW" and f[0].wait_states == 1


def test_padded_read_clean_and_short_pad_flagged():
    ok = HEAD + "\tv_mfma_f32_16x16x32_f16 v[8:11], v[0:3], v[4:7], 0\n\ts_nop 7\n" \
                "\tv_maximum3_f32 v1, v8, v9, v9\n\ts_endpgm\n"
    bad = ok.replace("s_nop 7", "s_nop 5")
    assert check_asm(ok) == []
    f = check_asm(bad)
    assert [x.wait_states for x in f] == [6]


def test_overwrite_of_unread_result_flagged():
    asm = HEAD + """
	v_mfma_f32_16x16x32_f16 v[20:23], v[0:3], v[4:7], 0
	s_cbranch_execz .LBB0_3
	s_nop 7
.LBB0_3:
	v_add_u32_e32 v21, v35, v24
	s_endpgm
"""
    f = check_asm(asm)
    assert len(f) == 1 and f[0].kind == "WAW"


def test_loop_back_edge_flagged():
    asm = HEAD + """
.LBB0_1:
	v_maximum3_f32 v1, v1, v8, v9
	v_mfma_f32_16x16x32_f16 v[8:11], v[0:3], v[4:7], 0
	s_cbranch_scc1 .LBB0_1
	s_endpgm
"""
    f = check_asm(asm)
    assert len(f) == 1 and f[0].kind == "RAW"


def test_chained_mfma_not_flagged():
    # An MFMA taking the previous result as its accumulator is interlocked.
    asm = HEAD + "\tv_mfma_f32_16x16x32_f16 v[8:11], v[0:3], v[4:7], 0\n" \
                 "\tv_mfma_f32_16x16x32_f16 v[8:11], v[12:15], v[4:7], v[8:11]\n\ts_endpgm\n"
    assert check_asm(asm) == []


@pytest.mark.skipif(not _have_hipcc(), reason="hipcc not available")
def test_library_kernels_have_no_mfma_hazards():
    findings = check_sources()
    assert findings == [], "\n".join(f"{f.kernel}: {f.line} (+{f.wait_states} {f.kind}) {f.instr}" for f in findings[:10])
