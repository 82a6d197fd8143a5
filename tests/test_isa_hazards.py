"""The built gfx950 code object keeps the wait states that the compiler cannot insert
inside inline assembly (CPU: disassembles the library built here; no GPU).

The checker itself is pinned first on planted cases: the 16-byte store whose data
registers the next-but-one instruction overwrote (the sequence of a build that stored
wrong values on the GPU), and an M0 write directly before an LDS DMA.
"""

from __future__ import annotations

from pathlib import Path

import pytest

from tests import isa_hazards as H

LIB = Path(__file__).resolve().parents[1] / "muon_fusion_ascend950_amd" / "libmuon_polar.so"


def _func(body: str):
    return H.parse("0000000000001000 <k>:\n" + body)[0]


def test_checker_flags_a_store_whose_data_is_overwritten_too_soon():
    # one SALU between the store and the VALU write of its data: one wait state of two
    bad = _func("""
	global_store_dwordx4 v[22:23], v[24:27], off sc1   // 0
	s_mov_b64 s[8:9], 0x800                             // 8
	v_lshl_add_u64 v[24:25], v[18:19], 0, s[8:9]        // 10
""")
    assert H.store_data_violations(bad) == [0]
    # two instructions between: enough
    ok = _func("""
	buffer_store_dwordx4 v[26:29], v14, s[12:15], 0 offen sc1
	s_and_saveexec_b64 s[38:39], s[4:5]
	s_cbranch_execz 65288
	v_lshlrev_b32_e32 v26, 16, v2
""")
    assert H.store_data_violations(ok) == []
    # s_nop 1 gives two wait states; a VALU write of other registers is no hazard
    assert H.store_data_violations(_func("""
	buffer_store_dwordx4 v[0:3], v9, s[0:3], 0 offen sc1
	s_nop 1
	v_mov_b32_e32 v1, 0
""")) == []
    assert H.store_data_violations(_func("""
	buffer_store_dwordx4 v[0:3], v9, s[0:3], 0 offen sc1
	v_mov_b32_e32 v4, 0
""")) == []
    # 8-byte stores are not subject to the rule
    assert H.store_data_violations(_func("""
	global_store_dwordx2 v[0:1], v[2:3], off
	v_mov_b32_e32 v2, 0
""")) == []


def test_checker_flags_an_m0_write_right_before_an_lds_dma():
    assert H.m0_dma_violations(_func("""
	s_mov_b32 m0, s35
	buffer_load_dwordx4 v8, s[40:43], 0 offen lds
""")) == [1]
    assert H.m0_dma_violations(_func("""
	s_mov_b32 m0, s14
	s_nop 0
	buffer_load_dwordx4 v8, s[36:39], 0 offen lds
""")) == []
    assert H.m0_dma_violations(_func("""
	s_mov_b32 m0, s14
	v_cndmask_b32_e32 v8, v45, v8, vcc
	buffer_load_dwordx4 v8, s[36:39], 0 offen lds
""")) == []
    # a load without the lds modifier does not read M0
    assert H.m0_dma_violations(_func("""
	s_mov_b32 m0, s35
	buffer_load_dwordx4 v[8:11], v1, s[40:43], 0 offen
""")) == []


def test_built_code_object_keeps_both_wait_states():
    if not LIB.exists():
        pytest.skip("libmuon_polar.so is not built")
    if not H.tools_available():
        pytest.skip("ROCm LLVM tools (llvm-objcopy, clang-offload-bundler, llvm-objdump) missing")
    res = H.scan(H.disassemble_library(LIB))
    # the scan found the code: the DMA-fed kernels' loads and the 16-byte stores
    assert res["lds_dma"] > 1000 and res["wide_stores"] > 1000, res
    assert res["m0_dma"] == [], res["m0_dma"][:5]
    assert res["store_data"] == [], res["store_data"][:5]
