"""The static check behind the hand-written memory statements
(hmoe.isa_check): small listings with a known answer, each a plausible
scheduling or register-allocation mistake (a use before the wait, a wait
that counts one load too few, a branch around the wait, a loop back edge, a
spill, compiler code that keeps a value in M0 or uses it implicitly, an
unrecognised memory form inside a hand-written block), and the listings the
build saved for the three sources it checks."""
from __future__ import annotations

from pathlib import Path

import pytest

from hmoe import isa_check
from hmoe.build import OBJ, _device_listing

HEAD = "k:\n"
LOAD = "\tbuffer_load_dwordx4 v[4:7], v0, s[0:3], s4 offen\n"
USE = "\tv_mfma_i32_32x32x32_i8 a[0:15], v[8:11], v[4:7], a[0:15]\n"
END = "\ts_endpgm\n"


def bad(text: str) -> int:
    return len(isa_check.check_text(text))


def test_wait_then_use_is_clean():
    assert bad(HEAD + LOAD + "\ts_waitcnt vmcnt(0)\n" + USE + END) == 0


def test_use_before_wait_is_flagged():
    assert bad(HEAD + LOAD + USE + "\ts_waitcnt vmcnt(0)\n" + END) >= 1


def test_count_covers_younger_loads_only():
    younger = "\t;;#ASMSTART\n\tbuffer_load_dwordx4 v12, s[0:3], s5 offen lds\n\t;;#ASMEND\n"
    # one younger load: vmcnt(1) completes the first load, vmcnt(2) does not
    assert bad(HEAD + LOAD + younger + "\ts_waitcnt vmcnt(1)\n" + USE + "\ts_waitcnt vmcnt(0)\n" + END) == 0
    assert bad(HEAD + LOAD + younger + "\ts_waitcnt vmcnt(2)\n" + USE + "\ts_waitcnt vmcnt(0)\n" + END) >= 1
    # a combined wait counts too; an lgkmcnt-only wait does not
    assert bad(HEAD + LOAD + "\ts_waitcnt vmcnt(0) lgkmcnt(0)\n" + USE + END) == 0
    assert bad(HEAD + LOAD + "\ts_waitcnt lgkmcnt(0)\n" + USE + "\ts_waitcnt vmcnt(0)\n" + END) >= 1


def test_branch_around_the_wait_is_flagged():
    text = HEAD + LOAD + "\ts_cbranch_scc1 .LBB0_1\n\ts_waitcnt vmcnt(0)\n.LBB0_1:\n" + USE + \
        "\ts_waitcnt vmcnt(0)\n" + END
    assert bad(text) >= 1


def test_loop_back_edge_reaches_the_use():
    text = HEAD + ".LBB0_1:\n" + USE + LOAD + "\ts_cbranch_scc1 .LBB0_1\n\ts_waitcnt vmcnt(0)\n" + END
    assert bad(text) >= 1
    ok = HEAD + ".LBB0_1:\n" + USE + LOAD + "\ts_waitcnt vmcnt(0)\n\ts_cbranch_scc1 .LBB0_1\n" + END
    assert bad(ok) == 0


def test_spill_or_copy_of_an_inflight_register_is_flagged():
    assert bad(HEAD + LOAD + "\tscratch_store_dword off, v5, off offset:4\n\ts_waitcnt vmcnt(0)\n" + END) >= 1
    assert bad(HEAD + LOAD + "\tv_mov_b32_e32 v20, v7\n\ts_waitcnt vmcnt(0)\n" + END) >= 1
    # an unrelated register is fine
    assert bad(HEAD + LOAD + "\tv_mov_b32_e32 v20, v8\n\ts_waitcnt vmcnt(0)\n" + END) == 0


def test_missing_wait_before_the_end_is_flagged():
    assert bad(HEAD + LOAD + END) >= 1


def test_lds_loads_write_no_registers():
    text = HEAD + "\t;;#ASMSTART\n\tbuffer_load_dwordx4 v4, s[0:3], s4 offen lds\n\t;;#ASMEND\n" + \
        "\tv_mov_b32_e32 v20, v4\n\ts_waitcnt vmcnt(0)\n" + END
    assert bad(text) == 0


ASM_DMA = "\t;;#ASMSTART\n\ts_mov_b32 m0, s6\n\tglobal_load_lds_dwordx4 v[2:3], off\n\t;;#ASMEND\n"


def test_compiler_code_must_leave_m0_alone():
    # the hand-written DMA sets M0 itself: clean
    assert bad(HEAD + ASM_DMA + "\ts_waitcnt vmcnt(0)\n" + END) == 0
    # the compiler keeping a value of its own in M0 (written, or read)
    assert bad(HEAD + "\ts_mov_b32 m0, -1\n" + ASM_DMA + "\ts_waitcnt vmcnt(0)\n" + END) >= 1
    assert bad(HEAD + ASM_DMA + "\ts_add_u32 s8, m0, 4\n\ts_waitcnt vmcnt(0)\n" + END) >= 1
    # instructions that use M0 without naming it
    assert bad(HEAD + "\tv_movrels_b32_e32 v1, v2\n" + END) >= 1
    assert bad(HEAD + "\ts_sendmsg sendmsg(MSG_INTERRUPT)\n" + END) >= 1
    assert bad(HEAD + "\tglobal_load_lds_dword v[2:3], off\n\ts_waitcnt vmcnt(0)\n" + END) >= 1
    assert bad(HEAD + "\tbuffer_load_dword v4, s[0:3], s5 offen lds\n\ts_waitcnt vmcnt(0)\n" + END) >= 1
    # an unrelated scalar register is fine
    assert bad(HEAD + "\ts_mov_b32 s9, s6\n" + ASM_DMA + "\ts_waitcnt vmcnt(0)\n" + END) == 0


def test_unrecognised_memory_forms_in_blocks_are_flagged():
    def blk(line):
        return HEAD + "\t;;#ASMSTART\n" + line + "\t;;#ASMEND\n\ts_waitcnt vmcnt(0)\n" + END
    # the recognised forms
    assert bad(blk(LOAD)) == 0
    assert bad(blk("\tbuffer_load_dwordx4 v4, s[0:3], s5 offen lds\n")) == 0
    assert bad(blk("\tglobal_load_lds_dword v[2:3], off\n")) == 0
    # an AGPR destination, another width, a register global load, a store
    assert bad(blk("\tbuffer_load_dwordx4 a[0:3], v0, s[0:3], s4 offen\n")) >= 1
    assert bad(blk("\tbuffer_load_dword v4, v0, s[0:3], s4 offen\n")) >= 1
    assert bad(blk("\tglobal_load_dwordx4 v[4:7], v[0:1], off\n")) >= 1
    assert bad(blk("\tglobal_store_dword v[0:1], v4, off\n")) >= 1


@pytest.mark.parametrize("source", ["hm_gemm_mfma", "hm_router", "hm_gemm_f32_mfma"])
def test_built_listings_are_clean(source):
    listing = _device_listing(OBJ / f"{source}.o")
    if not listing.exists():
        pytest.skip("no saved listing (library not built here)")
    assert isa_check.check_text(Path(listing).read_text()) == []


def test_built_gemm_listing_is_clean():
    listing = _device_listing(OBJ / "hm_gemm_mfma.o")
    if not listing.exists():
        pytest.skip("no saved listing (library not built here)")
    text = Path(listing).read_text()
    assert "limb_gemm_kernel" in text
    assert isa_check.check_text(text) == []
