"""The static check behind the GEMM's untracked B loads (hmoe.isa_check):
small listings with a known answer, each a plausible scheduling or
register-allocation mistake (a use before the wait, a wait that counts one
load too few, a branch around the wait, a loop back edge, a spill), and the
listing the build saved for hm_gemm_mfma.hip."""
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
    younger = "\tbuffer_load_dwordx4 v12, s[0:3], s5 offen lds\n"
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
    text = HEAD + "\tbuffer_load_dwordx4 v4, s[0:3], s4 offen lds\n\tv_mov_b32_e32 v20, v4\n" + \
        "\ts_waitcnt vmcnt(0)\n" + END
    assert bad(text) == 0


def test_built_gemm_listing_is_clean():
    listing = _device_listing(OBJ / "hm_gemm_mfma.o")
    if not listing.exists():
        pytest.skip("no saved listing (library not built here)")
    text = Path(listing).read_text()
    assert "limb_gemm_kernel" in text
    assert isa_check.check_text(text) == []
