"""The inline-asm load lint (light_amd/csrc/vmcnt_check.py) on small hand-written gfx950
assembly: what it must flag (a spill / copy / reuse of a load destination before its wait)
and what it must not (uses after a covering wait, stores counted in vmcnt, direct-to-LDS
loads, a second load into a register already in flight)."""
import importlib.util
import os

import pytest

_SPEC = importlib.util.spec_from_file_location(
    "vmcnt_check", os.path.join(os.path.dirname(__file__), "..", "light_amd", "csrc", "vmcnt_check.py"))
vc = importlib.util.module_from_spec(_SPEC)
_SPEC.loader.exec_module(vc)


def _hits(tmp_path, body):
    f = tmp_path / "k.s"
    f.write_text("_ZN2hq1kEv:\n" + "\n".join("\t" + l for l in body) + "\n\ts_endpgm\n.Lfunc_end0:\n")
    return [(h[2], h[3]) for h in vc.check_asm(str(f))]


def test_copy_before_wait_is_flagged(tmp_path):
    hits = _hits(tmp_path, ["global_load_dword v0, v[10:11], off", "v_accvgpr_write_b32 a1, v0",
                            "s_waitcnt vmcnt(0)"])
    assert len(hits) == 1 and "reads v0" in hits[0][1]


def test_reuse_as_address_before_wait_is_flagged(tmp_path):
    hits = _hits(tmp_path, ["global_load_dwordx4 v[4:7], v[10:11], off", "v_mad_i64_i32 v[4:5], s[2:3], v13, s10, 0",
                            "s_waitcnt vmcnt(0)"])
    assert any("overwrites v4" in h[1] for h in hits)


def test_use_after_covering_wait_is_clean(tmp_path):
    # Two loads; vmcnt(1) retires the older one, so reading v0 is fine, v1 is not yet.
    assert _hits(tmp_path, ["global_load_dword v0, v[10:11], off", "global_load_dword v1, v[12:13], off",
                            "s_waitcnt vmcnt(1)", "v_add_u32_e32 v2, v0, v0"]) == []
    hits = _hits(tmp_path, ["global_load_dword v0, v[10:11], off", "global_load_dword v1, v[12:13], off",
                            "s_waitcnt vmcnt(1)", "v_add_u32_e32 v2, v1, v1"])
    assert len(hits) == 1 and "reads v1" in hits[0][1]


def test_stores_count_in_vmcnt(tmp_path):
    # After the load, a store; vmcnt(1) leaves only the store outstanding: v9 has landed.
    assert _hits(tmp_path, ["global_load_dword v9, v[6:7], off", "global_store_dword v[0:1], v8, off",
                            "s_waitcnt vmcnt(1)", "v_bfe_u32 v0, v9, v4, 4"]) == []


def test_direct_to_lds_load_has_no_vgpr_result(tmp_path):
    # global_load_lds_dwordx4's operand is its address: writing it afterwards is fine.
    assert _hits(tmp_path, ["global_load_lds_dwordx4 v[2:3], off", "v_lshl_add_u64 v[2:3], v[4:5], 0, 16"]) == []


def test_second_load_into_in_flight_register_is_not_flagged(tmp_path):
    # Loads return in order: the later one's data is what stays.
    assert _hits(tmp_path, ["global_load_dwordx4 v[60:63], v[20:21], off offset:16",
                            "global_load_dword v60, v[20:21], off", "s_waitcnt vmcnt(0)"]) == []


def test_state_crosses_blocks(tmp_path):
    # The in-flight state follows the branch: a use in the target block before a wait is flagged.
    hits = _hits(tmp_path, ["global_load_dword v0, v[10:11], off", "s_branch .LBB0_1", ".LBB0_1:",
                            "v_add_u32_e32 v2, v0, v0"])
    assert len(hits) == 1 and "reads v0" in hits[0][1]
    assert _hits(tmp_path, ["global_load_dword v0, v[10:11], off", "s_branch .LBB0_1", ".LBB0_1:",
                            "s_waitcnt vmcnt(0)", "v_add_u32_e32 v2, v0, v0"]) == []


def test_merge_takes_the_worst_edge(tmp_path):
    # One edge waited, the fall-through did not: the join still has v0 in flight.
    hits = _hits(tmp_path, ["global_load_dword v0, v[10:11], off", "s_cbranch_scc1 .LBB0_2",
                            "s_waitcnt vmcnt(0)", ".LBB0_2:", "v_add_u32_e32 v2, v0, v0"])
    assert len(hits) == 1 and "reads v0" in hits[0][1]


_RING = ["global_load_dwordx4 v[4:7], v[10:11], off",      # slot 0, before the loop
         "global_load_dwordx4 v[8:11], v[12:13], off",     # slot 1
         ".LBB0_1:",
         "s_waitcnt vmcnt(1)",                             # slot 0 has landed
         "v_add_u32_e32 v20, v4, v4",
         "global_load_dwordx4 v[4:7], v[14:15], off",      # refill slot 0
         "s_waitcnt vmcnt(1)",                             # slot 1 has landed
         "v_add_u32_e32 v21, v8, v8",
         "global_load_dwordx4 v[8:11], v[16:17], off"]     # refill slot 1


def test_loop_carried_ring_is_clean(tmp_path):
    assert _hits(tmp_path, _RING + ["s_cbranch_scc1 .LBB0_1"]) == []


def test_loop_carried_copy_at_latch_is_flagged(tmp_path):
    # The compiler's phi copy of an in-flight slot at the back edge (the faulting pattern).
    hits = _hits(tmp_path, _RING + ["v_mov_b32_e32 v30, v5", "s_cbranch_scc1 .LBB0_1"])
    assert any(h[0] and "reads v5" in h[1] for h in hits)


def test_loop_carried_early_use_is_flagged(tmp_path):
    # A wait that is right on the first iteration but not once the loop has refilled both slots.
    body = ["global_load_dwordx4 v[4:7], v[10:11], off", ".LBB0_1:", "s_waitcnt vmcnt(0)",
            "v_add_u32_e32 v20, v4, v4", "global_load_dwordx4 v[4:7], v[14:15], off",
            "global_load_dwordx4 v[8:11], v[16:17], off", "s_waitcnt vmcnt(2)", "v_add_u32_e32 v21, v8, v8",
            "s_cbranch_scc1 .LBB0_1"]
    hits = _hits(tmp_path, body)
    assert len(hits) == 1 and "reads v8" in hits[0][1]


@pytest.mark.parametrize("line,regs", [("v7", [7]), ("v[2:5]", [2, 3, 4, 5]), ("s7", []), ("a[0:3]", [])])
def test_vgpr_operands(line, regs):
    assert list(vc.vgprs(line)) == regs


@pytest.mark.skipif(not os.path.exists(vc.HIPCC), reason="hipcc not installed")
@pytest.mark.parametrize("src", ["int4_small.hip", "gemm.hip", "int4_cu.hip", "moe_stream.hip"])
def test_real_sources_are_clean(src):
    """The kernels that load from inline asm with hand-counted waits, compiled as the library
    is: no in-flight destination is touched, across blocks and loop back edges."""
    path = os.path.join(vc.HERE, src)
    assert vc.main(["vmcnt_check.py", path]) == 0
