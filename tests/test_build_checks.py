"""The build's checks of the generated code (CPU): hot-loop direct-to-LDS loads and wide stores.

A vector instruction that writes an SGPR (a spill reload by v_readlane, v_readfirstlane) needs five
wait states before a vector memory instruction reads that SGPR; the compiler does not check inline
asm. The hot loads carry one wait state (M0's), so the build scans the generated code and falls back
to five everywhere if a load could read a freshly written resource or offset.

A store wider than 64 bits reads its data registers after it issues; a VALU write to one of them
right after the store (seen in the compiler's output for the adaLN bf16 store, where some lanes then
stored the new value) fails the build.
"""

import importlib.util
import pathlib

ROOT = pathlib.Path(__file__).resolve().parents[1]
_spec = importlib.util.spec_from_file_location("wanmi_build", ROOT / "vllm-omni-neuron_amd" / "build.py")
build = importlib.util.module_from_spec(_spec)
_spec.loader.exec_module(build)


def _asm(*lines):
    return "\n".join("\t" + ln if not ln.endswith(":") else ln for ln in lines) + "\n"


def test_flags_a_spill_reload_feeding_the_offset():
    asm = _asm("v_readlane_b32 s50, v255, 7", "s_nop 0", "buffer_load_dword v0, s[44:47], s50 offen lds")
    assert len(build.dma_sgpr_hazards(asm)) == 1


def test_flags_a_vector_write_of_the_resource():
    asm = _asm("v_readfirstlane_b32 s45, v3", "s_mov_b32 m0, s2", "s_nop 0",
               "buffer_load_dwordx4 v0, s[44:47], 0 offen lds")
    assert len(build.dma_sgpr_hazards(asm)) == 1


def test_five_wait_states_are_enough():
    asm = _asm("v_readlane_b32 s50, v255, 7", "s_nop 4", "buffer_load_dword v0, s[44:47], s50 offen lds")
    assert build.dma_sgpr_hazards(asm) == []
    asm = _asm("v_readlane_b32 s50, v255, 7", "s_mov_b32 s1, s2", "s_mov_b32 s3, s4", "s_mov_b32 s5, s6",
               "s_mov_b32 m0, s7", "s_nop 0", "buffer_load_dword v0, s[44:47], s50 offen lds")
    assert build.dma_sgpr_hazards(asm) == []


def test_scalar_writes_and_unrelated_vector_work_pass():
    asm = _asm("s_mov_b32 s44, s1", "v_add_u32_e32 v4, s9, v0", "s_mov_b32 m0, s2", "s_nop 0",
               "buffer_load_dwordx4 v4, s[44:47], 0 offen lds")
    assert build.dma_sgpr_hazards(asm) == []


def test_block_boundary_inside_the_window_is_a_hazard():
    asm = _asm(".LBB0_7:", "s_nop 0", "buffer_load_dwordx4 v0, s[44:47], 0 offen lds")
    assert len(build.dma_sgpr_hazards(asm)) == 1
    asm = _asm("s_cbranch_scc1 .LBB0_9", "s_nop 0", "buffer_load_dwordx4 v0, s[44:47], 0 offen lds")
    assert len(build.dma_sgpr_hazards(asm)) == 1


def test_ordinary_loads_are_not_checked():
    asm = _asm("v_readfirstlane_b32 s45, v3", "buffer_load_dwordx4 v[0:3], v1, s[44:47], 0 offen")
    assert build.dma_sgpr_hazards(asm) == []


def test_store_data_overwritten_right_after_a_wide_store():
    asm = _asm("buffer_store_dwordx4 v[46:49], v61, s[36:39], s12 offen", "v_mov_b32_e32 v47, v1")
    assert len(build.store_data_hazards(asm)) == 1
    asm = _asm("global_store_dwordx4 v[2:3], v[8:11], off", "s_nop 0", "v_add_f32_e32 v11, v1, v2")
    assert len(build.store_data_hazards(asm)) == 1


def test_store_data_hazard_cleared_by_wait_states_or_other_registers():
    asm = _asm("buffer_store_dwordx4 v[46:49], v61, s[36:39], s12 offen", "s_nop 1", "v_mov_b32_e32 v47, v1")
    assert build.store_data_hazards(asm) == []
    asm = _asm("buffer_store_dwordx4 v[46:49], v61, s[36:39], 0 offen", "v_mov_b32_e32 v50, v1",
               "v_mov_b32_e32 v51, v1", "v_mov_b32_e32 v46, v1")
    assert build.store_data_hazards(asm) == []
    # 64-bit stores are not affected
    asm = _asm("buffer_store_dwordx2 v[48:49], v63, s[36:39], 0 offen", "v_mov_b32_e32 v48, 0")
    assert build.store_data_hazards(asm) == []


def test_store_data_hazard_follows_branches():
    """The wait states after a wide store are counted along each path control can take: past an
    unconditional branch the text that follows is another block, and a conditional branch leads both
    to its target and to the next instruction."""
    store = "buffer_store_dwordx4 v[0:3], v9, s[0:3], 0 offen"
    # the next block in the text is not a successor; the target starts with two scalar instructions
    asm = _asm(store, "s_branch .LBB0_2", ".LBB0_1:", "v_mov_b32_e32 v1, 0", ".LBB0_2:", "s_mov_b32 s0, 0",
               "s_mov_b32 s1, 0", "v_mov_b32_e32 v1, 0")
    assert build.store_data_hazards(asm) == []
    # ... but a write right at the target is found
    asm = _asm(store, "s_branch .LBB0_2", ".LBB0_1:", "s_nop 7", ".LBB0_2:", "v_mov_b32_e32 v2, 0")
    assert len(build.store_data_hazards(asm)) == 1
    # a conditional branch: the target path and the fall-through path are both checked
    asm = _asm(store, "s_cbranch_scc1 .LBB0_2", "s_mov_b32 s0, 0", "s_mov_b32 s0, 0", ".LBB0_2:",
               "v_mov_b32_e32 v2, 0")
    assert len(build.store_data_hazards(asm)) == 1
    asm = _asm(store, "s_cbranch_scc1 .LBB0_2", "v_mov_b32_e32 v3, 0", "s_endpgm", ".LBB0_2:", "s_nop 3")
    assert len(build.store_data_hazards(asm)) == 1
