"""CPU check of the compiled attention kernels: no instruction touches a
register that an inline-asm LDS read (lgkmcnt) or vector-memory load
(vmcnt: the 36 query loads of the prologue, waited for by hand-counted
vmcnt values, and the paged cache's block-table entries) has not yet written
(see tests/lds_wait_check.py). Compiles latent-attn_amd/csrc/la_mfma.hip for
gfx950 to assembly with hipcc (about half a minute) and checks every
instantiation of decode_mfma_kernel. A compiler copy of such a register
before its wait once read a partner wave's rescale flag before it had landed;
a count that released a wait early would show up the same way, as a use of a
register whose load the in-order model has not retired. The kernels are
checked twice: by the linear walk and along their control-flow graph.
"""

from __future__ import annotations

import os
import shutil
import subprocess

import pytest

from lds_wait_check import kernels, kernels_with_labels, pending_uses, pending_uses_cfg

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"


@pytest.fixture(scope="module")
def decode_asm(tmp_path_factory):
    if not os.path.exists(HIPCC):
        pytest.skip("hipcc not available")
    out = tmp_path_factory.mktemp("asm") / "la_mfma.s"
    cmd = [HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang", "-target-feature", "-Xclang",
           "-packed-fp32-ops", "-I", os.path.join(ROOT, "include"), "-I", os.path.join(ROOT, "latent-attn_amd", "csrc"),
           "--cuda-device-only", "-S", os.path.join(ROOT, "latent-attn_amd", "csrc", "la_mfma.hip"), "-o", str(out)]
    subprocess.run(cmd, check=True, capture_output=True, timeout=600)
    return out.read_text()


@pytest.fixture(scope="module")
def decode_kernels(decode_asm):
    ks = kernels(decode_asm, "_ZN2la12_GLOBAL__N_118decode_mfma_kernel")
    assert len(ks) == 6, sorted(ks)  # {bf16, f16} x {contiguous, paged} and fp8 x {contiguous, paged}
    return ks


def test_checker_catches_an_early_copy():
    instrs = ["ds_read_b32 v0, v1", "v_mov_b32_e32 v2, v0", "s_waitcnt lgkmcnt(0)", "v_mov_b32_e32 v3, v0"]
    bad = pending_uses(instrs)
    assert [b[0] for b in bad] == [1]
    counted = ["ds_read_b128 v[0:3], v9", "ds_read_b128 v[4:7], v9", "s_waitcnt lgkmcnt(1)",
               "v_mov_b32_e32 v10, v0", "v_mov_b32_e32 v11, v4"]
    assert [b[0] for b in pending_uses(counted)] == [4]


def test_checker_models_vector_memory_loads():
    # a copy of a pending query-load register, before and after a counted wait
    loads = ["global_load_dwordx4 v[0:3], v[10:11], off", "global_load_dwordx4 v[4:7], v[10:11], off",
             "v_mov_b32_e32 v20, v1", "s_waitcnt vmcnt(1)", "v_mov_b32_e32 v21, v2", "v_mov_b32_e32 v22, v5"]
    assert [b[0] for b in pending_uses(loads, counters=("vm",))] == [2, 5]
    # HBM->LDS copies count without a destination: vmcnt(1) retires the load, not the copy
    mixed = ["global_load_dword v205, v[0:1], off", "global_load_lds_dwordx4 v[2:3], off",
             "s_waitcnt vmcnt(1)", "v_mov_b32_e32 v7, v205"]
    assert pending_uses(mixed, counters=("vm",)) == []
    # a 64-bit addend whose pending high half only feeds the dropped high half of the result
    dead = ["global_load_dword v205, v[0:1], off", "v_mad_u64_u32 v[192:193], vcc, v192, s96, v[204:205]",
            "v_mov_b32_e32 v193, 0"]
    assert pending_uses(dead, counters=("vm",)) == []
    used = dead[:2] + ["v_mov_b32_e32 v7, v193"]
    assert [b[0] for b in pending_uses(used, counters=("vm",))] == [1]


def test_no_register_touched_before_its_wait(decode_kernels):
    for name, instrs in decode_kernels.items():
        bad = pending_uses(instrs, counters=("lgkm", "vm"))
        assert not bad, f"{name}: " + "; ".join(f"#{n} {ins!r} before the wait of #{at} {rd!r}"
                                               for n, ins, at, rd in bad[:5])


def test_cfg_walk_matches_the_linear_walk_on_straight_code():
    for instrs, counters in ((["ds_read_b32 v0, v1", "v_mov_b32_e32 v2, v0", "s_waitcnt lgkmcnt(0)",
                               "v_mov_b32_e32 v3, v0"], ("lgkm",)),
                             (["global_load_dwordx4 v[0:3], v[10:11], off", "global_load_dwordx4 v[4:7], v[10:11], off",
                               "v_mov_b32_e32 v20, v1", "s_waitcnt vmcnt(1)", "v_mov_b32_e32 v21, v2",
                               "v_mov_b32_e32 v22, v5"], ("vm",))):
        assert [b[0] for b in pending_uses_cfg(instrs, counters=counters)] == \
            [b[0] for b in pending_uses(instrs, counters=counters)]


def test_cfg_walk_follows_branches():
    # an early copy in the arm that falls through is caught; the arm that
    # waits first is clean
    prog = ["ds_read_b32 v0, v1", "s_cbranch_scc1 .LA", "v_mov_b32_e32 v2, v0", "s_branch .LB", ".LA:",
            "s_waitcnt lgkmcnt(0)", "v_mov_b32_e32 v3, v0", ".LB:", "s_waitcnt lgkmcnt(0)", "s_endpgm"]
    assert [b[1] for b in pending_uses_cfg(prog)] == ["v_mov_b32_e32 v2, v0"]
    # an arm laid out after a path with a pending read, but not reached from
    # it, is not blamed for that read (the linear walk would)
    prog = ["s_cbranch_scc1 .LA", "ds_read_b32 v0, v1", "s_branch .LB", ".LA:", "v_mov_b32_e32 v0, 0", ".LB:",
            "s_waitcnt lgkmcnt(0)", "v_mov_b32_e32 v3, v0", "s_endpgm"]
    linear = [ln for ln in prog if not ln.endswith(":")]
    assert pending_uses(linear) and not pending_uses_cfg(prog)
    # a loop: the read of one trip is pending at the top of the next
    prog = [".LL:", "v_mov_b32_e32 v2, v0", "ds_read_b32 v0, v1", "s_cbranch_scc1 .LL", "s_waitcnt lgkmcnt(0)",
            "s_endpgm"]
    assert [b[1] for b in pending_uses_cfg(prog)] == ["v_mov_b32_e32 v2, v0"]


def test_cfg_walk_skips_only_the_no_lane_outcome_of_a_divergent_if():
    # a copy under a divergent if counts (some lane always takes it), so a
    # vmcnt that relies on it releases the older load on the path through it
    prog = ["global_load_dwordx4 v[0:3], v[10:11], off", "s_and_saveexec_b64 s[0:1], vcc", "s_cbranch_execz .LS",
            "global_load_lds_dwordx4 v4, s[2:3]", ".LS:", "s_or_b64 exec, exec, s[0:1]", "s_waitcnt vmcnt(1)",
            "v_mov_b32_e32 v20, v1", "s_endpgm"]
    assert pending_uses_cfg(prog, counters=("vm",)) == []
    # an exec branch that is not a divergent if's (a loop over lanes) keeps both edges
    prog = ["global_load_dwordx4 v[0:3], v[10:11], off", ".LW:", "s_xor_b64 exec, exec, s[0:1]",
            "s_cbranch_execz .LD", "global_load_lds_dwordx4 v4, s[2:3]", "s_branch .LW", ".LD:",
            "s_waitcnt vmcnt(1)", "v_mov_b32_e32 v20, v1", "s_endpgm"]
    assert [b[1] for b in pending_uses_cfg(prog, counters=("vm",))] == ["v_mov_b32_e32 v20, v1"]


def test_no_register_touched_before_its_wait_on_any_path(decode_asm):
    ks = kernels_with_labels(decode_asm, "_ZN2la12_GLOBAL__N_118decode_mfma_kernel")
    assert len(ks) == 6, sorted(ks)
    for name, lines in ks.items():
        bad = pending_uses_cfg(lines, counters=("lgkm", "vm"))
        assert not bad, f"{name}: " + "; ".join(f"#{n} {ins!r} before the wait of #{at} {rd!r}"
                                               for n, ins, at, rd in bad[:5])
