"""CPU check of the compiled attention kernels: no instruction touches a
register that an inline-asm LDS read has not yet written (see
tests/lds_wait_check.py). Compiles latent-attn_amd/csrc/la_mfma.hip for
gfx950 to assembly with hipcc (about half a minute) and checks every
instantiation of decode_mfma_kernel. A compiler copy of such a register
before its wait once read a partner wave's rescale flag before it had landed.
"""

from __future__ import annotations

import os
import shutil
import subprocess

import pytest

from lds_wait_check import kernels, pending_uses

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"


@pytest.fixture(scope="module")
def decode_kernels(tmp_path_factory):
    if not os.path.exists(HIPCC):
        pytest.skip("hipcc not available")
    out = tmp_path_factory.mktemp("asm") / "la_mfma.s"
    cmd = [HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang", "-target-feature", "-Xclang",
           "-packed-fp32-ops", "-I", os.path.join(ROOT, "include"), "-I", os.path.join(ROOT, "latent-attn_amd", "csrc"),
           "--cuda-device-only", "-S", os.path.join(ROOT, "latent-attn_amd", "csrc", "la_mfma.hip"), "-o", str(out)]
    subprocess.run(cmd, check=True, capture_output=True, timeout=600)
    ks = kernels(out.read_text(), "_ZN2la12_GLOBAL__N_118decode_mfma_kernel")
    assert len(ks) == 6, sorted(ks)  # {bf16, f16} x {contiguous, paged} and fp8 x {contiguous, paged}
    return ks


def test_checker_catches_an_early_copy():
    instrs = ["ds_read_b32 v0, v1", "v_mov_b32_e32 v2, v0", "s_waitcnt lgkmcnt(0)", "v_mov_b32_e32 v3, v0"]
    bad = pending_uses(instrs)
    assert [b[0] for b in bad] == [1]
    counted = ["ds_read_b128 v[0:3], v9", "ds_read_b128 v[4:7], v9", "s_waitcnt lgkmcnt(1)",
               "v_mov_b32_e32 v10, v0", "v_mov_b32_e32 v11, v4"]
    assert [b[0] for b in pending_uses(counted)] == [4]


def test_no_register_touched_before_its_lds_wait(decode_kernels):
    for name, instrs in decode_kernels.items():
        bad = pending_uses(instrs)
        assert not bad, f"{name}: " + "; ".join(f"#{n} {ins!r} before the wait of #{at} {rd!r}"
                                               for n, ins, at, rd in bad[:5])
