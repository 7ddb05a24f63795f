"""GPU run of a C++ caller of the drop-in headers (include/fused_mla.cuh,
fused_mla_batched.cuh, mla_config.cuh, included by the reference's own file names), checked against the float64 oracle.

tests/cpp/reference_caller.cpp is written the way the reference's C++ test
is (reference tests/test_correctness.cu): srand(42) uniform inputs of small
amplitude (cache 0.05, weights 0.02, queries 0.1; :15-23, :111-115), the
absorbed query built on the host (:29-46), a FusedMLAParams filled field by
field and launch_fused_mla (:182-199), over the reference's matrix of
DeepSeek-V2 at kv_len 512 / 2048 / 8192 and 16 and 64 heads at 512 / 2048
(:238-257); plus launch_batched_fused_mla over a shared cache with a caller
workspace, and LatentKVCache::append_host (reference src/mla_config.cuh
:57-72) whose rows must read back bit for bit and which must refuse a row past
max_seq_len with "KV cache full". The program is built by build()
(latent-attn_amd/build.py) and dumps every case's inputs and output; this
test replaces the reference's cosine > 0.998 gate (:212) with the oracle at
the fp16 tolerance (tests/conftest.py:assert_close): the naive
decompress-then-attend oracle from q_nope and W_UK (reference
tests/test_python.py:26-63) for kv_len <= 2048, the absorbed oracle from the
program's own q_absorbed at 8192.
"""

from __future__ import annotations

import os
import subprocess

import numpy as np
import pytest

from conftest import assert_close
from oracle import mla_oracle as mo

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
EXE = os.path.join(ROOT, "tests", "cpp", "reference_caller")
CASES = [("v2_512", 128, 512), ("v2_2048", 128, 2048), ("v2_8192", 128, 8192), ("h16_512", 16, 512),
         ("h16_2048", 16, 2048), ("h64_512", 64, 512), ("h64_2048", 64, 2048)]


@pytest.fixture(scope="module")
def dumped(tmp_path_factory, cuda):
    assert os.path.exists(EXE), "tests/cpp/reference_caller is not built: run __graft_entry__.build()"
    d = tmp_path_factory.mktemp("cpp_caller")
    print(f"[cpp caller] {EXE} {d}", flush=True)
    r = subprocess.run([EXE, str(d)], capture_output=True, text=True, timeout=300)
    print(r.stdout, r.stderr, flush=True)
    assert r.returncode == 0, r.stdout + r.stderr
    return d, r.stdout


def load(d, tag, name, dtype, shape):
    return np.fromfile(os.path.join(d, f"{tag}_{name}.bin"), dtype=dtype).reshape(shape).astype(np.float64)


@pytest.mark.parametrize("tag,nh,S", CASES)
def test_launch_fused_mla_from_cpp(dumped, tag, nh, S):
    d, _ = dumped
    cfg = mo.Dims(5120, 512, 128, 64, nh, 128)
    kv = load(d, tag, "kv", np.float16, (S, 576))
    W_UV = load(d, tag, "wuv", np.float16, (nh * 128, 512))
    qr = load(d, tag, "qr", np.float32, (nh, 64))
    cos = load(d, tag, "cos", np.float32, (S, 32))
    sin = load(d, tag, "sin", np.float32, (S, 32))
    out = load(d, tag, "out", np.float32, (nh, 128))
    if S <= 2048:
        W_UK = load(d, tag, "wuk", np.float16, (nh * 128, 512))
        qn = load(d, tag, "qn", np.float32, (nh, 128))
        ref = mo.naive_mla(kv, W_UK, W_UV, qn, qr, cos, sin, cfg)
    else:
        qa = load(d, tag, "qa", np.float32, (nh, 512))
        ref = mo.absorbed_mla(kv, qa, qr, W_UV, cos, sin, cfg)
    assert_close(out, ref, "f16", f"C++ launch_fused_mla {tag}")


def test_launch_batched_fused_mla_from_cpp(dumped):
    d, _ = dumped
    B, S = 4, 1024
    cfg = mo.Dims(5120, 512, 128, 64, 128, 128)
    ref = mo.batched_absorbed_mla(load(d, "batched", "kv", np.float16, (S, 576)),
                                  load(d, "batched", "qa", np.float32, (B, 128, 512)),
                                  load(d, "batched", "qr", np.float32, (B, 128, 64)),
                                  load(d, "batched", "wuv", np.float16, (128 * 128, 512)),
                                  load(d, "batched", "cos", np.float32, (S, 32)),
                                  load(d, "batched", "sin", np.float32, (S, 32)), cfg)
    assert_close(load(d, "batched", "out", np.float32, (B, 128, 128)), ref, "f16", "C++ launch_batched_fused_mla")


def test_latent_kv_cache_append_host(dumped):
    _, stdout = dumped
    assert "LatentKVCache append_host: ok" in stdout
