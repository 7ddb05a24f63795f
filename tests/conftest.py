"""Shared test setup: import paths, the `gpu` marker, seeded input builders."""

from __future__ import annotations

import math
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "latent-attn_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


def gpu_available() -> bool:
    import torch

    return torch.cuda.is_available()


@pytest.fixture(scope="session")
def cuda():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


# Tolerances from the north star: bf16/fp16 inputs with fp32 accumulation must
# match the float64 oracle within max-abs 2e-2 and max-rel 1e-2 (allclose form
# |d| <= atol + rtol*|ref|); fp32 mode within 1e-4. The normwise bound is an
# additional, stricter check that a near-zero output cannot pass vacuously.
BF16_ATOL, BF16_RTOL, BF16_NORM = 2e-2, 1e-2, 1e-2
FP32_ATOL, FP32_RTOL, FP32_NORM = 1e-4, 1e-4, 1e-5


def assert_close(out, ref, dtype: str, what: str = ""):
    from oracle.mla_oracle import norm_rel_err

    out = np.asarray(out, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert out.shape == ref.shape, (out.shape, ref.shape)
    assert np.isfinite(out).all(), f"{what}: non-finite output"
    if dtype == "f32":
        atol, rtol, nrm = FP32_ATOL, FP32_RTOL, FP32_NORM
    else:
        atol, rtol, nrm = BF16_ATOL, BF16_RTOL, BF16_NORM
    d = np.abs(out - ref)
    bad = d > atol + rtol * np.abs(ref)
    ne = norm_rel_err(out, ref)
    assert not bad.any(), f"{what}: {bad.sum()} elements outside atol={atol} rtol={rtol}; max abs {d.max():.3e}"
    assert ne <= nrm, f"{what}: normwise relative error {ne:.3e} > {nrm}"
    return ne
