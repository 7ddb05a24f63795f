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


# Achieved margins of every assert_close call in this session: (what, dtype,
# max abs, floored max rel, normwise, cosine). With LA_MARGINS_FILE set, the
# session writes them there as JSON lines.
MARGINS: list = []


def pytest_sessionfinish(session, exitstatus):
    path = os.environ.get("LA_MARGINS_FILE")
    if path and MARGINS:
        import json

        with open(path, "w") as f:
            for m in MARGINS:
                f.write(json.dumps(m) + "\n")


def assert_close(out, ref, dtype: str, what: str = ""):
    """Elementwise |d| <= atol + rtol*|ref| and normwise ||d|| / ||ref|| <=
    norm; also computes (and records in MARGINS) the floored max-rel
    |d| / max(|ref|, 1e-3 max|ref|) and the cosine, which are reported, not
    gated. Returns the margins as a dict."""
    from oracle.mla_oracle import max_rel_err, norm_rel_err

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
    den = np.linalg.norm(out) * np.linalg.norm(ref)
    m = {
        "what": what,
        "dtype": dtype,
        "max_abs": float(d.max()) if d.size else 0.0,
        "max_rel_floored": max_rel_err(out, ref),
        "norm_rel": ne,
        "cosine": float((out * ref).sum() / den) if den > 0 else 1.0,
        "max_abs_ref": float(np.abs(ref).max()) if ref.size else 0.0,
    }
    MARGINS.append(m)
    print(f"[margins] {what}: max_abs {m['max_abs']:.3e} max_rel(floored) {m['max_rel_floored']:.3e} "
          f"norm {ne:.3e} cos {m['cosine']:.7f} (max|ref| {m['max_abs_ref']:.3e})")
    assert not bad.any(), f"{what}: {bad.sum()} elements outside atol={atol} rtol={rtol}; max abs {d.max():.3e}"
    assert ne <= nrm, f"{what}: normwise relative error {ne:.3e} > {nrm}"
    return m
