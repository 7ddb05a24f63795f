"""CPU check that the staircase inputs of tests/test_gpu_rescale.py drive the
MFMA kernel's lazy-rescale branches (tests/mla_cases.py:staircase_case).

The kernel raises a head's running maximum, and rescales its O accumulators,
only when a 32-position tile holds a score more than 8 base-2 units above it.
Walking the planned segments tile by tile over the same base-2 scores the
kernel forms, every wave must take that branch several times per plan, and
waves 0 and 1 (a PV pair: each applies the other's rescale to the O rows it
holds) must take it at different tiles, so both the own-head rescale and the
partner-head rescale (read from LDS) run with the other one idle.
"""

from __future__ import annotations

import numpy as np
import pytest

from mla_cases import lazy_rescale_tiles, scores_log2, segments, staircase_case, to_np

from latent_attn import build_rope_tables

S, B = 3000, 3


@pytest.mark.parametrize("chunk_rows", [1024, 320])
def test_staircase_triggers_rescales_in_every_wave(chunk_rows):
    kv, qa, qr = staircase_case(B, S, "bf16", 5, "cpu")
    cos, sin = build_rope_tables(S, 64)
    cos, sin = to_np(cos), to_np(sin)
    per_wave = np.zeros(4, int)
    own_only = partner_only = 0
    for b, lo, hi in segments([S] * B, chunk_rows, S):
        s = scores_log2(to_np(kv[b])[lo:hi], to_np(qa[b]), to_np(qr[b]), cos[lo:hi], sin[lo:hi])
        # the tile maxima of the staircase heads span more than one rescale step
        tmax = [s[:64, i:i + 32].max() for i in range(0, hi - lo, 32)]
        assert max(tmax) - min(tmax) > 10 or hi - lo <= 256
        r = lazy_rescale_tiles(s)
        waves = [set().union(*[set(r[h]) for h in range(32 * w, 32 * w + 32)]) for w in range(4)]
        per_wave += [len(x) for x in waves]
        own_only += len(waves[0] - waves[1])
        partner_only += len(waves[1] - waves[0])
    assert (per_wave >= 10).all(), per_wave
    assert own_only >= 5 and partner_only >= 5, (own_only, partner_only)


def test_no_rescale_with_gaussian_scores():
    """The contrast: N(0,1) caches and queries (the other GPU tests' inputs)
    never move the running maximum by more than 8 after the first tile."""
    from mla_cases import LOG2E

    rs = np.random.RandomState(0)
    kv = rs.standard_normal((2048, 576))
    qa = rs.standard_normal((128, 512)) / np.sqrt(512) * np.sqrt(128)  # q_nope . W_UK scale
    qr = rs.standard_normal((128, 64))
    cos, sin = build_rope_tables(2048, 64)
    s = scores_log2(kv, qa, qr, to_np(cos), to_np(sin))
    assert LOG2E > 1 and all(len(t) == 0 for t in lazy_rescale_tiles(s))


def _lazy_tile_decode(s, V, skip_rescale: bool, slack: float = 8.0):
    """numpy restatement of the kernel's lazily rescaled base-2 softmax over
    32-position tiles of one segment (s (H, n) base-2 scores, V (n, d)):
    O and l accumulate 2^(s - m) with m raised only when a tile beats it by
    more than `slack`, then O and l are multiplied by 2^(m_old - m_new)
    (or, with skip_rescale, left as they are: the mistake to detect)."""
    H, n = s.shape
    m = np.full(H, -np.inf)
    O = np.zeros((H, V.shape[1]))
    l = np.zeros(H)
    for t in range((n + 31) // 32):
        st = s[:, 32 * t:32 * t + 32]
        tmax = st.max(axis=1)
        need = tmax > m + slack
        if need.any():
            m_new = np.maximum(m, tmax)
            alpha = np.where(np.isinf(m), 0.0, np.exp2(m - m_new))
            if not skip_rescale:
                O *= alpha[:, None]
                l *= alpha
            m = m_new
        p = np.exp2(st - m[:, None])
        O += p @ V[32 * t:32 * t + 32]
        l += p.sum(axis=1)
    return O / l[:, None]


def test_staircase_detects_a_missing_rescale():
    """Planted on the CPU: the lazy tile softmax without its rescale step is
    far outside the bf16 tolerance on the staircase inputs, while the correct
    one matches the plain softmax, so the GPU tests' inputs can see that
    mistake."""
    kv, qa, qr = staircase_case(1, 1024, "bf16", 5, "cpu")
    cos, sin = build_rope_tables(1024, 64)
    kv = to_np(kv[0])
    s = scores_log2(kv, to_np(qa[0]), to_np(qr[0]), to_np(cos), to_np(sin))
    w = np.exp2(s - s.max(axis=1, keepdims=True))
    ref = (w @ kv[:, :512]) / w.sum(axis=1, keepdims=True)
    good = _lazy_tile_decode(s, kv[:, :512], skip_rescale=False)
    bad = _lazy_tile_decode(s, kv[:, :512], skip_rescale=True)
    err = lambda x: np.linalg.norm(x - ref) / np.linalg.norm(ref)
    assert err(good) < 1e-12
    assert err(bad) > 0.05
