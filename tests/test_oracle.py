"""Pins for the CPU oracle (oracle/mla_oracle.py) -- CPU only.

The reference ships no golden vectors (its tests only compare implementations
by cosine similarity, reference tests/test_python.py:136-138). These tests pin
the oracle with closed forms, invariants, a library routine (torch's bf16
conversion) and an independent loop implementation, each chosen so that a
plausible mistake (wrong scale, interleaved instead of rotate-half RoPE, sign
of sin, transposed weights, missing normalisation) fails one of them. Some
tests also plant such a mistake in a copy of the oracle and check that the pin
catches it.
"""

from __future__ import annotations

import math

import numpy as np
import pytest

from oracle import mla_oracle as mo

SMALL = mo.Dims(d_model=64, kv_lora_rank=16, qk_nope_head_dim=8, qk_rope_head_dim=8, num_heads=3, v_head_dim=6)
CFG1 = mo.Dims(5120, 512, 128, 64, 16, 128)  # BASELINE config 1 (B=1, H=16, S=256)


def rand_case(cfg, S, seed=0, batch=None):
    return mo.make_inputs(cfg, S, seed=seed, cache_dtype="f32", batch=batch)


# ---------------------------------------------------------------------------
# number formats and RoPE
# ---------------------------------------------------------------------------

def test_bf16_round_matches_torch():
    import torch

    rs = np.random.RandomState(1)
    x = np.concatenate([
        rs.standard_normal(20000).astype(np.float32) * 10.0 ** rs.randint(-6, 6, 20000),
        np.array([1.0 + 2.0 ** -8, 1.0 + 3 * 2.0 ** -8, -1.0 - 2.0 ** -8, 0.0, -0.0, 65504.0], np.float32),
    ]).astype(np.float32)
    ours = mo.bf16_round(x)
    ref = torch.from_numpy(x).to(torch.bfloat16).to(torch.float32).numpy()
    assert np.array_equal(ours.view(np.uint32), ref.view(np.uint32))
    assert mo.bf16_round(np.float32([1.0 + 2.0 ** -8]))[0] == 1.0  # tie -> even
    assert mo.bf16_round(np.float32([1.0 + 3 * 2.0 ** -8]))[0] == np.float32(1.0 + 2.0 ** -6)


def test_rope_tables_closed_form():
    d_R = 64
    cos, sin = mo.build_rope_tables(4096, d_R)
    assert cos.shape == (4096, 32) and cos.dtype == np.float32
    p = np.arange(4096)[:, None].astype(np.float64)
    i = np.arange(32)[None, :].astype(np.float64)
    ang = p * 10000.0 ** (-2.0 * i / d_R)
    # float32 angle rounding bounds the error by ~p * 2^-23
    bound = p * 2.0 ** -22 + 2e-7
    assert (np.abs(cos - np.cos(ang)) <= bound).all()
    assert (np.abs(sin - np.sin(ang)) <= bound).all()
    assert cos[0].tolist() == [1.0] * 32 and sin[0].tolist() == [0.0] * 32  # RoPE at pos 0 is identity
    assert abs(cos[1, 1] - math.cos(10000.0 ** (-2.0 / 64))) < 1e-7  # frequency formula


def test_rope_rotation_closed_form():
    cos, sin = mo.build_rope_tables(16, 8)
    for pos in (0, 1, 5, 15):
        for i in range(4):
            e = np.zeros((1, 8))
            e[0, i] = 1.0
            r = mo.rope_rotate(e, cos[pos:pos + 1], sin[pos:pos + 1])[0]
            assert r[i] == pytest.approx(cos[pos, i]) and r[i + 4] == pytest.approx(sin[pos, i])
            e2 = np.zeros((1, 8))
            e2[0, i + 4] = 1.0
            r2 = mo.rope_rotate(e2, cos[pos:pos + 1], sin[pos:pos + 1])[0]
            assert r2[i] == pytest.approx(-sin[pos, i]) and r2[i + 4] == pytest.approx(cos[pos, i])
    k = np.random.RandomState(3).standard_normal((16, 8))
    r = mo.rope_rotate(k, cos.astype(np.float64), sin.astype(np.float64))
    assert np.allclose(np.linalg.norm(r, axis=1), np.linalg.norm(k, axis=1), rtol=1e-6)


# ---------------------------------------------------------------------------
# decode math
# ---------------------------------------------------------------------------

def _loop_naive(inp, cfg):
    """Independent decompress-then-attend with explicit loops (tiny shapes)."""
    kv, W_UK, W_UV = inp["kv_cache"].astype(float), inp["W_UK"].astype(float), inp["W_UV"].astype(float)
    qn, qr = inp["q_nope"].astype(float), inp["q_rope"].astype(float)
    cs, sn = inp["rope_cos"].astype(float), inp["rope_sin"].astype(float)
    S = kv.shape[0]
    dc, dR, nh, dn, dv = cfg.kv_lora_rank, cfg.qk_rope_head_dim, cfg.num_heads, cfg.qk_nope_head_dim, cfg.v_head_dim
    half = dR // 2
    out = np.zeros((nh, dv))
    for h in range(nh):
        scores = []
        for pos in range(S):
            s = 0.0
            for i in range(dn):
                k = sum(kv[pos, c] * W_UK[h * dn + i, c] for c in range(dc))
                s += qn[h, i] * k
            for i in range(half):
                k0, k1 = kv[pos, dc + i], kv[pos, dc + i + half]
                s += qr[h, i] * (k0 * cs[pos, i] - k1 * sn[pos, i])
                s += qr[h, i + half] * (k0 * sn[pos, i] + k1 * cs[pos, i])
            scores.append(s / math.sqrt(dn + dR))
        m = max(scores)
        w = [math.exp(x - m) for x in scores]
        z = sum(w)
        for j in range(dv):
            acc = 0.0
            for pos in range(S):
                v = sum(kv[pos, c] * W_UV[h * dv + j, c] for c in range(dc))
                acc += w[pos] / z * v
            out[h, j] = acc
    return out


def test_brute_force_loops_tiny():
    inp = rand_case(SMALL, 5, seed=7)
    ref = _loop_naive(inp, SMALL)
    out = mo.naive_mla(inp["kv_cache"], inp["W_UK"], inp["W_UV"], inp["q_nope"], inp["q_rope"], inp["rope_cos"],
                       inp["rope_sin"], SMALL)
    assert np.allclose(out, ref, rtol=1e-12, atol=1e-14)


@pytest.mark.parametrize("cfg,S", [(SMALL, 37), (CFG1, 256)])
def test_naive_equals_absorbed(cfg, S):
    """The absorption identity q_nope.(c W_UK^T) = (q_nope W_UK).c (README.md:25-35)."""
    inp = rand_case(cfg, S, seed=0)
    naive = mo.naive_mla(inp["kv_cache"], inp["W_UK"], inp["W_UV"], inp["q_nope"], inp["q_rope"], inp["rope_cos"],
                         inp["rope_sin"], cfg)
    qa = mo.absorb_q(inp["q_nope"], inp["W_UK"], cfg)
    fused = mo.absorbed_mla(inp["kv_cache"], qa, inp["q_rope"], inp["W_UV"], inp["rope_cos"], inp["rope_sin"], cfg)
    assert np.abs(naive - fused).max() <= 1e-12 * max(1.0, np.abs(naive).max())


def test_absorb_q_matches_reference_indexing():
    """Index order of reference tests/test_correctness.cu:29-46:
    q_abs[h,c] = sum_i q_nope[h*dn+i] * W_UK[h*dn*dc + i*dc + c]."""
    inp = rand_case(SMALL, 1, seed=2)
    cfg = SMALL
    qa = mo.absorb_q(inp["q_nope"], inp["W_UK"], cfg)
    W = inp["W_UK"].reshape(-1)
    qn = inp["q_nope"].reshape(-1)
    dn, dc = cfg.qk_nope_head_dim, cfg.kv_lora_rank
    for h in range(cfg.num_heads):
        for c in range(dc):
            ref = sum(float(qn[h * dn + i]) * float(W[h * dn * dc + i * dc + c]) for i in range(dn))
            assert qa[h, c] == pytest.approx(ref, rel=1e-12, abs=1e-12)


def test_single_position_is_projection():
    """S = 1: softmax weight 1, output = W_UV_h . c_0."""
    inp = rand_case(CFG1, 1, seed=4)
    qa = mo.absorb_q(inp["q_nope"], inp["W_UK"], CFG1)
    out = mo.absorbed_mla(inp["kv_cache"], qa, inp["q_rope"], inp["W_UV"], inp["rope_cos"], inp["rope_sin"], CFG1)
    c0 = inp["kv_cache"][0, :512].astype(float)
    W = inp["W_UV"].astype(float).reshape(16, 128, 512)
    assert np.allclose(out, W @ c0, rtol=1e-12, atol=1e-13)


def test_zero_query_is_uniform_mean():
    inp = rand_case(CFG1, 100, seed=5)
    zq = np.zeros((16, 512))
    zr = np.zeros((16, 64))
    out = mo.absorbed_mla(inp["kv_cache"], zq, zr, inp["W_UV"], inp["rope_cos"], inp["rope_sin"], CFG1)
    mean = inp["kv_cache"][:, :512].astype(float).mean(axis=0)
    W = inp["W_UV"].astype(float).reshape(16, 128, 512)
    assert np.allclose(out, W @ mean, rtol=1e-12, atol=1e-13)


def test_dominant_key():
    inp = rand_case(CFG1, 64, seed=6)
    j = 17
    cj = inp["kv_cache"][j, :512].astype(float)
    qa = np.tile(cj * 50.0, (16, 1))
    out = mo.absorbed_mla(inp["kv_cache"], qa, np.zeros((16, 64)), inp["W_UV"], inp["rope_cos"], inp["rope_sin"],
                          CFG1)
    W = inp["W_UV"].astype(float).reshape(16, 128, 512)
    assert np.allclose(out, W @ cj, rtol=1e-9, atol=1e-12)


def _rope_closed_form_case(cfg, p, qi):
    """Two keys at positions 0 and p. Latent part zero except an indicator
    coordinate, k_rope = e_0, q_rope = e_qi. Score(pos) = scale * (cos(pos)
    if qi == 0 else sin(pos)) with frequency 1 for pair index 0."""
    S = p + 1
    dc, dR = cfg.kv_lora_rank, cfg.qk_rope_head_dim
    kv = np.zeros((S, dc + dR), np.float32)
    kv[0, 0] = 1.0  # c_0 = e_0
    kv[p, 1] = 1.0  # c_p = e_1
    kv[:, dc] = 1.0  # k_rope = e_0 at every position
    keep = np.zeros(S, bool)
    keep[[0, p]] = True
    kv = kv[keep]
    cos, sin = mo.build_rope_tables(S, dR)
    cos, sin = cos[keep], sin[keep]
    qa = np.zeros((1, dc))
    qr = np.zeros((1, dR))
    qr[0, qi] = 1.0
    acc, _ = mo.absorbed_latent(kv, qa, qr, cos, sin, cfg)
    f = math.cos if qi == 0 else math.sin
    s0, sp = cfg.scale * f(0.0), cfg.scale * f(float(p))
    w0, wp = math.exp(s0), math.exp(sp)
    return acc[0], (w0 / (w0 + wp), wp / (w0 + wp))


@pytest.mark.parametrize("p,qi", [(3, 0), (3, 32), (50, 0), (50, 32), (1000, 32)])
def test_rope_score_closed_form(p, qi):
    cfg = mo.Dims(0, 512, 128, 64, 1, 128)
    acc, (a0, ap) = _rope_closed_form_case(cfg, p, qi)
    assert acc[0] == pytest.approx(a0, rel=1e-6) and acc[1] == pytest.approx(ap, rel=1e-6)
    assert abs(acc[2:]).max() == 0.0


def test_rope_pin_catches_interleaved_pairing(monkeypatch):
    """Plant interleaved (i, i+1) pairing in a copy of the oracle: the closed
    form must reject it."""
    def interleaved(k, cos, sin):
        k0, k1 = k[..., 0::2], k[..., 1::2]
        out = np.empty_like(k)
        out[..., 0::2] = k0 * cos - k1 * sin
        out[..., 1::2] = k0 * sin + k1 * cos
        return out

    monkeypatch.setattr(mo, "rope_rotate", interleaved)
    cfg = mo.Dims(0, 512, 128, 64, 1, 128)
    acc, (a0, ap) = _rope_closed_form_case(cfg, 50, 32)
    assert acc[0] != pytest.approx(a0, rel=1e-6)


def test_scale_pin_catches_wrong_scale(monkeypatch):
    """Plant scale 1/sqrt(dn) (forgetting d_R) -- the closed form rejects it."""
    cfg = mo.Dims(0, 512, 128, 64, 1, 128)
    bad = mo.Dims(0, 512, 128, 0, 1, 128)  # scale 1/sqrt(128)
    acc_good, (a0, ap) = _rope_closed_form_case(cfg, 50, 0)
    monkeypatch.setattr(mo.Dims, "scale", property(lambda self: 1.0 / math.sqrt(128)))
    acc_bad, _ = _rope_closed_form_case(cfg, 50, 0)
    assert acc_good[0] == pytest.approx(a0, rel=1e-6)
    assert acc_bad[0] != pytest.approx(a0, rel=1e-6)
    del bad


def test_common_latent_shift_adds_projection():
    """c_t -> c_t + t*u with q_abs . u = 0 leaves the weights unchanged, so the
    output moves by exactly t * W_UV u (pins sum of weights == 1)."""
    cfg = CFG1
    inp = rand_case(cfg, 80, seed=8)
    qa = mo.absorb_q(inp["q_nope"], inp["W_UK"], cfg)
    rs = np.random.RandomState(9)
    u = rs.standard_normal(512)
    # remove the component of u seen by any head's q_abs (project onto the
    # null space of the 16 query rows)
    Q, _ = np.linalg.qr(qa.T)
    u = u - Q @ (Q.T @ u)
    kv2 = inp["kv_cache"].astype(float).copy()
    kv2[:, :512] += 0.7 * u
    o1 = mo.absorbed_mla(inp["kv_cache"], qa, inp["q_rope"], inp["W_UV"], inp["rope_cos"], inp["rope_sin"], cfg)
    o2 = mo.absorbed_mla(kv2, qa, inp["q_rope"], inp["W_UV"], inp["rope_cos"], inp["rope_sin"], cfg)
    W = inp["W_UV"].astype(float).reshape(16, 128, 512)
    assert np.allclose(o2 - o1, 0.7 * (W @ u), rtol=1e-9, atol=1e-11)


def test_permutation_invariance():
    cfg = CFG1
    inp = rand_case(cfg, 90, seed=10)
    qa = mo.absorb_q(inp["q_nope"], inp["W_UK"], cfg)
    perm = np.random.RandomState(11).permutation(90)
    o1 = mo.absorbed_mla(inp["kv_cache"], qa, inp["q_rope"], inp["W_UV"], inp["rope_cos"], inp["rope_sin"], cfg)
    o2 = mo.absorbed_mla(inp["kv_cache"][perm], qa, inp["q_rope"], inp["W_UV"], inp["rope_cos"][perm],
                         inp["rope_sin"][perm], cfg)
    assert np.allclose(o1, o2, rtol=1e-12, atol=1e-14)


def test_split_lse_combine_invariance():
    cfg = CFG1
    inp = rand_case(cfg, 300, seed=12)
    qa = mo.absorb_q(inp["q_nope"], inp["W_UK"], cfg)
    acc, lse = mo.absorbed_latent(inp["kv_cache"], qa, inp["q_rope"], inp["rope_cos"], inp["rope_sin"], cfg)
    for bounds in ([(0, 300)], [(0, 1), (1, 300)], [(0, 100), (100, 164), (164, 300)]):
        parts = mo.split_lse_partials(inp["kv_cache"], qa, inp["q_rope"], inp["rope_cos"], inp["rope_sin"], cfg,
                                      bounds)
        acc2, lse2 = mo.lse_combine(parts)
        assert np.allclose(acc2, acc, rtol=1e-12, atol=1e-14)
        assert np.allclose(lse2, lse, rtol=1e-12)


def test_batched_shared_cache_equals_loop():
    """Reference invariant tests/test_batched.py:68-86: batched == loop of singles."""
    cfg = CFG1
    inp = rand_case(cfg, 50, seed=13, batch=3)
    qa = mo.absorb_q(inp["q_nope"], inp["W_UK"], cfg)
    b = mo.batched_absorbed_mla(inp["kv_cache"], qa, inp["q_rope"], inp["W_UV"], inp["rope_cos"], inp["rope_sin"],
                                cfg)
    for i in range(3):
        s = mo.absorbed_mla(inp["kv_cache"], qa[i], inp["q_rope"][i], inp["W_UV"], inp["rope_cos"],
                            inp["rope_sin"], cfg)
        assert np.allclose(b[i], s, rtol=1e-12, atol=1e-14)


def test_ragged_sequences_use_in_sequence_positions():
    cfg = CFG1
    lens = [5, 0, 40, 1]
    offs = np.concatenate([[0], np.cumsum(lens)])
    inp = rand_case(cfg, int(offs[-1]), seed=14, batch=len(lens))
    qa = mo.absorb_q(inp["q_nope"], inp["W_UK"], cfg)
    cos, sin = mo.build_rope_tables(64, 64)
    out = mo.decode_sequences(inp["kv_cache"], offs, qa, inp["q_rope"], inp["W_UV"], cos, sin, cfg)
    assert np.all(out[1] == 0.0)
    for b in (0, 2, 3):
        sl = inp["kv_cache"][offs[b]:offs[b + 1]]
        ref = mo.absorbed_mla(sl, qa[b], inp["q_rope"][b], inp["W_UV"], cos, sin, cfg)
        assert np.allclose(out[b], ref, rtol=1e-12, atol=1e-14)


# ---- cache append and query RoPE (device-side append_host) ----------------

def test_append_rows_places_rows_and_refuses_full():
    """Rows land at start + length (src/mla_config.cuh:57-72), lengths
    advance, other rows are untouched, a sequence without room is left as it
    was and reported; checked against hand-written expectations."""
    row = 576
    kv = np.full((12, row), -7.0, dtype=np.float32)
    starts, caps, lens = [0, 4, 8], [4, 4, 4], [1, 3, 0]
    c_t = np.arange(3 * 2 * 512, dtype=np.float32).reshape(3, 2, 512)
    k_rope = -np.arange(3 * 2 * 64, dtype=np.float32).reshape(3, 2, 64)
    out, new_lens, full = mo.append_rows(kv, starts, caps, lens, c_t, k_rope, "f32")
    assert full  # sequence 1 has 3 of 4 rows filled: no room for 2
    assert list(new_lens) == [3, 3, 2]
    for b, r in ((0, 1), (2, 8)):
        for t in range(2):
            assert np.array_equal(out[r + t, :512], c_t[b, t]) and np.array_equal(out[r + t, 512:], k_rope[b, t])
    untouched = [0, 3, 4, 5, 6, 7, 10, 11]
    assert np.all(out[untouched] == -7.0)


def test_append_rows_rounds_to_the_cache_dtype():
    kv = np.zeros((2, 576), dtype=np.float32)
    c_t = np.full((1, 1, 512), 1.0 + 2.0 ** -9, dtype=np.float32)  # halfway between two bf16 values
    k_rope = np.full((1, 1, 64), 3.0 + 2.0 ** -7, dtype=np.float32)
    out, _, _ = mo.append_rows(kv, [0], [2], [0], c_t, k_rope, "bf16")
    assert out[0, 0] == 1.0            # ties go to the even mantissa
    assert out[0, 512] == 3.0 + 2.0 ** -6 or out[0, 512] == 3.0
    assert np.array_equal(out[0, 512:], mo.bf16_round(k_rope[0, 0]))


def test_rotate_queries_closed_form():
    """A one-hot q_rope e_i at position p rotates to cos(p w_i) e_i +
    sin(p w_i) e_{i+32}, w_i = 10000^(-2i/64) (textbook 2-D rotation); query
    j of a sequence with old length L and T appended tokens sits at
    L + T - qps + j; position 0 is the identity; norms are preserved."""
    nh, dR, qps, T = 2, 64, 2, 3
    cos, sin = mo.build_rope_tables(64, dR)
    lens_old = [5, 0]
    q = np.zeros((2 * qps, nh, dR))
    for r in range(2 * qps):
        q[r, 0, r] = 1.0          # e_r in head 0
        q[r, 1, :] = np.linspace(-1, 1, dR) * (r + 1)
    got = mo.rotate_queries(q, lens_old, T, qps, cos, sin)
    for b in range(2):
        for j in range(qps):
            r = b * qps + j
            pos = lens_old[b] + T - qps + j
            w = 10000.0 ** (-2.0 * r / dR)
            expect = np.zeros(dR)
            expect[r], expect[r + 32] = math.cos(pos * w), math.sin(pos * w)
            assert np.allclose(got[r, 0], expect, atol=2e-6), (b, j)
            assert math.isclose(np.linalg.norm(got[r, 1]), np.linalg.norm(q[r, 1]), rel_tol=1e-6)
    # T == qps with an empty cache: the first query sits at position 0
    same = mo.rotate_queries(q[:1], [0], 1, 1, cos, sin)
    assert np.array_equal(same, q[:1])


# ---- LatentAttentionLayer.forward ---------------------------------------

def _layer_case(seed=3, d_model=96, nh=4, S=20):
    cfg = mo.Dims(d_model, 16, 8, 8, nh, 12)
    rs = np.random.RandomState(seed)
    p = dict(W_Q_absorbed=rs.standard_normal((nh * 16, d_model)) * 0.02,
             W_Q_rope=rs.standard_normal((nh * 8, d_model)) * 0.02,
             W_UV=rs.standard_normal((nh * 12, 16)) * 0.3,
             W_O=rs.standard_normal((d_model, nh * 12)) * 0.02)
    kv = rs.standard_normal((S, 24))
    cos, sin = mo.build_rope_tables(S, 8)
    return cfg, p, kv, cos, sin, rs


def test_layer_forward_zero_token_is_projected_mean():
    """x = 0 gives q = 0, uniform attention weights, so y = W_O . concat_h(
    W_UV_h . mean(c_t)) with W_UV rounded to fp16 (_w_uv_fp16,
    latent_attn/__init__.py:98-99): computed here from means and per-head
    products only."""
    cfg, p, kv, cos, sin, _ = _layer_case()
    y = mo.layer_forward(np.zeros(cfg.d_model), kv, p["W_Q_absorbed"], p["W_Q_rope"], p["W_UV"], p["W_O"], cos, sin,
                         cfg)
    mean_c = kv[:, :16].mean(axis=0)
    W_UV16 = mo.f16_round(p["W_UV"]).astype(np.float64)
    heads = np.concatenate([W_UV16[h * 12:(h + 1) * 12] @ mean_c for h in range(cfg.num_heads)])
    assert np.allclose(y, p["W_O"] @ heads, rtol=1e-12, atol=1e-14)
    # the fp16 rounding of W_UV is part of the path: unrounded weights differ
    assert not np.allclose(y, p["W_O"] @ np.concatenate(
        [p["W_UV"][h * 12:(h + 1) * 12] @ mean_c for h in range(cfg.num_heads)]), rtol=1e-9, atol=0)


def test_layer_forward_is_linear_in_w_o_and_uses_unrotated_queries():
    """y is linear in W_O; the query projections enter the attention as they
    are (the reference never rotates q): the result equals absorbed_mla on
    (W_Q_absorbed x, W_Q_rope x)."""
    cfg, p, kv, cos, sin, rs = _layer_case(seed=4)
    x = rs.standard_normal(cfg.d_model)
    y1 = mo.layer_forward(x, kv, p["W_Q_absorbed"], p["W_Q_rope"], p["W_UV"], p["W_O"], cos, sin, cfg)
    y2 = mo.layer_forward(x, kv, p["W_Q_absorbed"], p["W_Q_rope"], p["W_UV"], 2.5 * p["W_O"], cos, sin, cfg)
    assert np.allclose(y2, 2.5 * y1, rtol=1e-12, atol=1e-15)
    qa = (p["W_Q_absorbed"] @ x).reshape(4, 16)
    qr = (p["W_Q_rope"] @ x).reshape(4, 8)
    out = mo.absorbed_mla(kv, qa, qr, mo.f16_round(p["W_UV"]), cos, sin, cfg)
    assert np.allclose(y1, p["W_O"] @ out.reshape(-1), rtol=1e-12, atol=1e-15)


# ---- FP8 E4M3 cache format ----------------------------------------------

def test_fp8_decode_known_codes_and_torch():
    """Every one of the 256 codes decodes as torch's float8_e4m3fn does (a
    library routine); spot values from the format's definition."""
    import torch

    codes = np.arange(256, dtype=np.uint8)
    ours = mo.fp8_e4m3_decode(codes)
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    assert np.array_equal(np.isnan(ours), np.isnan(ref))
    ok = ~np.isnan(ref)
    assert np.array_equal(ours[ok], ref[ok])
    assert mo.fp8_e4m3_decode(np.array([0x38, 0x7E, 0x01, 0x08, 0xB8], np.uint8)).tolist() == \
        [1.0, 448.0, 2.0 ** -9, 2.0 ** -6, -1.0]


def test_fp8_encode_rounds_to_nearest_even_and_saturates():
    """In range the encoder equals torch's float8_e4m3fn conversion (round to
    nearest even) on a dense sweep including every midpoint between codes;
    beyond +-448 it saturates (torch gives NaN there); decode(encode(v)) == v
    for every finite code value."""
    import torch

    codes = np.arange(256, dtype=np.uint8)
    vals = mo.fp8_e4m3_decode(codes)
    fin = vals[np.isfinite(vals)]
    pos = np.unique(np.abs(fin))
    mids = (pos[:-1] + pos[1:]) / 2
    rs = np.random.RandomState(0)
    sweep = np.concatenate([fin, mids, -mids, rs.uniform(-448, 448, 4000), rs.standard_normal(4000) * 1e-3]).astype(np.float32)
    ours = mo.fp8_e4m3_encode(sweep)
    ref = torch.from_numpy(sweep).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(ours, ref)
    assert np.array_equal(mo.fp8_e4m3_encode(fin), codes[np.isfinite(vals)])
    big = np.array([448.0, 460.0, 464.0, 500.0, 1e30, -1e30], np.float32)
    assert mo.fp8_e4m3_encode(big).tolist() == [0x7E, 0x7E, 0x7E, 0x7E, 0x7E, 0xFE]
    assert mo.fp8_e4m3_encode(np.array([np.nan], np.float32))[0] & 0x7F == 0x7F
