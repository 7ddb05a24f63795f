"""CPU restatement of the reference's MLA decode math -- TEST INFRASTRUCTURE ONLY.

This module is the parity checker for the HIP path. Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it; the product path (``latent_attn`` and the C-ABI library) never does,
and fails loudly when its HIP library is missing.

Everything here is numpy, computed in float64 by default (``dtype`` switches the
arithmetic type for the CPU-baseline timing, which runs the same code in
float32). Each function cites the reference code it restates:

* ``build_rope_tables``  -- /root/reference/tests/test_python.py:17-23
  (also latent_attn/__init__.py:31-38): angles = pos * 10000^(-2i/d_R), fp32.
* ``naive_mla``          -- /root/reference/tests/test_python.py:26-63
  (``torch_mla_reference``): decompress K_nope = c_t W_UK^T, V = c_t W_UV^T,
  rotate-half RoPE on k_rope, scores scaled by 1/sqrt(dn+dR), softmax, P V.
* ``absorb_q``           -- /root/reference/tests/test_correctness.cu:29-46,
  tests/test_python.py:97-99: q_abs[h,c] = sum_i q_nope[h,i] W_UK[h*dn+i, c].
* ``absorbed_mla``       -- /root/reference/src/fused_mla.cu:218-267 with the
  helpers at :11-27 (latent dot) and :34-54 (RoPE score): two-pass softmax in
  latent space, normalise, then project with W_UV.
* ``batched_absorbed_mla`` -- /root/reference/src/fused_mla_batched.cu:62-106:
  B queries over ONE shared cache.
* ``decode_sequences``   -- the per-sequence / ragged decode that the north
  star adds (no reference counterpart): sequence b owns rows
  [offsets[b], offsets[b+1]) of a packed cache; RoPE position = index inside
  the sequence.
* ``split_lse_partials`` / ``lse_combine`` -- split-KV partials and their
  log-sum-exp merge (no reference counterpart; pinned by split invariance).
* ``append_rows``        -- /root/reference/src/mla_config.cuh:57-72
  (``LatentKVCache::append_host``: row current_len receives [c_t | k_rope],
  k_rope un-rotated; a full cache is refused), per sequence of a batch with
  capacity regions.
* ``layer_forward``      -- /root/reference/latent_attn/__init__.py:110-145
  (``LatentAttentionLayer.forward``): q_abs = W_Q_absorbed x, q_rope =
  W_Q_rope x (not rotated), the absorbed attention with W_UV rounded to fp16
  (``_w_uv_fp16``, :98-99), then W_O over the flattened heads.
* ``fp8_e4m3_encode`` / ``fp8_e4m3_decode`` -- the OCP FP8 E4M3 cache format
  of this build (no reference counterpart): round to nearest even, saturating
  at +-448.
* ``rotate_queries``     -- rotate-half RoPE of q_rope (the pairing of
  /root/reference/src/fused_mla.cu:43-51 and tests/test_python.py:50-54) at
  the position of the token each query belongs to; the reference itself never
  rotates the query, so this pins the build's own addition.

Packed cache row layout: [c_t (d_c) | k_rope (d_R)]
(/root/reference/src/mla_config.cuh:25-28,43-48).

Pinning (see tests/test_oracle.py): naive == absorbed (the absorption
identity), closed forms (S=1, q=0, one dominant key, one-hot RoPE angle),
shift and permutation invariance, split invariance, brute-force loops on tiny
shapes. The reference ships no golden vectors.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np


@dataclass(frozen=True)
class Dims:
    """MLA dimensions; same fields as the reference MLAConfig
    (/root/reference/src/mla_config.cuh:7-13)."""

    d_model: int
    kv_lora_rank: int
    qk_nope_head_dim: int
    qk_rope_head_dim: int
    num_heads: int
    v_head_dim: int

    @property
    def scale(self) -> float:
        # /root/reference/src/fused_mla.cu:284, tests/test_python.py:53
        return 1.0 / math.sqrt(self.qk_nope_head_dim + self.qk_rope_head_dim)


DEEPSEEK_V2 = Dims(5120, 512, 128, 64, 128, 128)


# ----------------------------------------------------------------------------
# number formats
# ----------------------------------------------------------------------------

def bf16_round(x: np.ndarray) -> np.ndarray:
    """Round float32 values to the nearest bfloat16 (ties to even), returned as
    float32. NaN/Inf are not expected in test inputs."""
    a = np.ascontiguousarray(x, dtype=np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    lsb = (u >> 16) & 1
    u = (u + 0x7FFF + lsb) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32).reshape(a.shape)


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """uint16 bit patterns of bf16_round(x)."""
    return (bf16_round(x).view(np.uint32) >> 16).astype(np.uint16)


def f16_round(x: np.ndarray) -> np.ndarray:
    return np.asarray(x, dtype=np.float32).astype(np.float16).astype(np.float32)


def fp8_e4m3_encode(x: np.ndarray) -> np.ndarray:
    """float -> OCP FP8 E4M3 (e4m3fn) codes (uint8): round to nearest even,
    saturate at +-448, NaN -> 0x7F | sign. The cache-write rule of this build
    (la_append_kv); the reference has no fp8 cache. In range it equals
    torch's float8_e4m3fn conversion (pinned in tests/test_oracle.py)."""
    x = np.asarray(x, dtype=np.float32)
    sign = (np.signbit(x)).astype(np.uint8) << 7
    a = np.abs(x).astype(np.float64)
    code = np.zeros(x.shape, dtype=np.int64)
    nan = np.isnan(a)
    sat = a >= 448.0
    sub = a < 2.0 ** -6
    code = np.where(sub, np.rint(a * 512.0), code)          # 0..8 (8 is 2^-6, the first normal)
    norm = ~(nan | sat | sub)
    with np.errstate(divide="ignore", invalid="ignore"):
        e = np.floor(np.log2(np.where(norm, a, 1.0)))
        m = np.rint((np.where(norm, a, 1.0) / 2.0 ** e - 1.0) * 8.0)   # np.rint: half to even
    e = np.where(m == 8, e + 1, e)
    m = np.where(m == 8, 0, m)
    code = np.where(norm, np.minimum(((e + 7) * 8 + m), 0x7E), code)
    code = np.where(sat, 0x7E, code)
    code = np.where(nan, 0x7F, code)
    return (code.astype(np.uint8) | sign).astype(np.uint8)


def fp8_e4m3_decode(c: np.ndarray) -> np.ndarray:
    """OCP FP8 E4M3 codes -> float32 values."""
    c = np.asarray(c, dtype=np.uint8).astype(np.int64)
    e, m = (c >> 3) & 15, c & 7
    v = np.where(e == 0, m * 2.0 ** -9, (1.0 + m / 8.0) * 2.0 ** (e - 7))
    v = np.where((e == 15) & (m == 7), np.nan, v)
    return np.where(c & 0x80, -v, v).astype(np.float32)


def round_to(x: np.ndarray, dtype: str) -> np.ndarray:
    if dtype == "bf16":
        return bf16_round(x)
    if dtype == "f16":
        return f16_round(x)
    if dtype == "fp8":
        return fp8_e4m3_decode(fp8_e4m3_encode(x))
    return np.asarray(x, dtype=np.float32)


# ----------------------------------------------------------------------------
# RoPE
# ----------------------------------------------------------------------------

def build_rope_tables(seq_len: int, d_R: int, base: float = 10000.0):
    """(cos, sin), each (seq_len, d_R//2) float32.

    Restates /root/reference/tests/test_python.py:17-23: float32 positions
    times float32 inverse frequencies 1/base^(2i/d_R), then cos/sin.
    """
    half = d_R // 2
    pos = np.arange(seq_len, dtype=np.float32)
    dims = np.arange(half, dtype=np.float32)
    freqs = (np.float32(1.0) / (np.float32(base) ** (np.float32(2.0) * dims / np.float32(d_R)))).astype(np.float32)
    ang = (pos[:, None] * freqs[None, :]).astype(np.float32)
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


def rope_rotate(k: np.ndarray, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    """Rotate-half RoPE of k (S, d_R): pairs (i, i + d_R/2).

    /root/reference/tests/test_python.py:50-54, src/fused_mla.cu:43-51.
    """
    half = k.shape[-1] // 2
    k0, k1 = k[..., :half], k[..., half:]
    return np.concatenate([k0 * cos - k1 * sin, k0 * sin + k1 * cos], axis=-1)


# ----------------------------------------------------------------------------
# reference math
# ----------------------------------------------------------------------------

def _softmax_rows(s: np.ndarray) -> np.ndarray:
    m = s.max(axis=-1, keepdims=True)
    w = np.exp(s - m)
    return w / w.sum(axis=-1, keepdims=True)


def naive_mla(kv_cache, W_UK, W_UV, q_nope, q_rope, rope_cos, rope_sin, cfg: Dims, dtype=np.float64):
    """Decompress-then-attend. /root/reference/tests/test_python.py:26-63.

    kv_cache (S, dc+dR); W_UK (nh*dn, dc); W_UV (nh*dv, dc); q_nope (nh, dn);
    q_rope (nh, dR); rope tables (S, dR/2). Returns (nh, dv).
    """
    f = lambda a: np.asarray(a, dtype=dtype)
    S = kv_cache.shape[0]
    dc, dR, nh, dn, dv = cfg.kv_lora_rank, cfg.qk_rope_head_dim, cfg.num_heads, cfg.qk_nope_head_dim, cfg.v_head_dim
    if S == 0:
        return np.zeros((nh, dv), dtype=dtype)
    c_t = f(kv_cache)[:, :dc]
    k_r = f(kv_cache)[:, dc:dc + dR]
    K_nope = (c_t @ f(W_UK).T).reshape(S, nh, dn)
    V = (c_t @ f(W_UV).T).reshape(S, nh, dv)
    K_rope = rope_rotate(k_r, f(rope_cos)[:S], f(rope_sin)[:S])
    sc = dtype(cfg.scale) if dtype is not np.float64 else cfg.scale
    scores = np.einsum("hd,shd->hs", f(q_nope), K_nope) * sc + np.einsum("hd,sd->hs", f(q_rope), K_rope) * sc
    attn = _softmax_rows(scores)
    return np.einsum("hs,shv->hv", attn, V)


def absorb_q(q_nope, W_UK, cfg: Dims, dtype=np.float64):
    """q_abs[..., h, c] = sum_i q_nope[..., h, i] * W_UK[h*dn + i, c].

    /root/reference/tests/test_correctness.cu:29-46 (host loop),
    tests/test_python.py:97-99 (einsum "hd,hdc->hc").
    """
    nh, dn, dc = cfg.num_heads, cfg.qk_nope_head_dim, cfg.kv_lora_rank
    W = np.asarray(W_UK, dtype=dtype).reshape(nh, dn, dc)
    return np.einsum("...hd,hdc->...hc", np.asarray(q_nope, dtype=dtype), W)


def absorbed_latent(kv_cache, q_absorbed, q_rope, rope_cos, rope_sin, cfg: Dims, dtype=np.float64):
    """Normalised latent accumulator acc[h, :] = sum_pos softmax_pos * c_t[pos]
    and the log-sum-exp of the scaled scores, per head.

    Scores follow /root/reference/src/fused_mla.cu:234-235 (latent dot and RoPE
    term each multiplied by scale), softmax with the max subtracted (:236-249),
    normalisation (:255-256). Returns (acc (nh, dc), lse (nh,)) with lse in
    natural-log units; an empty cache returns zeros and lse = -inf.
    """
    f = lambda a: np.asarray(a, dtype=dtype)
    dc, dR = cfg.kv_lora_rank, cfg.qk_rope_head_dim
    S = kv_cache.shape[0]
    nh = np.asarray(q_absorbed).shape[0]
    if S == 0:
        return np.zeros((nh, dc), dtype=dtype), np.full((nh,), -np.inf, dtype=dtype)
    c_t = f(kv_cache)[:, :dc]
    k_rot = rope_rotate(f(kv_cache)[:, dc:dc + dR], f(rope_cos)[:S], f(rope_sin)[:S])
    sc = dtype(cfg.scale) if dtype is not np.float64 else cfg.scale
    s = (f(q_absorbed) @ c_t.T) * sc + (f(q_rope) @ k_rot.T) * sc  # (nh, S)
    m = s.max(axis=1, keepdims=True)
    w = np.exp(s - m)
    l = w.sum(axis=1, keepdims=True)
    acc = (w @ c_t) / l
    return acc, (m + np.log(l))[:, 0]


def project_wuv(acc, W_UV, cfg: Dims, dtype=np.float64):
    """out[..., h, j] = sum_i acc[..., h, i] * W_UV[h*dv + j, i].

    /root/reference/src/fused_mla.cu:258-267. ``acc`` may carry leading batch
    axes and a head axis that is a multiple of num_heads (the shared-cache
    batched form uses head index b*nh + h with weight block h).
    """
    nh, dv, dc = cfg.num_heads, cfg.v_head_dim, cfg.kv_lora_rank
    W = np.asarray(W_UV, dtype=dtype).reshape(nh, dv, dc)
    a = np.asarray(acc, dtype=dtype)
    H = a.shape[-2]
    rep = H // nh
    a4 = a.reshape(a.shape[:-2] + (rep, nh, dc))
    out = np.einsum("...rhc,hjc->...rhj", a4, W)
    return out.reshape(a.shape[:-2] + (H, dv))


def absorbed_mla(kv_cache, q_absorbed, q_rope, W_UV, rope_cos, rope_sin, cfg: Dims, dtype=np.float64):
    """Single-token absorbed decode, /root/reference/src/fused_mla.cu:218-267.
    Returns (nh, dv)."""
    acc, _ = absorbed_latent(kv_cache, q_absorbed, q_rope, rope_cos, rope_sin, cfg, dtype)
    return project_wuv(acc, W_UV, cfg, dtype)


def batched_absorbed_mla(kv_cache, q_absorbed, q_rope, W_UV, rope_cos, rope_sin, cfg: Dims, dtype=np.float64):
    """B tokens over one shared cache, /root/reference/src/fused_mla_batched.cu:62-106.
    q_absorbed (B, nh, dc), q_rope (B, nh, dR). Returns (B, nh, dv)."""
    B, nh = q_absorbed.shape[0], q_absorbed.shape[1]
    acc, _ = absorbed_latent(kv_cache, np.asarray(q_absorbed).reshape(B * nh, -1),
                             np.asarray(q_rope).reshape(B * nh, -1), rope_cos, rope_sin, cfg, dtype)
    return project_wuv(acc.reshape(B, nh, -1), W_UV, cfg, dtype)


def decode_sequences(kv_packed, offsets, q_absorbed, q_rope, W_UV, rope_cos, rope_sin, cfg: Dims,
                     dtype=np.float64):
    """Per-sequence decode over a packed cache (north-star addition).

    kv_packed (T, dc+dR); offsets (B+1,) int; sequence b uses rows
    [offsets[b], offsets[b+1]) with RoPE positions 0..len-1.
    q_absorbed (B, nh, dc); q_rope (B, nh, dR). Returns (B, nh, dv);
    an empty sequence yields zeros.
    """
    B = len(offsets) - 1
    nh, dv = q_absorbed.shape[1], cfg.v_head_dim
    out = np.zeros((B, nh, dv), dtype=dtype)
    for b in range(B):
        lo, hi = int(offsets[b]), int(offsets[b + 1])
        if hi == lo:
            continue
        acc, _ = absorbed_latent(kv_packed[lo:hi], q_absorbed[b], q_rope[b], rope_cos, rope_sin, cfg, dtype)
        out[b] = project_wuv(acc, W_UV, cfg, dtype)
    return out


def split_lse_partials(kv_cache, q_absorbed, q_rope, rope_cos, rope_sin, cfg: Dims, bounds, dtype=np.float64):
    """Split-KV partials: for each [lo, hi) in ``bounds`` the normalised latent
    accumulator and lse over those positions only (RoPE positions stay
    absolute)."""
    parts = []
    for lo, hi in bounds:
        acc, lse = absorbed_latent(kv_cache[lo:hi], q_absorbed, q_rope, rope_cos[lo:hi], rope_sin[lo:hi], cfg, dtype)
        parts.append((acc, lse))
    return parts


def lse_combine(parts):
    """Merge split partials: o = sum_s e^{lse_s - L} o_s, L = log sum_s e^{lse_s}."""
    lses = np.stack([p[1] for p in parts])  # (nsplit, nh)
    accs = np.stack([p[0] for p in parts])  # (nsplit, nh, dc)
    L = np.logaddexp.reduce(lses, axis=0)
    w = np.exp(lses - L[None, :])
    return np.einsum("sh,shc->hc", w, accs), L


def layer_forward(x, kv_cache, W_Q_absorbed, W_Q_rope, W_UV, W_O, rope_cos, rope_sin, cfg: Dims,
                  dtype=np.float64):
    """LatentAttentionLayer.forward (latent_attn/__init__.py:110-145) for one
    token x (d_model,) over kv_cache (S, dc+dR): returns (d_model,)."""
    nh, dc, dR = cfg.num_heads, cfg.kv_lora_rank, cfg.qk_rope_head_dim
    x = np.asarray(x, dtype=dtype)
    q_abs = (np.asarray(W_Q_absorbed, dtype=dtype) @ x).reshape(nh, dc)
    q_r = (np.asarray(W_Q_rope, dtype=dtype) @ x).reshape(nh, dR)
    S = kv_cache.shape[0]
    out = absorbed_mla(kv_cache, q_abs, q_r, f16_round(np.asarray(W_UV, dtype=np.float32)), rope_cos[:S],
                       rope_sin[:S], cfg, dtype)
    return np.asarray(W_O, dtype=dtype) @ out.reshape(-1)


# ----------------------------------------------------------------------------
# cache append and query RoPE
# ----------------------------------------------------------------------------

def append_rows(kv, starts, caps, lens, c_t, k_rope, cache_dtype: str):
    """Append tokens to every sequence of a capacity cache.

    kv (rows, dc+dR) float; sequence b owns rows [starts[b], starts[b] +
    caps[b]) with its first lens[b] filled; c_t (B, T, dc), k_rope (B, T, dR).
    Following LatentKVCache::append_host (src/mla_config.cuh:57-72), token t
    lands in row starts[b] + lens[b] + t as [c_t | k_rope] (rounded to the
    cache dtype, k_rope not rotated) and the length advances; a sequence
    without room for all T tokens is left unchanged and reported.
    Returns (kv', lens', full) with full True when any sequence had no room.
    """
    kv = np.array(kv, copy=True)
    lens = np.array(lens, dtype=np.int64, copy=True)
    T = c_t.shape[1]
    full = False
    for b in range(len(lens)):
        if lens[b] < 0 or lens[b] + T > caps[b]:
            full = True
            continue
        r0 = int(starts[b] + lens[b])
        kv[r0:r0 + T] = round_to(np.concatenate([c_t[b], k_rope[b]], axis=-1).astype(np.float32), cache_dtype)
        lens[b] += T
    return kv, lens, full


def rotate_queries(q_rope, lens_old, tokens: int, qps: int, cos, sin):
    """q_rope (B*qps, nh, dR) rotated for its token's position: query j of
    sequence b belongs to the token at lens_old[b] + tokens - qps + j
    (positions past the table use its last row). Rotate-half pairing of
    src/fused_mla.cu:43-51."""
    q = np.array(q_rope, dtype=np.float64, copy=True)
    B = len(lens_old)
    for b in range(B):
        for j in range(qps):
            pos = min(int(lens_old[b]) + tokens - qps + j, cos.shape[0] - 1)
            q[b * qps + j] = rope_rotate(q[b * qps + j], cos[pos].astype(np.float64), sin[pos].astype(np.float64))
    return q


# ----------------------------------------------------------------------------
# deterministic synthetic inputs (numpy RandomState: stable stream)
# ----------------------------------------------------------------------------

def make_inputs(cfg: Dims, seq_len: int, seed: int = 0, cache_dtype: str = "f32", batch: int | None = None,
                w_std: float | None = None):
    """Inputs in the BASELINE.json recipe: c_t, k_rope, q ~ N(0,1);
    W_UK, W_UV ~ N(0, std = 1/sqrt(d_c)); RoPE base 10000; seed ``seed``.

    Cache and weights are rounded to ``cache_dtype`` (values stay float32);
    queries stay float32. ``batch`` None gives single-token shapes.
    """
    rs = np.random.RandomState(seed)
    dc, dR, nh, dn, dv = cfg.kv_lora_rank, cfg.qk_rope_head_dim, cfg.num_heads, cfg.qk_nope_head_dim, cfg.v_head_dim
    std = (1.0 / math.sqrt(dc)) if w_std is None else w_std
    kv = round_to(rs.standard_normal((seq_len, dc + dR)).astype(np.float32), cache_dtype)
    W_UK = round_to((rs.standard_normal((nh * dn, dc)) * std).astype(np.float32), cache_dtype)
    W_UV = round_to((rs.standard_normal((nh * dv, dc)) * std).astype(np.float32), cache_dtype)
    lead = () if batch is None else (batch,)
    q_nope = rs.standard_normal(lead + (nh, dn)).astype(np.float32)
    q_rope = rs.standard_normal(lead + (nh, dR)).astype(np.float32)
    cos, sin = build_rope_tables(max(seq_len, 1), dR)
    return dict(kv_cache=kv, W_UK=W_UK, W_UV=W_UV, q_nope=q_nope, q_rope=q_rope, rope_cos=cos, rope_sin=sin)


def max_rel_err(out: np.ndarray, ref: np.ndarray) -> float:
    """max |out-ref| / max(|ref|, 1e-3 * max|ref|)."""
    ref = np.asarray(ref, dtype=np.float64)
    d = np.abs(np.asarray(out, dtype=np.float64) - ref)
    den = np.maximum(np.abs(ref), 1e-3 * max(np.abs(ref).max(), 1e-30))
    return float((d / den).max()) if d.size else 0.0


def norm_rel_err(out: np.ndarray, ref: np.ndarray) -> float:
    ref = np.asarray(ref, dtype=np.float64)
    n = np.linalg.norm(ref)
    return float(np.linalg.norm(np.asarray(out, dtype=np.float64) - ref) / (n if n > 0 else 1.0))
