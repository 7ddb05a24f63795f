"""Seeded input builders shared by the GPU parity tests, smoke() and bench.py's
checks. Inputs follow the BASELINE.json recipe: c_t, k_rope, q ~ N(0,1);
W_UK, W_UV ~ N(0, std 1/sqrt(d_c)); RoPE base 10000. Tensors are generated on
the CPU with torch's seeded generator (deterministic), stored in the cache
dtype, then moved to the device. ``to_np`` gives the exact float64 values the
oracle sees.
"""

from __future__ import annotations

import math

import numpy as np
import torch

from latent_attn import MLAConfig, build_rope_tables

TORCH_DTYPE = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}


def cfg_with_heads(num_heads: int) -> MLAConfig:
    c = MLAConfig.deepseek_v2()
    c.num_heads = num_heads
    return c


def to_np(t: torch.Tensor) -> np.ndarray:
    return t.detach().to("cpu", torch.float32).numpy().astype(np.float64)


def make_weights(cfg: MLAConfig, dtype: str, seed: int, device):
    g = torch.Generator().manual_seed(seed)
    std = 1.0 / math.sqrt(cfg.kv_lora_rank)
    W_UK = (torch.randn(cfg.num_heads * cfg.qk_nope_head_dim, cfg.kv_lora_rank, generator=g) * std)
    W_UV = (torch.randn(cfg.num_heads * cfg.v_head_dim, cfg.kv_lora_rank, generator=g) * std)
    dt = TORCH_DTYPE[dtype]
    return W_UK.to(dt).to(device), W_UV.to(dt).to(device)


def make_cache(rows_shape, cfg: MLAConfig, dtype: str, seed: int, device):
    g = torch.Generator().manual_seed(seed)
    row = cfg.kv_lora_rank + cfg.qk_rope_head_dim
    return torch.randn(*rows_shape, row, generator=g).to(TORCH_DTYPE[dtype]).to(device)


def make_queries(lead, cfg: MLAConfig, seed: int, device):
    g = torch.Generator().manual_seed(seed)
    q_nope = torch.randn(*lead, cfg.num_heads, cfg.qk_nope_head_dim, generator=g).to(device)
    q_rope = torch.randn(*lead, cfg.num_heads, cfg.qk_rope_head_dim, generator=g).to(device)
    return q_nope.contiguous(), q_rope.contiguous()


def rope(rows: int, cfg: MLAConfig, device):
    cos, sin = build_rope_tables(max(rows, 1), cfg.qk_rope_head_dim, device="cpu")
    return cos.to(device).contiguous(), sin.to(device).contiguous()


def ragged_lengths(batch: int, lo: int, hi: int, seed: int) -> list[int]:
    """Sequence lengths uniform in [lo, hi] (BASELINE config 4 uses
    RandomState(seed).randint(512, 32769, 64))."""
    return [int(x) for x in np.random.RandomState(seed).randint(lo, hi + 1, batch)]


# ---------------------------------------------------------------------------
# Inputs whose running score maximum climbs in steps (lazy-rescale coverage)
# ---------------------------------------------------------------------------
# The MFMA decode kernel keeps a running maximum m per head and raises it only
# when a 32-position tile holds a score above m + 8 (base-2 units); then the O
# accumulators of that head are multiplied by 2^(m_old - m_new), for the
# wave's own heads and, through LDS, for its PV partner's. With N(0,1) inputs
# the scores stay within a few units of the first tile's maximum and that
# branch never runs. Here two latent coordinates carry staircases: c_t[pos][0]
# = A * tier1(tile), c_t[pos][1] = A * tier2(tile), and the absorbed queries
# weight them per head group, so a head's score rises by a fixed number of
# base-2 units at every tier step:
#   heads   0- 31 (wave 0): 10.0 per tier1 step
#   heads  32- 63 (wave 1): 10.0 per tier2 step  (PV partner of wave 0,
#                           rising at other tiles)
#   heads  64- 95 (wave 2):  7.5 per tier1 step  (below the slack of 8: a
#                           rescale every second step; P up to 2^7.5)
#   heads  96-127 (wave 3):  5.0 per tier1 step + 15.0 per tier2 step
# tier1 = ((tile + shift) % 24) // 4 rises every 4 tiles and falls back to 0
# every 24, tier2 = ((tile + shift + 3) % 20) // 5 rises every 5 tiles; shift
# differs per sequence so chunk boundaries meet every phase. A = 96 makes
# every cache value an integer multiple of 96 below 2^11 (exact in bf16 and
# fp16) and 0.75 / 1.5 exact query weights, so the staircase part of each
# score is exact up to the kernel's 16-bit rounding of q * scale * log2(e).
STAIR_A = 96.0
LOG2E = 1.4426950408889634


def stair_tiers(S: int, shift: int):
    tile = (np.arange(S) // 32) + shift
    return (tile % 24) // 4, ((tile + 3) % 20) // 5


def staircase_case(B: int, S: int, dtype: str, seed: int, device):
    """(kv (B, S, 576) in dtype, q_abs (B, 128, 512) f32, q_rope (B, 128, 64)
    f32) on `device`; see the comment above."""
    g = torch.Generator().manual_seed(seed)
    kv = torch.randn(B, S, 576, generator=g)
    for b in range(B):
        t1, t2 = stair_tiers(S, 7 * b)
        kv[b, :, 0] = torch.from_numpy(STAIR_A * t1).float()
        kv[b, :, 1] = torch.from_numpy(STAIR_A * t2).float()
    q_abs = torch.randn(B, 128, 512, generator=g) * 0.2
    q_abs[:, :, 0:2] = 0.0
    q_abs[:, 0:32, 0] = 1.0
    q_abs[:, 32:64, 1] = 1.0
    q_abs[:, 64:96, 0] = 0.75
    q_abs[:, 96:128, 0] = 0.5
    q_abs[:, 96:128, 1] = 1.5
    q_rope = torch.randn(B, 128, 64, generator=g)
    return kv.to(TORCH_DTYPE[dtype]).to(device), q_abs.to(device), q_rope.to(device)


def scores_log2(kv: np.ndarray, q_abs: np.ndarray, q_rope: np.ndarray, cos: np.ndarray, sin: np.ndarray):
    """Base-2 scores (H, S) of one sequence, as the kernel forms them
    (scale * log2(e) * (q_abs . c_t + q_rope . RoPE(k_rope)))."""
    from oracle import mla_oracle as mo

    S = kv.shape[0]
    k_rot = mo.rope_rotate(kv[:, 512:], cos[:S], sin[:S])
    return (q_abs @ kv[:, :512].T + q_rope @ k_rot.T) * (LOG2E / math.sqrt(192.0))


def lazy_rescale_tiles(s: np.ndarray, slack: float = 8.0):
    """For base-2 scores s (H, n) of one segment walked in 32-position tiles
    from its first position: for each head, the tile indices at which a score
    exceeds the running maximum by more than `slack` after the first tile
    (where the kernel's ballot raises the maximum and rescales O)."""
    H, n = s.shape
    out = [[] for _ in range(H)]
    m = np.full(H, -np.inf)
    for t in range((n + 31) // 32):
        tmax = s[:, 32 * t:32 * t + 32].max(axis=1)
        if t == 0:
            m = tmax
            continue
        need = tmax > m + slack
        for h in np.nonzero(need)[0]:
            out[h].append(t)
        # every head of a wave with a triggering head takes max(m, tile max)
        for w in range(H // 32):
            if need[32 * w:32 * w + 32].any():
                m[32 * w:32 * w + 32] = np.maximum(m[32 * w:32 * w + 32], tmax[32 * w:32 * w + 32])
    return out


def segments(lens, chunk_rows: int, region: int):
    """(sequence, first position, last position + 1) of every segment of the
    split plan for sequences of lengths `lens` in regions of `region` rows
    cut into chunks of chunk_rows rows (the row space is the concatenation
    of the regions)."""
    segs = []
    for b, n in enumerate(lens):
        lo = b * region
        hi = lo + n
        r = lo
        while r < hi:
            e = min(hi, (r // chunk_rows + 1) * chunk_rows)
            segs.append((b, r - lo, e - lo))
            r = e
    return segs
