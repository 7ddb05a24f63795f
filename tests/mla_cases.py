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
