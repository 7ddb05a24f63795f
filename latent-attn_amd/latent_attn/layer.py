"""``LatentAttentionLayer``: the reference's decode module
(latent_attn/__init__.py:40-145 in the reference repo) on this build's kernels.

Same parameters (names, shapes, fp32 storage, initialisation), the same RoPE
buffers and the same ``forward(x, kv_cache)`` contract:

    q_absorbed = x . W_Q_absorbed^T        (num_heads, kv_lora_rank)
    q_rope     = x . W_Q_rope^T            (num_heads, qk_rope_head_dim), NOT rotated
    out        = fused_mla(kv_cache, q_absorbed, q_rope, W_UV as fp16, cos, sin)
    y          = out.flatten() . W_O^T     (d_model,)

The two query projections and W_O are plain GEMV/GEMMs (torch, i.e. the
ROCm BLAS libraries); the attention, combine and W_UV projection run in the
HIP library. ``forward_batch`` is the batched form over per-sequence or ragged
caches (one decode token per sequence), which the reference does not have.
"""

from __future__ import annotations

import math
from typing import Optional

import torch
import torch.nn as nn

from . import MLAConfig, build_rope_tables
from . import functional as F


class LatentAttentionLayer(nn.Module):
    """Multi-head latent attention decode with the absorbed query projection
    W_Q_absorbed = W_Q . W_UK (reference latent_attn/__init__.py:40-46)."""

    def __init__(self, cfg: MLAConfig, max_seq_len: int = 8192) -> None:
        super().__init__()
        self.cfg = cfg
        self.max_seq_len = max_seq_len
        # shapes as in the reference constructor (latent_attn/__init__.py:48-73)
        self.W_Q_absorbed = nn.Parameter(torch.empty(cfg.num_heads * cfg.kv_lora_rank, cfg.d_model))
        self.W_Q_rope = nn.Parameter(torch.empty(cfg.num_heads * cfg.qk_rope_head_dim, cfg.d_model))
        self.W_UK = nn.Parameter(torch.empty(cfg.num_heads * cfg.qk_nope_head_dim, cfg.kv_lora_rank))
        self.W_UV = nn.Parameter(torch.empty(cfg.num_heads * cfg.v_head_dim, cfg.kv_lora_rank))
        self.W_O = nn.Parameter(torch.empty(cfg.d_model, cfg.num_heads * cfg.v_head_dim))
        self._init_weights()
        cos, sin = build_rope_tables(max_seq_len, cfg.qk_rope_head_dim, torch.device("cpu"))
        self.register_buffer("rope_cos", cos)  # (max_seq_len, d_R/2)
        self.register_buffer("rope_sin", sin)

    def _init_weights(self) -> None:
        # normal(0, 0.02), W_O with 0.02/sqrt(2) (reference latent_attn/__init__.py:83-90)
        std = 0.02
        nn.init.normal_(self.W_Q_absorbed, std=std)
        nn.init.normal_(self.W_Q_rope, std=std)
        nn.init.normal_(self.W_UK, std=std)
        nn.init.normal_(self.W_UV, std=std)
        nn.init.normal_(self.W_O, std=std / math.sqrt(2.0))

    @staticmethod
    def from_config(cfg: MLAConfig, max_seq_len: int = 8192) -> "LatentAttentionLayer":
        return LatentAttentionLayer(cfg, max_seq_len)

    def _w_uv_fp16(self) -> torch.Tensor:
        return self.W_UV.detach().to(torch.float16).contiguous()

    def _w_uk_fp16(self) -> torch.Tensor:
        return self.W_UK.detach().to(torch.float16).contiguous()

    def _queries(self, x: torch.Tensor):
        cfg = self.cfg
        lead = x.shape[:-1]
        q_abs = (x @ self.W_Q_absorbed.T).reshape(*lead, cfg.num_heads, cfg.kv_lora_rank)
        q_r = (x @ self.W_Q_rope.T).reshape(*lead, cfg.num_heads, cfg.qk_rope_head_dim)
        return q_abs.float().contiguous(), q_r.float().contiguous()

    @torch.no_grad()
    def forward(self, x: torch.Tensor, kv_cache: torch.Tensor) -> torch.Tensor:
        """One decode token over one cache (reference latent_attn/__init__.py:110-145).

        x: (d_model,) or (1, d_model); kv_cache: (seq_len, kv_lora_rank +
        qk_rope_head_dim), fp16 (reference contract), bf16 or fp32.
        Returns (d_model,) fp32.
        """
        if x.dim() == 2:
            x = x.squeeze(0)
        if x.dim() != 1 or x.size(0) != self.cfg.d_model:
            raise ValueError(f"x must be ({self.cfg.d_model},) or (1, {self.cfg.d_model})")
        seq_len = kv_cache.size(0)
        q_abs, q_r = self._queries(x)
        out = F.fused_mla(kv_cache=kv_cache, q_absorbed=q_abs, q_rope=q_r, W_UV=self._w_uv_fp16(),
                          rope_cos=self.rope_cos[:seq_len].contiguous(), rope_sin=self.rope_sin[:seq_len].contiguous(),
                          cfg=self.cfg)
        return out.reshape(-1) @ self.W_O.T

    @torch.no_grad()
    def forward_batch(self, x: torch.Tensor, kv_cache: torch.Tensor, seq_offsets: Optional[torch.Tensor] = None,
                      seq_lens: Optional[torch.Tensor] = None, block_table: Optional[torch.Tensor] = None,
                      block_size: int = 0) -> torch.Tensor:
        """One decode token per sequence of a batch: x (batch, d_model);
        kv_cache (batch, seq_len, dc + dR), or packed (rows, dc + dR) with
        int32 seq_offsets (batch + 1,), optionally with device seq_lens
        (capacity caches filled by ``functional.append_kv``), or a paged pool
        with block_table / block_size (see ``functional.mla_decode``). Row b
        of the result equals ``forward(x[b], cache of sequence b)``. Returns
        (batch, d_model) fp32."""
        if x.dim() != 2 or x.size(1) != self.cfg.d_model:
            raise ValueError(f"x must be (batch, {self.cfg.d_model})")
        q_abs, q_r = self._queries(x)
        out = F.mla_decode_absorbed(kv_cache, q_abs, q_r, self._w_uv_fp16(), self.rope_cos, self.rope_sin, self.cfg,
                                    seq_offsets=seq_offsets, seq_lens=seq_lens, block_table=block_table,
                                    block_size=block_size)
        return out.reshape(x.size(0), -1) @ self.W_O.T
