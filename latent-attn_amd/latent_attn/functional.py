"""Stateless functional API for the MLA decode kernels.

Same entry points and argument order as the reference
(latent_attn/functional.py:24-116 in the reference repo): ``fused_mla``,
``naive_mla``, ``batched_fused_mla``; plus ``mla_decode`` (per-sequence and
ragged caches with query absorption, split-KV and the W_UV projection in one
call) and ``absorb_q``. All compute runs in the HIP library; nothing here
falls back to PyTorch math -- if the extension is missing, the call raises.
"""

from __future__ import annotations

from typing import TYPE_CHECKING, Optional

import torch

if TYPE_CHECKING:
    from latent_attn import MLAConfig


def _load_ext():
    try:
        from latent_attn import _C

        return _C
    except ImportError as e:  # reference functional.py:13-21
        raise ImportError(
            "latent_attn C extension not found. "
            "Run `python latent-attn_amd/build.py` from the repo root to build it."
        ) from e


def _cfg_args(cfg: "MLAConfig"):
    return (cfg.d_model, cfg.kv_lora_rank, cfg.qk_nope_head_dim, cfg.qk_rope_head_dim, cfg.num_heads, cfg.v_head_dim)


def fused_mla(
    kv_cache: torch.Tensor,
    q_absorbed: torch.Tensor,
    q_rope: torch.Tensor,
    W_UV: torch.Tensor,
    rope_cos: torch.Tensor,
    rope_sin: torch.Tensor,
    cfg: "MLAConfig",
) -> torch.Tensor:
    """Single-token fused absorbed MLA forward.

    Args:
        kv_cache:   (seq_len, kv_lora_rank + qk_rope_head_dim) fp16 / bf16 / fp32
        q_absorbed: (num_heads, kv_lora_rank) fp32
        q_rope:     (num_heads, qk_rope_head_dim) fp32, already rotated
        W_UV:       (num_heads * v_head_dim, kv_lora_rank) fp16 / bf16 / fp32
        rope_cos:   (seq_len, qk_rope_head_dim // 2) fp32
        rope_sin:   (seq_len, qk_rope_head_dim // 2) fp32
        cfg:        MLAConfig

    Returns:
        (num_heads, v_head_dim) fp32
    """
    _C = _load_ext()
    return _C.fused_mla_forward(kv_cache, q_absorbed, q_rope, W_UV, rope_cos, rope_sin, *_cfg_args(cfg))


def naive_mla(
    kv_cache: torch.Tensor,
    W_UK: torch.Tensor,
    W_UV: torch.Tensor,
    q_nope: torch.Tensor,
    q_rope: torch.Tensor,
    rope_cos: torch.Tensor,
    rope_sin: torch.Tensor,
    cfg: "MLAConfig",
) -> torch.Tensor:
    """Single-token MLA forward from the un-absorbed query (q_nope, W_UK).

    Returns the decompress-then-attend result (num_heads, v_head_dim) fp32. It
    is computed on the GPU by absorbing q_nope into the latent space and
    running the fused decode (the same function of the inputs).
    """
    _C = _load_ext()
    return _C.naive_mla_forward(kv_cache, W_UK, W_UV, q_nope, q_rope, rope_cos, rope_sin, *_cfg_args(cfg))


def batched_fused_mla(
    kv_cache: torch.Tensor,
    q_absorbed: torch.Tensor,
    q_rope: torch.Tensor,
    W_UV: torch.Tensor,
    rope_cos: torch.Tensor,
    rope_sin: torch.Tensor,
    cfg: "MLAConfig",
) -> torch.Tensor:
    """Batched fused absorbed MLA forward over multiple tokens sharing one KV cache.

    Args:
        kv_cache:   (seq_len, kv_lora_rank + qk_rope_head_dim)
        q_absorbed: (batch, num_heads, kv_lora_rank) fp32
        q_rope:     (batch, num_heads, qk_rope_head_dim) fp32
        W_UV:       (num_heads * v_head_dim, kv_lora_rank)
        rope_cos / rope_sin: (seq_len, qk_rope_head_dim // 2) fp32

    Returns:
        (batch, num_heads, v_head_dim) fp32
    """
    _C = _load_ext()
    return _C.batched_fused_mla_forward(kv_cache, q_absorbed, q_rope, W_UV, rope_cos, rope_sin, *_cfg_args(cfg))


def mla_decode(
    kv_cache: torch.Tensor,
    q_nope: torch.Tensor,
    q_rope: torch.Tensor,
    W_UK: torch.Tensor,
    W_UV: torch.Tensor,
    rope_cos: torch.Tensor,
    rope_sin: torch.Tensor,
    cfg: "MLAConfig",
    seq_offsets: Optional[torch.Tensor] = None,
    chunk_rows: int = 0,
    kernel_variant: int = 0,
) -> torch.Tensor:
    """One decode step for a batch of sequences, each with its own cache.

    Args:
        kv_cache:    (batch, seq_len, dc + dR) when ``seq_offsets`` is None, else
                     a packed (total_rows, dc + dR) cache
        q_nope:      (batch, num_heads, qk_nope_head_dim) fp32
        q_rope:      (batch, num_heads, qk_rope_head_dim) fp32, already rotated
        W_UK, W_UV:  (num_heads * {qk_nope,v}_head_dim, kv_lora_rank)
        rope_cos / rope_sin: (>= longest sequence, qk_rope_head_dim // 2) fp32,
                     indexed by the position inside each sequence
        seq_offsets: optional int32 (batch + 1,) device tensor; sequence b is
                     rows [seq_offsets[b], seq_offsets[b+1])
        chunk_rows, kernel_variant: tuning overrides (0 = automatic; variant
                     1 = VALU kernel, 2 = MFMA kernel)

    Returns:
        (batch, num_heads, v_head_dim) fp32
    """
    _C = _load_ext()
    return _C.mla_decode_forward(kv_cache, q_nope, q_rope, W_UK, W_UV, rope_cos, rope_sin, seq_offsets,
                                 *_cfg_args(cfg), chunk_rows, kernel_variant)


def absorb_q(q_nope: torch.Tensor, W_UK: torch.Tensor, cfg: "MLAConfig") -> torch.Tensor:
    """q_absorbed[..., h, c] = sum_i q_nope[..., h, i] * W_UK[h*dn + i, c] (fp32)."""
    _C = _load_ext()
    return _C.absorb_q_forward(q_nope, W_UK, *_cfg_args(cfg))
