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

    Returns the decompress-then-attend result (num_heads, v_head_dim) fp32,
    computed on the GPU by la_naive_mla: K_nope = c_t W_UK^T and V = c_t
    W_UV^T materialised in fp32, RoPE on k_rope, softmax, P V -- independent
    of the absorbed kernels (reference tests/test_python.py:26-63).
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
    seq_lens: Optional[torch.Tensor] = None,
    block_table: Optional[torch.Tensor] = None,
    block_size: int = 0,
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
        seq_lens:    optional int32 (batch,) device tensor; sequence b is the
                     first seq_lens[b] rows of its region (a capacity cache
                     filled by ``append_kv``)
        block_table, block_size: optional paged cache: kv_cache is a pool of
                     (num_blocks * block_size, dc + dR) rows and position p of
                     sequence b lives in row block_table[b, p // block_size] *
                     block_size + p % block_size (int32 (batch, blocks_per_seq)
                     device tensor; needs seq_lens)

    Returns:
        (batch, num_heads, v_head_dim) fp32
    """
    _C = _load_ext()
    return _C.mla_decode_forward(kv_cache, q_nope, q_rope, W_UK, W_UV, rope_cos, rope_sin, seq_offsets,
                                 *_cfg_args(cfg), chunk_rows, kernel_variant, seq_lens, block_table, block_size)


def mla_decode_absorbed(
    kv_cache: torch.Tensor,
    q_absorbed: torch.Tensor,
    q_rope: torch.Tensor,
    W_UV: torch.Tensor,
    rope_cos: torch.Tensor,
    rope_sin: torch.Tensor,
    cfg: "MLAConfig",
    seq_offsets: Optional[torch.Tensor] = None,
    seq_lens: Optional[torch.Tensor] = None,
    chunk_rows: int = 0,
    kernel_variant: int = 0,
    block_table: Optional[torch.Tensor] = None,
    block_size: int = 0,
) -> torch.Tensor:
    """``mla_decode`` for queries already in latent space: q_absorbed
    (batch, num_heads, kv_lora_rank) fp32 (e.g. x . W_Q_absorbed^T). Same
    cache / sequence arguments; returns (batch, num_heads, v_head_dim) fp32."""
    _C = _load_ext()
    return _C.mla_decode_absorbed_forward(kv_cache, q_absorbed, q_rope, W_UV, rope_cos, rope_sin, seq_offsets,
                                          *_cfg_args(cfg), chunk_rows, kernel_variant, seq_lens, block_table,
                                          block_size)


def append_kv(
    kv_cache: torch.Tensor,
    seq_lens: torch.Tensor,
    c_t: torch.Tensor,
    k_rope: torch.Tensor,
    cfg: "MLAConfig",
    q_rope: Optional[torch.Tensor] = None,
    rope_cos: Optional[torch.Tensor] = None,
    rope_sin: Optional[torch.Tensor] = None,
    seq_offsets: Optional[torch.Tensor] = None,
    status: Optional[torch.Tensor] = None,
    block_table: Optional[torch.Tensor] = None,
    block_size: int = 0,
) -> None:
    """Append new latent rows to every sequence's cache on the device.

    The device-side counterpart of the reference's
    ``LatentKVCache::append_host`` (src/mla_config.cuh:57-72) for a batch:
    no host copies and no synchronize; lengths are kept on the device.

    Args:
        kv_cache:    (batch, capacity, dc + dR) when ``seq_offsets`` is None,
                     else a packed (rows, dc + dR) cache whose sequence b owns
                     rows [seq_offsets[b], seq_offsets[b+1])
        seq_lens:    int32 (batch,) device tensor of filled rows, advanced in
                     place by the number of appended tokens
        c_t, k_rope: (batch, tokens, dc) and (batch, tokens, dR), one dtype;
                     k_rope un-rotated (keys are rotated by position inside
                     the attention)
        q_rope:      optional (batch * queries_per_seq, num_heads, dR) fp32,
                     rotated in place for the positions of the last
                     queries_per_seq appended tokens (needs rope_cos/sin)
        status:      optional int32 device tensor; element 0 is set to 1 when
                     a sequence has no room (that sequence is left unchanged)
        block_table, block_size: optional paged cache, as in ``mla_decode``
                     (capacity block_table.shape[1] * block_size per sequence)
    """
    _C = _load_ext()
    _C.append_kv_forward(kv_cache, seq_lens, c_t, k_rope, q_rope, rope_cos, rope_sin, seq_offsets, status,
                         *_cfg_args(cfg), block_table, block_size)


def absorb_q(q_nope: torch.Tensor, W_UK: torch.Tensor, cfg: "MLAConfig") -> torch.Tensor:
    """q_absorbed[..., h, c] = sum_i q_nope[..., h, i] * W_UK[h*dn + i, c] (fp32)."""
    _C = _load_ext()
    return _C.absorb_q_forward(q_nope, W_UK, *_cfg_args(cfg))
