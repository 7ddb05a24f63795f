"""MI355X-native multi-head latent attention (MLA) decode.

Drop-in for the reference package's API (latent_attn/__init__.py and
latent_attn/functional.py in the reference repo): ``MLAConfig``,
``_build_rope_tables`` and the functional entry points, backed by hand-written
gfx950 HIP kernels in ``liblatent_attn_hip.so`` through the ``_C`` extension.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

__all__ = ["MLAConfig", "LatentAttentionLayer", "build_rope_tables", "_build_rope_tables"]


@dataclass
class MLAConfig:
    """Same fields and defaults as the reference MLAConfig
    (latent_attn/__init__.py:13-28, src/mla_config.cuh:7-23)."""

    d_model: int
    kv_lora_rank: int  # d_c: compressed KV latent dimension
    qk_nope_head_dim: int  # per-head non-RoPE dim
    qk_rope_head_dim: int  # per-head RoPE dim (d_R)
    num_heads: int
    v_head_dim: int

    @staticmethod
    def deepseek_v2() -> "MLAConfig":
        return MLAConfig(5120, 512, 128, 64, 128, 128)

    @staticmethod
    def deepseek_v3() -> "MLAConfig":
        return MLAConfig(7168, 512, 128, 64, 128, 128)

    def bytes_per_kv_entry(self, dtype: torch.dtype = torch.float16) -> int:
        """Bytes of one packed cache row [c_t | k_rope] (src/mla_config.cuh:26-28)."""
        return (self.kv_lora_rank + self.qk_rope_head_dim) * torch.empty((), dtype=dtype).element_size()

    def kv_cache_bytes(self, seq_len: int, dtype: torch.dtype = torch.float16) -> int:
        return seq_len * self.bytes_per_kv_entry(dtype)

    def validate(self) -> None:
        """Raise ValueError on non-positive dims (src/mla_config.cuh:35-40)."""
        if self.kv_lora_rank <= 0 or self.qk_nope_head_dim <= 0 or self.qk_rope_head_dim <= 0:
            raise ValueError("MLA dims must be positive")
        if self.num_heads <= 0 or self.v_head_dim <= 0:
            raise ValueError("num_heads and v_head_dim must be positive")


def build_rope_tables(seq_len: int, d_R: int, device=None, base: float = 10000.0):
    """(cos, sin), each (seq_len, d_R // 2) float32: angle = pos * base^(-2i/d_R).

    Same construction as the reference (latent_attn/__init__.py:31-38).
    """
    half = d_R // 2
    positions = torch.arange(seq_len, dtype=torch.float32, device=device)
    dims = torch.arange(half, dtype=torch.float32, device=device)
    freqs = 1.0 / (base ** (2.0 * dims / d_R))
    angles = positions[:, None] * freqs[None, :]
    return angles.cos(), angles.sin()


def _build_rope_tables(seq_len: int, d_R: int, device: torch.device):
    return build_rope_tables(seq_len, d_R, device)


from .layer import LatentAttentionLayer  # noqa: E402  (needs MLAConfig and build_rope_tables above)
