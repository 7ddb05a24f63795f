"""CPU checks of latent_attn.LatentAttentionLayer against the reference
module's constructor (latent_attn/__init__.py:48-90 in the reference repo):
parameter names, shapes and dtype, initialisation scale, RoPE buffers, and
the forward's argument checks. No kernel runs here."""

from __future__ import annotations

import math

import pytest
import torch

from latent_attn import LatentAttentionLayer, MLAConfig, build_rope_tables


def test_parameters_and_buffers_match_the_reference_module():
    cfg = MLAConfig(256, 64, 32, 16, 8, 24)
    torch.manual_seed(0)
    layer = LatentAttentionLayer(cfg, max_seq_len=100)
    shapes = {n: tuple(p.shape) for n, p in layer.named_parameters()}
    assert shapes == {
        "W_Q_absorbed": (8 * 64, 256),
        "W_Q_rope": (8 * 16, 256),
        "W_UK": (8 * 32, 64),
        "W_UV": (8 * 24, 64),
        "W_O": (256, 8 * 24),
    }
    assert all(p.dtype == torch.float32 for p in layer.parameters())
    cos, sin = build_rope_tables(100, 16)
    assert torch.equal(layer.rope_cos, cos) and torch.equal(layer.rope_sin, sin)
    assert LatentAttentionLayer.from_config(cfg, 16).rope_cos.shape == (16, 8)


def test_initialisation_scale():
    """normal(0, 0.02) for the projections, 0.02/sqrt(2) for W_O."""
    cfg = MLAConfig(512, 128, 64, 32, 16, 64)
    torch.manual_seed(1)
    layer = LatentAttentionLayer(cfg, max_seq_len=8)
    for name in ("W_Q_absorbed", "W_Q_rope", "W_UK", "W_UV"):
        std = getattr(layer, name).std().item()
        assert abs(std - 0.02) < 0.02 * 0.03, (name, std)
    assert abs(layer.W_O.std().item() - 0.02 / math.sqrt(2.0)) < 0.02 * 0.03
    assert abs(layer.W_Q_absorbed.mean().item()) < 1e-3


def test_forward_checks_the_token_shape():
    cfg = MLAConfig(64, 32, 16, 8, 2, 16)
    layer = LatentAttentionLayer(cfg, max_seq_len=8)
    kv = torch.zeros(4, 40, dtype=torch.float16)
    with pytest.raises(ValueError):
        layer.forward(torch.zeros(2, 64), kv)
    with pytest.raises(ValueError):
        layer.forward(torch.zeros(63), kv)
    with pytest.raises(ValueError):
        layer.forward_batch(torch.zeros(64), kv)
