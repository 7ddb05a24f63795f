"""GPU parity of latent_attn.LatentAttentionLayer (the reference module's
forward, latent_attn/__init__.py:110-145 in the reference repo) against the
oracle's layer_forward on the module's own parameters, and of the batched
forward against per-sequence single-token forwards.

Tolerance: the 16-bit one of the other parity tests (fp16 / bf16 caches, the
fp16 W_UV the reference itself uses), including the scale-free normwise
bound 1e-2 (tests/conftest.py:assert_close).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import assert_close
from mla_cases import to_np
from oracle import mla_oracle as mo

from latent_attn import LatentAttentionLayer, MLAConfig

pytestmark = pytest.mark.gpu


def dims(cfg):
    return mo.Dims(cfg.d_model, cfg.kv_lora_rank, cfg.qk_nope_head_dim, cfg.qk_rope_head_dim, cfg.num_heads,
                   cfg.v_head_dim)


def oracle_y(layer, x, kv):
    return mo.layer_forward(to_np(x), to_np(kv), to_np(layer.W_Q_absorbed), to_np(layer.W_Q_rope),
                            to_np(layer.W_UV), to_np(layer.W_O), to_np(layer.rope_cos), to_np(layer.rope_sin),
                            dims(layer.cfg))


@pytest.mark.parametrize("heads,S,dtype", [(16, 300, torch.float16), (128, 1000, torch.float16),
                                            (16, 257, torch.bfloat16)])
def test_layer_forward_matches_oracle(cuda, heads, S, dtype):
    cfg = MLAConfig(1024, 512, 128, 64, heads, 128)
    torch.manual_seed(7)
    layer = LatentAttentionLayer(cfg, max_seq_len=2048).to(cuda)
    g = torch.Generator().manual_seed(8)
    kv = torch.randn(S, 576, generator=g).to(dtype).to(cuda)
    x = torch.randn(cfg.d_model, generator=g).to(cuda)
    y = layer(x, kv)
    torch.cuda.synchronize()
    assert y.shape == (cfg.d_model,) and y.dtype == torch.float32
    assert_close(y.cpu().numpy(), oracle_y(layer, x, kv), "bf16", f"layer forward H={heads} S={S}")
    y2 = layer(x.unsqueeze(0), kv)  # (1, d_model) is accepted too
    torch.cuda.synchronize()
    assert torch.equal(y, y2)


def test_layer_forward_batch_equals_single_tokens(cuda):
    """forward_batch over a uniform batch, a packed ragged batch and a
    capacity cache with device lengths equals forward on each sequence."""
    cfg = MLAConfig(1024, 512, 128, 64, 32, 128)
    torch.manual_seed(9)
    layer = LatentAttentionLayer(cfg, max_seq_len=1024).to(cuda)
    g = torch.Generator().manual_seed(10)
    B, S = 3, 400
    kv = torch.randn(B, S, 576, generator=g).to(torch.float16).to(cuda)
    x = torch.randn(B, cfg.d_model, generator=g).to(cuda)
    singles = torch.stack([layer(x[b], kv[b]) for b in range(B)])
    yb = layer.forward_batch(x, kv)
    lens = [400, 1, 123]
    packed = torch.cat([kv[b, :lens[b]] for b in range(B)])
    offsets = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int32, device=cuda)
    yr = layer.forward_batch(x, packed, seq_offsets=offsets)
    yl = layer.forward_batch(x, kv, seq_lens=torch.tensor(lens, dtype=torch.int32, device=cuda))
    singles_r = torch.stack([layer(x[b], kv[b, :lens[b]]) for b in range(B)])
    torch.cuda.synchronize()
    ref = np.stack([oracle_y(layer, x[b], kv[b]) for b in range(B)])
    assert_close(yb.cpu().numpy(), ref, "bf16", "forward_batch uniform")
    assert_close(singles.cpu().numpy(), ref, "bf16", "forward singles")
    ref_r = np.stack([oracle_y(layer, x[b], kv[b, :lens[b]]) for b in range(B)])
    assert_close(yr.cpu().numpy(), ref_r, "bf16", "forward_batch ragged")
    assert_close(yl.cpu().numpy(), ref_r, "bf16", "forward_batch seq_lens")
    assert_close(singles_r.cpu().numpy(), ref_r, "bf16", "forward singles ragged")


def test_layer_forward_batch_over_a_paged_cache(cuda):
    """forward_batch through a block table equals forward_batch over the same
    rows laid out contiguously (bit for bit: same kernel, same rows)."""
    cfg = MLAConfig(1024, 512, 128, 64, 16, 128)
    torch.manual_seed(11)
    layer = LatentAttentionLayer(cfg, max_seq_len=512).to(cuda)
    g = torch.Generator().manual_seed(12)
    B, cap, bs = 2, 512, 64
    kv = torch.randn(B, cap, 576, generator=g).to(torch.bfloat16).to(cuda)
    perm = torch.from_numpy(np.random.RandomState(13).permutation(B * cap // bs).astype(np.int32)).to(cuda)
    pool = torch.empty(B * cap, 576, dtype=torch.bfloat16, device=cuda)
    pool.view(-1, bs, 576)[perm.long()] = kv.view(-1, bs, 576)
    lens = torch.tensor([512, 200], dtype=torch.int32, device=cuda)
    x = torch.randn(B, cfg.d_model, generator=g).to(cuda)
    y_c = layer.forward_batch(x, kv, seq_lens=lens)
    y_p = layer.forward_batch(x, pool, seq_lens=lens, block_table=perm.view(B, cap // bs), block_size=bs)
    torch.cuda.synchronize()
    assert torch.equal(y_c, y_p)
