"""GPU parity of the device-side cache append (la_append_kv, through the torch
extension) and of decode over a capacity cache with device-side lengths
(la_decode_args.seq_lens), against the oracle's append_rows /
rotate_queries / decode_sequences.

The append is byte work: the cache rows must equal the oracle's rows
bit-for-bit (values rounded to the cache dtype, round-to-nearest-even) and the
lengths exactly. The query rotation is fp32 arithmetic on fp32 inputs:
|d| <= 1e-5 + 1e-5*|ref|. Decode uses the bf16 tolerance of the other parity
tests (tests/conftest.py:assert_close). Replaces the reference's host-side
LatentKVCache::append_host (src/mla_config.cuh:57-72), which has no tests of
its own.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import assert_close
from mla_cases import TORCH_DTYPE, make_queries, make_weights, rope, to_np
from oracle import mla_oracle as mo

from latent_attn import MLAConfig
from latent_attn import functional as F

pytestmark = pytest.mark.gpu

ROW = 576


def dims(cfg: MLAConfig) -> mo.Dims:
    return mo.Dims(cfg.d_model, cfg.kv_lora_rank, cfg.qk_nope_head_dim, cfg.qk_rope_head_dim, cfg.num_heads,
                   cfg.v_head_dim)


def new_rows(B, T, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    c_t = torch.randn(B, T, 512, generator=g).to(TORCH_DTYPE[dtype])
    k_rope = torch.randn(B, T, 64, generator=g).to(TORCH_DTYPE[dtype])
    return c_t, k_rope


def filled_decode_ref(kv_np, starts, lens, q_nope, q_rope, W_UK, W_UV, cos, sin, cfg):
    """Oracle decode over the filled rows of each region (positions from 0)."""
    rows = [kv_np[s:s + l] for s, l in zip(starts, lens)]
    packed = np.concatenate(rows, axis=0) if rows else np.zeros((0, ROW))
    offsets = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    d = dims(cfg)
    qa = mo.absorb_q(to_np(q_nope), to_np(W_UK), d)
    return mo.decode_sequences(packed, offsets, qa, to_np(q_rope), to_np(W_UV), to_np(cos), to_np(sin), d)


@pytest.mark.parametrize("cache_dtype,src_dtype", [("bf16", "f32"), ("bf16", "bf16"), ("f16", "f32"), ("f32", "f16")])
def test_append_steps_then_decode(cuda, cache_dtype, src_dtype):
    """Eight single-token appends into a (B, capacity) cache, then decode with
    seq_lens: rows and lengths equal the oracle's exactly, the decode equals
    the oracle's decode over the filled rows."""
    cfg = MLAConfig.deepseek_v2()
    B, cap, steps = 3, 300, 8
    lens0 = [0, 37, 250]
    g = torch.Generator().manual_seed(5)
    kv = torch.randn(B, cap, ROW, generator=g).to(TORCH_DTYPE[cache_dtype]).to(cuda)
    kv_np = to_np(kv).reshape(B * cap, ROW)
    lens = torch.tensor(lens0, dtype=torch.int32, device=cuda)
    lens_np = np.array(lens0)
    starts, caps = [b * cap for b in range(B)], [cap] * B
    for step in range(steps):
        c_t, k_rope = new_rows(B, 1, src_dtype, 100 + step)
        F.append_kv(kv, lens, c_t.to(cuda), k_rope.to(cuda), cfg)
        kv_np, lens_np, full = mo.append_rows(kv_np, starts, caps, lens_np, to_np(c_t), to_np(k_rope), cache_dtype)
        assert not full
    torch.cuda.synchronize()
    assert lens.cpu().tolist() == list(lens_np)
    assert np.array_equal(to_np(kv).reshape(B * cap, ROW), kv_np), "cache rows differ from the oracle's"

    W_UK, W_UV = make_weights(cfg, "bf16", 7, cuda)
    q_nope, q_rope = make_queries((B,), cfg, 8, cuda)
    cos, sin = rope(cap, cfg, cuda)
    out = F.mla_decode(kv, q_nope, q_rope, W_UK, W_UV, cos, sin, cfg, seq_lens=lens)
    torch.cuda.synchronize()
    ref = filled_decode_ref(kv_np, starts, list(lens_np), q_nope, q_rope, W_UK, W_UV, cos, sin, cfg)
    # bf16 weights in every case: the 16-bit tolerance applies
    assert_close(out.cpu().numpy(), ref, "bf16", "decode after appends")


def test_append_multi_token_rotates_queries(cuda):
    """Four tokens per sequence, two queries each: q_rope row j of sequence b
    is rotated for position len_b + 4 - 2 + j (rotate-half, fp32 tables)."""
    cfg = MLAConfig.deepseek_v2()
    B, cap, T, qps = 2, 64, 4, 2
    kv = torch.zeros(B, cap, ROW, dtype=torch.bfloat16, device=cuda)
    lens0 = [3, 60]
    lens = torch.tensor(lens0, dtype=torch.int32, device=cuda)
    c_t, k_rope = new_rows(B, T, "bf16", 11)
    g = torch.Generator().manual_seed(12)
    q = torch.randn(B * qps, cfg.num_heads, 64, generator=g)
    q_dev = q.to(cuda)
    cos, sin = rope(cap, cfg, cuda)
    F.append_kv(kv, lens, c_t.to(cuda), k_rope.to(cuda), cfg, q_rope=q_dev, rope_cos=cos, rope_sin=sin)
    torch.cuda.synchronize()
    ref = mo.rotate_queries(q.numpy().astype(np.float64), lens0, T, qps, to_np(cos), to_np(sin))
    got = q_dev.cpu().numpy().astype(np.float64)
    assert np.all(np.abs(got - ref) <= 1e-5 + 1e-5 * np.abs(ref)), float(np.abs(got - ref).max())
    # sequence 1 (60 + 4 = 64 = capacity) fits exactly
    assert lens.cpu().tolist() == [7, 64]


def test_append_refuses_a_full_sequence(cuda):
    """A sequence without room keeps its rows, length and query untouched
    and raises the status flag; the others are appended."""
    cfg = MLAConfig.deepseek_v2()
    B, cap, T = 2, 4, 3
    kv = torch.full((B, cap, ROW), 0.5, dtype=torch.bfloat16, device=cuda)
    lens = torch.tensor([1, 2], dtype=torch.int32, device=cuda)
    status = torch.zeros(1, dtype=torch.int32, device=cuda)
    c_t, k_rope = new_rows(B, T, "bf16", 21)
    q = torch.randn(B, cfg.num_heads, 64, generator=torch.Generator().manual_seed(22)).to(cuda)
    q0 = q.clone()
    cos, sin = rope(16, cfg, cuda)
    F.append_kv(kv, lens, c_t.to(cuda), k_rope.to(cuda), cfg, q_rope=q, rope_cos=cos, rope_sin=sin, status=status)
    torch.cuda.synchronize()
    assert status.item() == 1
    assert lens.cpu().tolist() == [4, 2]
    assert torch.equal(kv[1].cpu(), torch.full((cap, ROW), 0.5, dtype=torch.bfloat16))
    assert torch.equal(q[1], q0[1])
    assert torch.equal(kv[0, 1:4, :512].cpu(), c_t[0]) and torch.equal(kv[0, 1:4, 512:].cpu(), k_rope[0])


@pytest.mark.parametrize("variant", [1, 2])
def test_packed_regions_append_and_ragged_decode(cuda, variant):
    """Packed regions (seq_offsets) with ragged lengths, one of them still
    empty: append one token each, then decode with offsets + lengths on both
    attention kernels; unfilled capacity between regions is never read (it
    holds huge values that would dominate any softmax)."""
    cfg = MLAConfig.deepseek_v2()
    offsets0 = [0, 100, 130, 400]
    lens0 = [0, 29, 200]
    rows = offsets0[-1]
    kv = torch.full((rows, ROW), 1e4, dtype=torch.bfloat16)
    g = torch.Generator().manual_seed(31)
    for b in range(3):
        kv[offsets0[b]:offsets0[b] + lens0[b]] = torch.randn(lens0[b], ROW, generator=g).to(torch.bfloat16)
    kv = kv.to(cuda)
    kv_np = to_np(kv)
    offsets = torch.tensor(offsets0, dtype=torch.int32, device=cuda)
    lens = torch.tensor(lens0, dtype=torch.int32, device=cuda)
    c_t, k_rope = new_rows(3, 1, "f32", 32)
    F.append_kv(kv, lens, c_t.to(cuda), k_rope.to(cuda), cfg, seq_offsets=offsets)
    caps = [offsets0[b + 1] - offsets0[b] for b in range(3)]
    kv_np, lens_np, full = mo.append_rows(kv_np, offsets0[:3], caps, lens0, to_np(c_t), to_np(k_rope), "bf16")
    assert not full
    torch.cuda.synchronize()
    assert lens.cpu().tolist() == list(lens_np)
    assert np.array_equal(to_np(kv), kv_np)

    W_UK, W_UV = make_weights(cfg, "bf16", 33, cuda)
    q_nope, q_rope = make_queries((3,), cfg, 34, cuda)
    cos, sin = rope(300, cfg, cuda)
    out = F.mla_decode(kv, q_nope, q_rope, W_UK, W_UV, cos, sin, cfg, seq_offsets=offsets, seq_lens=lens,
                       kernel_variant=variant, chunk_rows=64)
    torch.cuda.synchronize()
    ref = filled_decode_ref(kv_np, offsets0[:3], list(lens_np), q_nope, q_rope, W_UK, W_UV, cos, sin, cfg)
    assert_close(out.cpu().numpy(), ref, "bf16", f"packed regions variant {variant}")


@pytest.mark.parametrize("chunk_rows", [0, 64, 96])
def test_seq_lens_decode_equals_trimmed_cache(cuda, chunk_rows):
    """Decode of a (B, capacity) cache with seq_lens equals decode of the
    same rows without the unfilled tail (a packed ragged cache), for chunk
    sizes that split the regions at different rows."""
    cfg = MLAConfig.deepseek_v2()
    B, cap = 4, 512
    lens0 = [512, 1, 300, 0]
    g = torch.Generator().manual_seed(41)
    kv = torch.randn(B, cap, ROW, generator=g).to(torch.bfloat16).to(cuda)
    lens = torch.tensor(lens0, dtype=torch.int32, device=cuda)
    W_UK, W_UV = make_weights(cfg, "bf16", 42, cuda)
    q_nope, q_rope = make_queries((B,), cfg, 43, cuda)
    cos, sin = rope(cap, cfg, cuda)
    out = F.mla_decode(kv, q_nope, q_rope, W_UK, W_UV, cos, sin, cfg, seq_lens=lens, chunk_rows=chunk_rows)
    packed = torch.cat([kv[b, :lens0[b]] for b in range(B)], dim=0)
    offsets = torch.tensor(np.concatenate([[0], np.cumsum(lens0)]), dtype=torch.int32, device=cuda)
    out2 = F.mla_decode(packed, q_nope, q_rope, W_UK, W_UV, cos, sin, cfg, seq_offsets=offsets,
                        chunk_rows=chunk_rows)
    torch.cuda.synchronize()
    assert torch.equal(out[3].cpu(), torch.zeros(cfg.num_heads, cfg.v_head_dim))
    ref = filled_decode_ref(to_np(kv).reshape(B * cap, ROW), [b * cap for b in range(B)], lens0, q_nope, q_rope,
                            W_UK, W_UV, cos, sin, cfg)
    assert_close(out.cpu().numpy(), ref, "bf16", "seq_lens decode")
    assert_close(out2.cpu().numpy(), ref, "bf16", "packed decode")
