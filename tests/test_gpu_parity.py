"""GPU parity: HIP kernels (through the torch extension, which calls the C ABI)
against the float64 oracle on the same seeded inputs.

Tolerances (north star): bf16/fp16 inputs with fp32 accumulation match within
|d| <= 2e-2 + 1e-2*|ref| elementwise and 1e-2 normwise; fp32 mode within
1e-4 + 1e-4*|ref| and 1e-5 normwise (tests/conftest.py:assert_close).

Ports of the reference's tests: tests/test_python.py:72-138 (fused vs naive
vs torch reference at H=128, kv_len 512/2048/8192) and tests/test_batched.py
:33-88 (batched == loop of single calls, B in {1,4,16,64}, S=1024), with the
cosine > 0.998 gate replaced by the oracle tolerance above.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import assert_close
from mla_cases import cfg_with_heads, make_cache, make_queries, make_weights, rope, to_np
from oracle import mla_oracle as mo

from latent_attn import MLAConfig
from latent_attn import functional as F

pytestmark = pytest.mark.gpu


def dims(cfg: MLAConfig) -> mo.Dims:
    return mo.Dims(cfg.d_model, cfg.kv_lora_rank, cfg.qk_nope_head_dim, cfg.qk_rope_head_dim, cfg.num_heads,
                   cfg.v_head_dim)


def oracle_decode(kv, offsets, q_nope, q_rope, W_UK, W_UV, cos, sin, cfg):
    """float64 oracle for mla_decode: absorb then per-sequence latent attention."""
    d = dims(cfg)
    qa = mo.absorb_q(to_np(q_nope), to_np(W_UK), d)
    return mo.decode_sequences(to_np(kv), offsets, qa, to_np(q_rope), to_np(W_UV), to_np(cos), to_np(sin), d)


def single_case(cfg, S, dtype, seed, cuda):
    kv = make_cache((S,), cfg, dtype, seed, cuda)
    W_UK, W_UV = make_weights(cfg, dtype, seed + 1, cuda)
    q_nope, q_rope = make_queries((), cfg, seed + 2, cuda)
    cos, sin = rope(S, cfg, cuda)
    return kv, W_UK, W_UV, q_nope, q_rope, cos, sin


# ---------------------------------------------------------------------------
# B=1, H=16, S=256 -- fp32 mode (1e-4) and 16-bit modes
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
def test_config1_fused_and_naive(cuda, dtype):
    cfg = cfg_with_heads(16)
    kv, W_UK, W_UV, q_nope, q_rope, cos, sin = single_case(cfg, 256, dtype, 0, cuda)
    d = dims(cfg)
    ref = mo.naive_mla(to_np(kv), to_np(W_UK), to_np(W_UV), to_np(q_nope), to_np(q_rope), to_np(cos), to_np(sin), d)
    q_abs = torch.from_numpy(mo.absorb_q(to_np(q_nope), to_np(W_UK), d).astype(np.float32)).to(cuda)
    out = F.fused_mla(kv, q_abs, q_rope, W_UV, cos, sin, cfg)
    torch.cuda.synchronize()
    assert out.shape == (16, 128) and out.dtype == torch.float32
    assert_close(out.cpu().numpy(), ref, dtype, f"fused_mla cfg1 {dtype}")
    out2 = F.naive_mla(kv, W_UK, W_UV, q_nope, q_rope, cos, sin, cfg)
    assert_close(out2.cpu().numpy(), ref, dtype, f"naive_mla cfg1 {dtype}")


@pytest.mark.parametrize("variant", [1, 2])
def test_config1_both_kernels(cuda, variant):
    """Same bf16 inputs through the VALU (1) and the MFMA (2) decode kernels."""
    cfg = cfg_with_heads(16)
    kv, W_UK, W_UV, q_nope, q_rope, cos, sin = single_case(cfg, 256, "bf16", 3, cuda)
    ref = oracle_decode(kv, [0, 256], q_nope[None], q_rope[None], W_UK, W_UV, cos, sin, cfg)
    out = F.mla_decode(kv[None], q_nope[None].contiguous(), q_rope[None].contiguous(), W_UK, W_UV, cos, sin, cfg,
                       kernel_variant=variant)
    assert_close(out.cpu().numpy(), ref, "bf16", f"variant {variant}")


# ---------------------------------------------------------------------------
# port of reference tests/test_python.py:72-138
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("kv_len", [512, 2048, 8192])
@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_fused_vs_naive_and_oracle(cuda, kv_len, dtype):
    cfg = MLAConfig.deepseek_v2()
    kv, W_UK, W_UV, q_nope, q_rope, cos, sin = single_case(cfg, kv_len, dtype, 42, cuda)
    d = dims(cfg)
    qa_np = mo.absorb_q(to_np(q_nope), to_np(W_UK), d)
    ref = mo.absorbed_mla(to_np(kv), qa_np, to_np(q_rope), to_np(W_UV), to_np(cos), to_np(sin), d)
    q_abs = torch.from_numpy(qa_np.astype(np.float32)).to(cuda)
    fused = F.fused_mla(kv, q_abs, q_rope, W_UV, cos, sin, cfg).cpu().numpy()
    naive = F.naive_mla(kv, W_UK, W_UV, q_nope, q_rope, cos, sin, cfg).cpu().numpy()
    assert_close(fused, ref, dtype, f"fused kv_len={kv_len}")
    assert_close(naive, ref, dtype, f"naive kv_len={kv_len}")


def test_naive_oracle_agrees_on_reference_shape(cuda):
    """Decompress-then-attend oracle at the reference test's smallest shape,
    against the GPU: pins the GPU to the naive math directly (not only the
    absorbed restatement)."""
    cfg = MLAConfig.deepseek_v2()
    kv, W_UK, W_UV, q_nope, q_rope, cos, sin = single_case(cfg, 512, "bf16", 7, cuda)
    ref = mo.naive_mla(to_np(kv), to_np(W_UK), to_np(W_UV), to_np(q_nope), to_np(q_rope), to_np(cos), to_np(sin),
                       dims(cfg))
    out = F.naive_mla(kv, W_UK, W_UV, q_nope, q_rope, cos, sin, cfg).cpu().numpy()
    assert_close(out, ref, "bf16", "naive S=512")


# ---------------------------------------------------------------------------
# port of reference tests/test_batched.py:33-88 (shared cache)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("batch", [1, 4, 16, 64])
def test_batched_vs_single_loop(cuda, batch):
    cfg = MLAConfig.deepseek_v2()
    S = 1024
    kv = make_cache((S,), cfg, "bf16", batch, cuda)
    _, W_UV = make_weights(cfg, "bf16", batch + 1, cuda)
    g = torch.Generator().manual_seed(batch + 2)
    q_abs = (torch.randn(batch, cfg.num_heads, cfg.kv_lora_rank, generator=g) * 0.5).to(cuda)
    q_rope = torch.randn(batch, cfg.num_heads, cfg.qk_rope_head_dim, generator=g).to(cuda)
    cos, sin = rope(S, cfg, cuda)
    out_b = F.batched_fused_mla(kv, q_abs, q_rope, W_UV, cos, sin, cfg)
    out_l = torch.stack([F.fused_mla(kv, q_abs[i].contiguous(), q_rope[i].contiguous(), W_UV, cos, sin, cfg)
                         for i in range(batch)])
    ref = mo.batched_absorbed_mla(to_np(kv), to_np(q_abs), to_np(q_rope), to_np(W_UV), to_np(cos), to_np(sin),
                                  dims(cfg))
    assert_close(out_b.cpu().numpy(), ref, "bf16", f"batched B={batch}")
    assert_close(out_l.cpu().numpy(), ref, "bf16", f"loop B={batch}")


# ---------------------------------------------------------------------------
# mla_decode: per-sequence caches, split invariance, ragged, edge cases
# ---------------------------------------------------------------------------

def test_uniform_batch_decode(cuda):
    cfg = MLAConfig.deepseek_v2()
    B, S = 6, 1500
    kv = make_cache((B, S), cfg, "bf16", 11, cuda)
    W_UK, W_UV = make_weights(cfg, "bf16", 12, cuda)
    q_nope, q_rope = make_queries((B,), cfg, 13, cuda)
    cos, sin = rope(S, cfg, cuda)
    ref = oracle_decode(kv.reshape(B * S, -1), [b * S for b in range(B + 1)], q_nope, q_rope, W_UK, W_UV, cos, sin,
                        cfg)
    out = F.mla_decode(kv, q_nope, q_rope, W_UK, W_UV, cos, sin, cfg)
    assert_close(out.cpu().numpy(), ref, "bf16", "uniform B=6 S=1500")


@pytest.mark.parametrize("chunk_rows", [32, 96, 100, 777, 3000])
@pytest.mark.parametrize("variant", [1, 2])
def test_split_invariance(cuda, chunk_rows, variant):
    """Any split-KV chunking (including chunks that cut tiles and sequences
    mid-way) gives the unsplit oracle's answer."""
    cfg = MLAConfig.deepseek_v2()
    B, S = 2, 1000
    kv = make_cache((B, S), cfg, "bf16", 21, cuda)
    W_UK, W_UV = make_weights(cfg, "bf16", 22, cuda)
    q_nope, q_rope = make_queries((B,), cfg, 23, cuda)
    cos, sin = rope(S, cfg, cuda)
    ref = oracle_decode(kv.reshape(B * S, -1), [0, S, 2 * S], q_nope, q_rope, W_UK, W_UV, cos, sin, cfg)
    out = F.mla_decode(kv, q_nope, q_rope, W_UK, W_UV, cos, sin, cfg, chunk_rows=chunk_rows, kernel_variant=variant)
    assert_close(out.cpu().numpy(), ref, "bf16", f"chunk_rows={chunk_rows} variant={variant}")


@pytest.mark.parametrize("B,S,picks", [(17, 4096, (0, 8, 16)), (1, 32768, (0,))])
def test_merge_over_many_slots(cuda, B, S, picks):
    """32-row chunks give every query row S/32 partial slots (plus one where a
    chunk straddles two sequences). B = 17 (272 row blocks x heads: the
    full-row merge) has 128 slots per row, one wave per row: its slot weights
    come in two blocks of 64. B = 1 (the latent-half merge, a row's slots split
    over 8 waves) has 1,024 slots, 128 per wave: two blocks as well, and the
    row maximum and denominator loop past the first 64 slots."""
    cfg = MLAConfig.deepseek_v2()
    kv = make_cache((B, S), cfg, "bf16", 26, cuda)
    W_UK, W_UV = make_weights(cfg, "bf16", 27, cuda)
    q_nope, q_rope = make_queries((B,), cfg, 28, cuda)
    cos, sin = rope(S, cfg, cuda)
    out = F.mla_decode(kv, q_nope, q_rope, W_UK, W_UV, cos, sin, cfg, chunk_rows=32).cpu().numpy()
    print(f"[many slots] B={B} S={S} chunk_rows=32: {S // 32} slots per row", flush=True)
    assert np.isfinite(out).all()
    for b in picks:
        ref = oracle_decode(kv[b], [0, S], q_nope[b:b + 1], q_rope[b:b + 1], W_UK, W_UV, cos, sin, cfg)
        assert_close(out[b], ref[0], "bf16", f"B={B} S={S} seq {b}, {S // 32} slots per row")


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_other_head_dims(cuda, dtype):
    """A shape other than DeepSeek's (kv_lora_rank 256, qk_rope_head_dim 32,
    qk_nope_head_dim 64, v_head_dim 96, 12 heads; MLAConfig allows any
    positive dims with an even rope dim, src/mla_config.cuh:35-40) runs on the
    VALU kernels (absorb on MFMA, whose 128-column blocks still fit), over a
    ragged batch with a one-position sequence, against the oracle; the naive
    path on one sequence too."""
    cfg = MLAConfig(1024, 256, 64, 32, 12, 96)
    lens = [100, 1, 333]
    offs = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    kv = make_cache((int(offs[-1]),), cfg, dtype, 36, cuda)
    W_UK, W_UV = make_weights(cfg, dtype, 37, cuda)
    q_nope, q_rope = make_queries((len(lens),), cfg, 38, cuda)
    cos, sin = rope(max(lens), cfg, cuda)
    ref = oracle_decode(kv, offs, q_nope, q_rope, W_UK, W_UV, cos, sin, cfg)
    off_t = torch.tensor(offs, dtype=torch.int32, device=cuda)
    out = F.mla_decode(kv, q_nope, q_rope, W_UK, W_UV, cos, sin, cfg, seq_offsets=off_t).cpu().numpy()
    assert_close(out, ref, dtype, f"dims 256/32/64/96 x 12 heads ({dtype})")
    d = dims(cfg)
    kv2 = kv[int(offs[2]):int(offs[3])]
    naive = F.naive_mla(kv2, W_UK, W_UV, q_nope[2], q_rope[2], cos, sin, cfg).cpu().numpy()
    ref2 = mo.naive_mla(to_np(kv2), to_np(W_UK), to_np(W_UV), to_np(q_nope[2]), to_np(q_rope[2]), to_np(cos),
                        to_np(sin), d)
    assert_close(naive, ref2, "f32" if dtype == "f32" else dtype, f"naive, other dims ({dtype})")


@pytest.mark.parametrize("variant", [1, 2])
def test_ragged_with_empty_and_short_sequences(cuda, variant):
    cfg = MLAConfig.deepseek_v2()
    lens = [5, 0, 1, 33, 700, 31, 64, 2049]
    offs = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    T = int(offs[-1])
    kv = make_cache((T,), cfg, "bf16", 31, cuda)
    W_UK, W_UV = make_weights(cfg, "bf16", 32, cuda)
    q_nope, q_rope = make_queries((len(lens),), cfg, 33, cuda)
    cos, sin = rope(max(lens), cfg, cuda)
    ref = oracle_decode(kv, offs, q_nope, q_rope, W_UK, W_UV, cos, sin, cfg)
    off_t = torch.tensor(offs, dtype=torch.int32, device=cuda)
    out = F.mla_decode(kv, q_nope, q_rope, W_UK, W_UV, cos, sin, cfg, seq_offsets=off_t, kernel_variant=variant,
                       chunk_rows=256)
    o = out.cpu().numpy()
    assert np.all(o[1] == 0.0), "empty sequence must give zeros"
    assert_close(o, ref, "bf16", f"ragged variant {variant}")


def test_single_position_closed_form(cuda):
    """S = 1: out = W_UV_h . c_0 for every head, whatever the query."""
    cfg = MLAConfig.deepseek_v2()
    kv, W_UK, W_UV, q_nope, q_rope, cos, sin = single_case(cfg, 1, "bf16", 41, cuda)
    out = F.naive_mla(kv, W_UK, W_UV, q_nope, q_rope, cos, sin, cfg).cpu().numpy()
    W = to_np(W_UV).reshape(128, 128, 512)
    assert_close(out, W @ to_np(kv)[0, :512], "f32", "S=1 closed form")


def test_zero_query_is_uniform_mean(cuda):
    cfg = MLAConfig.deepseek_v2()
    S = 777
    kv = make_cache((S,), cfg, "bf16", 51, cuda)
    _, W_UV = make_weights(cfg, "bf16", 52, cuda)
    cos, sin = rope(S, cfg, cuda)
    q_abs = torch.zeros(cfg.num_heads, cfg.kv_lora_rank, device=cuda)
    q_rope = torch.zeros(cfg.num_heads, cfg.qk_rope_head_dim, device=cuda)
    out = F.fused_mla(kv, q_abs, q_rope, W_UV, cos, sin, cfg).cpu().numpy()
    W = to_np(W_UV).reshape(128, 128, 512)
    # P = 1 exactly for every position, so the only rounding left is the split
    # partials, stored as fp16 with a power-of-two scale per half row (error at
    # most 2^-12 of the half row's max |O| per element): 1e-3 normwise and
    # elementwise relative to max|ref| -- ten times tighter than the 16-bit contract
    ref = W @ to_np(kv)[:, :512].mean(axis=0)
    from oracle.mla_oracle import norm_rel_err
    assert norm_rel_err(out, ref) <= 1e-3, norm_rel_err(out, ref)
    assert np.abs(out - ref).max() <= 1e-3 * np.abs(ref).max()


def test_extension_checks_on_device(cuda):
    cfg = MLAConfig.deepseek_v2()
    kv, W_UK, W_UV, q_nope, q_rope, cos, sin = single_case(cfg, 64, "bf16", 61, cuda)
    with pytest.raises(RuntimeError, match="q_absorbed must be float32"):
        F.fused_mla(kv, q_nope.half(), q_rope, W_UV, cos, sin, cfg)
    with pytest.raises(RuntimeError, match="q_absorbed shape mismatch"):
        F.fused_mla(kv, q_nope, q_rope, W_UV, cos, sin, cfg)
    with pytest.raises(ValueError, match="MLA dims must be positive"):
        from latent_attn import _C
        _C.fused_mla_forward(kv, torch.zeros(128, 512, device=cuda), q_rope, W_UV, cos, sin, 5120, 0, 128, 64, 128,
                             128)
    with pytest.raises(RuntimeError, match="rope_cos / rope_sin need at least"):
        F.fused_mla(kv, torch.zeros(128, 512, device=cuda), q_rope, W_UV, cos[:10], sin[:10], cfg)
    # FP8 E4M3 is a cache format only: an fp8 weight is refused with the
    # weights' message, an int cache with the caches' message (which names fp8)
    qa = torch.zeros(128, 512, device=cuda)
    with pytest.raises(RuntimeError, match="W_UV must be float16, bfloat16 or float32, got"):
        F.fused_mla(kv, qa, q_rope, W_UV.to(torch.float8_e4m3fn), cos, sin, cfg)
    with pytest.raises(RuntimeError, match="kv_cache must be float16, bfloat16, float32 or float8_e4m3fn"):
        F.fused_mla(kv.to(torch.int16), qa, q_rope, W_UV, cos, sin, cfg)


# ---------------------------------------------------------------------------
# C ABI: several query tokens per sequence, head counts that leave padded rows
# in the 32-row query blocks, absorption inside the call, ragged caches; 20
# heads (query heads not a multiple of 16) take the VALU decode and the MFMA
# projection of its fp32 partials under the automatic plan
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("heads,qps,variant", [(48, 1, 2), (48, 3, 2), (16, 2, 2), (128, 2, 2), (48, 3, 1),
                                                (20, 1, 0), (20, 3, 0)])
def test_capi_multi_query_absorb(cuda, heads, qps, variant):
    import ctypes

    from latent_attn import capi

    lib = capi.load()
    cfg = cfg_with_heads(heads)
    d = dims(cfg)
    lens = [257, 1000, 64]
    offs = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    T = int(offs[-1])
    B = len(lens)
    kv = make_cache((T,), cfg, "bf16", 71 + heads + qps, cuda)
    W_UK, W_UV = make_weights(cfg, "bf16", 72, cuda)
    q_nope, q_rope = make_queries((B * qps,), cfg, 73 + qps, cuda)
    cos, sin = rope(max(lens), cfg, cuda)
    off_t = torch.tensor(offs, dtype=torch.int32, device=cuda)
    out = torch.full((B * qps, heads, cfg.v_head_dim), float("nan"), device=cuda)
    a = capi.DecodeArgs()
    a.kv_cache, a.kv_dtype, a.total_rows, a.num_seqs = kv.data_ptr(), capi.LA_DTYPE_BF16, T, B
    a.seq_offsets, a.queries_per_seq = off_t.data_ptr(), qps
    a.q_nope, a.W_UK, a.w_uk_dtype = q_nope.data_ptr(), W_UK.data_ptr(), capi.LA_DTYPE_BF16
    a.q_rope, a.W_UV, a.w_uv_dtype = q_rope.data_ptr(), W_UV.data_ptr(), capi.LA_DTYPE_BF16
    a.rope_cos, a.rope_sin, a.rope_rows = cos.data_ptr(), sin.data_ptr(), cos.shape[0]
    a.output, a.cfg, a.kernel_variant, a.chunk_rows = out.data_ptr(), capi.config(cfg), variant, 192
    ws = torch.empty(lib.la_mla_decode_workspace_size(ctypes.byref(a)), dtype=torch.uint8, device=cuda)
    a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel()
    st = lib.la_mla_decode(ctypes.byref(a), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert st == 0, lib.la_status_string(st).decode()
    torch.cuda.synchronize()
    kvn, qn, qr, wk, wv = to_np(kv), to_np(q_nope), to_np(q_rope), to_np(W_UK), to_np(W_UV)
    ref = np.zeros((B * qps, heads, cfg.v_head_dim))
    for s_ in range(B):
        for j in range(qps):
            t = s_ * qps + j
            qa = mo.absorb_q(qn[t], wk, d)
            acc, _ = mo.absorbed_latent(kvn[offs[s_]:offs[s_ + 1]], qa, qr[t], to_np(cos), to_np(sin), d)
            ref[t] = mo.project_wuv(acc, wv, d)
    assert_close(out.cpu().numpy(), ref, "bf16", f"heads {heads} qps {qps} variant {variant}")


@pytest.mark.parametrize("wdtype", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("tokens", [1, 37])
def test_absorb_q_matches_oracle(cuda, wdtype, tokens):
    """la_absorb_q (F.absorb_q) against the oracle's absorption (reference
    tests/test_correctness.cu:29-46): the MFMA kernel for 16-bit weights
    (q_nope split into 16-bit high and low parts) and the VALU kernel for
    fp32 weights, at the fp32 tolerance; 37 tokens leave a partial 32-token
    block."""
    cfg = MLAConfig.deepseek_v2()
    W_UK, _ = make_weights(cfg, wdtype, 131, cuda)
    g = torch.Generator().manual_seed(132)
    q_nope = torch.randn(tokens, 128, 128, generator=g).to(cuda)
    out = F.absorb_q(q_nope, W_UK, cfg)
    torch.cuda.synchronize()
    ref = mo.absorb_q(to_np(q_nope), to_np(W_UK), dims(cfg))
    assert out.shape == (tokens, 128, 512) and out.dtype == torch.float32
    assert_close(out.cpu().numpy(), ref, "f32", f"absorb_q {wdtype} x{tokens}")


@pytest.mark.parametrize("chunk_rows", [1, 7])
@pytest.mark.parametrize("variant", [1, 2])
def test_chunks_shorter_than_a_tile(cuda, chunk_rows, variant):
    """Explicit chunk sizes below one 32-position tile: every chunk is a
    partial tile (masked), and a row merges up to 200 slots. B = 2 ragged
    sequences (200 and 37 positions) against the oracle."""
    cfg = MLAConfig.deepseek_v2()
    lens = [200, 37]
    offs = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    kv = make_cache((int(offs[-1]),), cfg, "bf16", 46, cuda)
    W_UK, W_UV = make_weights(cfg, "bf16", 47, cuda)
    q_nope, q_rope = make_queries((len(lens),), cfg, 48, cuda)
    cos, sin = rope(max(lens), cfg, cuda)
    ref = oracle_decode(kv, offs, q_nope, q_rope, W_UK, W_UV, cos, sin, cfg)
    off_t = torch.tensor(offs, dtype=torch.int32, device=cuda)
    out = F.mla_decode(kv, q_nope, q_rope, W_UK, W_UV, cos, sin, cfg, seq_offsets=off_t, chunk_rows=chunk_rows,
                       kernel_variant=variant)
    assert_close(out.cpu().numpy(), ref, "bf16", f"chunk_rows={chunk_rows} variant={variant}")


@pytest.mark.parametrize("kv_dtype,w_dtype", [("bf16", "f16"), ("f16", "bf16")])
def test_mixed_cache_and_weight_dtypes(cuda, kv_dtype, w_dtype):
    """Cache and weights in different 16-bit types: the attention kernel's
    queries follow the cache type, the absorb and W_UV projection follow the
    weights' type."""
    cfg = MLAConfig.deepseek_v2()
    B, S = 3, 700
    kv = make_cache((B, S), cfg, kv_dtype, 56, cuda)
    W_UK, W_UV = make_weights(cfg, w_dtype, 57, cuda)
    q_nope, q_rope = make_queries((B,), cfg, 58, cuda)
    cos, sin = rope(S, cfg, cuda)
    ref = oracle_decode(kv.reshape(B * S, -1), [b * S for b in range(B + 1)], q_nope, q_rope, W_UK, W_UV, cos, sin,
                        cfg)
    out = F.mla_decode(kv, q_nope, q_rope, W_UK, W_UV, cos, sin, cfg)
    assert_close(out.cpu().numpy(), ref, "bf16", f"cache {kv_dtype}, weights {w_dtype}")
