"""GPU parity of the MFMA decode kernel's lazy-rescale path against the
float64 oracle.

The kernel (csrc/la_mfma.hip) keeps a running maximum per head, raised only
when a tile of 32 positions beats it by more than 8 base-2 units; then O is
rescaled in AGPRs for the wave's own heads, and the wave's PV partner reads
the rescale factors from a parity-double-buffered LDS table and applies them
to the partner-head rows it holds. The staircase inputs
(tests/mla_cases.py:staircase_case) raise the maximum of every wave tens of
times per plan, at different tiles for waves 0 and 1, across chunk
boundaries (tests/test_rescale_inputs.py checks that on the CPU: per segment
the scores span tens of base-2 units, and heads 0-31 / 32-63 cross the
threshold at different tiles). A missing or misapplied rescale weights the
earlier tiers 2^10 too much, far outside the tolerance.

Semantics: reference src/fused_mla.cu:222-256 (max-subtracted softmax over
the scaled scores, then W_UV). Tolerance: bf16/fp16 allclose 2e-2 + 1e-2|ref|
and 1e-2 normwise (tests/conftest.py:assert_close), margins printed.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import assert_close
from mla_cases import make_weights, rope, staircase_case, to_np
from oracle import mla_oracle as mo
from test_gpu_paged import scatter

from latent_attn import MLAConfig
from latent_attn import functional as F

pytestmark = pytest.mark.gpu

S, B = 3000, 3
D = mo.Dims(5120, 512, 128, 64, 128, 128)


def oracle(kv, qa, qr, W_UV, cos, sin, lens):
    kv = to_np(kv)
    packed = np.concatenate([kv[b, :lens[b]] for b in range(len(lens))])
    offsets = np.concatenate([[0], np.cumsum(lens)])
    return mo.decode_sequences(packed, offsets, to_np(qa), to_np(qr), to_np(W_UV), to_np(cos), to_np(sin), D)


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
@pytest.mark.parametrize("chunk_rows", [0, 1024, 320])
def test_rescale_contiguous(cuda, dtype, chunk_rows):
    cfg = MLAConfig.deepseek_v2()
    kv, qa, qr = staircase_case(B, S, dtype, 5, cuda)
    _, W_UV = make_weights(cfg, dtype, 6, cuda)
    cos, sin = rope(S, cfg, cuda)
    out = F.mla_decode_absorbed(kv, qa, qr, W_UV, cos, sin, cfg, chunk_rows=chunk_rows, kernel_variant=2)
    torch.cuda.synchronize()
    ref = oracle(kv, qa, qr, W_UV, cos, sin, [S] * B)
    assert_close(out.cpu().numpy(), ref, dtype, f"rescale contiguous {dtype} chunk {chunk_rows}")


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
@pytest.mark.parametrize("chunk_rows", [0, 1024])
def test_rescale_paged(cuda, dtype, chunk_rows):
    """Same inputs in a 64-row-block pool with device lengths (capacity 3072
    per sequence, 3000 filled)."""
    cfg = MLAConfig.deepseek_v2()
    cap = 3072
    kv, qa, qr = staircase_case(B, S, dtype, 5, cuda)
    full = torch.zeros(B, cap, 576, dtype=kv.dtype, device=cuda)
    full[:, :S] = kv
    pool, table = scatter(full, 64, 9)
    lens = torch.full((B,), S, dtype=torch.int32, device=cuda)
    _, W_UV = make_weights(cfg, dtype, 6, cuda)
    cos, sin = rope(cap, cfg, cuda)
    out = F.mla_decode_absorbed(pool, qa, qr, W_UV, cos, sin, cfg, seq_lens=lens, chunk_rows=chunk_rows,
                                kernel_variant=2, block_table=table, block_size=64)
    torch.cuda.synchronize()
    ref = oracle(kv, qa, qr, W_UV, cos, sin, [S] * B)
    assert_close(out.cpu().numpy(), ref, dtype, f"rescale paged {dtype} chunk {chunk_rows}")


@pytest.mark.parametrize("paged", [False, True])
def test_rescale_fp8_cache(cuda, paged):
    """The staircase in an FP8 E4M3 cache (the fp8 instantiations of the
    kernel: rows expanded to bf16 in LDS). The staircase columns are halved
    (48 x tier, exact in E4M3, whose largest value is 448) and the query
    weights on them doubled, so the scores climb exactly as in the 16-bit
    cases; the other values are the fp8 codes of the random part, and the
    oracle reads the same codes."""
    cfg = MLAConfig.deepseek_v2()
    kv16, qa, qr = staircase_case(B, S, "bf16", 5, cuda)
    kv8 = (kv16.float() * 0.5).to(torch.float8_e4m3fn)
    qa = qa.clone()
    qa[:, :, 0:2] *= 2.0
    kv_np = mo.fp8_e4m3_decode(kv8.view(torch.uint8).cpu().numpy())
    assert np.array_equal(kv_np[:, :, 0:2], to_np(kv16)[:, :, 0:2] * 0.5), "staircase columns exact in E4M3"
    _, W_UV = make_weights(cfg, "bf16", 6, cuda)
    if paged:
        cap, bs = 3072, 64
        bps = cap // bs
        full = torch.zeros(B, cap, 576, dtype=torch.uint8, device=cuda)
        full[:, :S] = kv8.view(torch.uint8)
        perm = torch.from_numpy(np.random.RandomState(9).permutation(B * bps).astype(np.int32)).to(cuda)
        pool = torch.empty(B * cap, 576, dtype=torch.float8_e4m3fn, device=cuda)
        pool.view(torch.uint8).view(B * bps, bs, 576)[perm.long()] = full.view(B * bps, bs, 576)
        table = perm.view(B, bps)
        lens = torch.full((B,), S, dtype=torch.int32, device=cuda)
        cos, sin = rope(cap, cfg, cuda)
        out = F.mla_decode_absorbed(pool, qa, qr, W_UV, cos, sin, cfg, seq_lens=lens, kernel_variant=2,
                                    block_table=table, block_size=bs)
    else:
        cos, sin = rope(S, cfg, cuda)
        out = F.mla_decode_absorbed(kv8, qa, qr, W_UV, cos, sin, cfg, kernel_variant=2)
    torch.cuda.synchronize()
    packed = np.concatenate([kv_np[b] for b in range(B)]).astype(np.float64)
    ref = mo.decode_sequences(packed, [b * S for b in range(B + 1)], to_np(qa), to_np(qr), to_np(W_UV),
                              to_np(cos)[:S], to_np(sin)[:S], D)
    assert_close(out.cpu().numpy(), ref, "bf16", f"rescale fp8 {'paged' if paged else 'contiguous'}")
