"""GPU parity of paged latent caches (block tables: la_decode_args /
la_append_args.block_table) against the same data laid out contiguously.

A paged cache holds each sequence's rows in fixed-size blocks of a shared
pool, listed per sequence in an int32 block table. The kernels read the same
rows in the same order either way, so decode over a pool whose blocks are
scattered by a random permutation must equal decode over the contiguous
capacity cache bit for bit. That equality is the check, at every block size
and kernel variant tested. One case is also compared with the oracle directly
(bf16 tolerance, tests/conftest.py:assert_close). Appends into a paged cache
must place rows exactly where the oracle's contiguous append puts them, read
back through the table. Unused pool blocks hold 1e4, so any read of a row
outside the sequences would show.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import assert_close
from mla_cases import make_queries, make_weights, rope, to_np
from oracle import mla_oracle as mo

from latent_attn import MLAConfig
from latent_attn import functional as F

pytestmark = pytest.mark.gpu

ROW = 576


def scatter(cache, bs, seed, spare=3):
    """Pool + table holding cache (B, cap, ROW) in permuted blocks, with
    `spare` extra blocks of 1e4 mixed in."""
    B, cap, _ = cache.shape
    bps = cap // bs
    nblk = B * bps + spare
    perm = torch.from_numpy(np.random.RandomState(seed).permutation(nblk)[:B * bps].astype(np.int32))
    pool = torch.full((nblk * bs, ROW), 1e4, dtype=cache.dtype, device=cache.device)
    table = perm.view(B, bps).to(cache.device)
    for b in range(B):
        for j in range(bps):
            blk = int(perm[b * bps + j])
            pool[blk * bs:(blk + 1) * bs] = cache[b, j * bs:(j + 1) * bs]
    return pool, table


def gather(pool, table, bs):
    """The contiguous (B, cap, ROW) view of a paged cache."""
    B, bps = table.shape
    rows = (table.long().unsqueeze(-1) * bs + torch.arange(bs, device=table.device)).reshape(B, bps * bs)
    return pool[rows]


# chunk_rows: multiples of 64 for the MFMA kernel (the launcher rounds a paged
# plan's chunks up to one, which would split the contiguous run differently)
# 96- and 160-row blocks hold 3 and 5 tiles: the MFMA kernel's divide by tiles per block
@pytest.mark.parametrize("bs,variant,chunk_rows,dtype", [(32, 0, 0, torch.bfloat16), (64, 0, 0, torch.bfloat16),
                                                         (64, 2, 128, torch.bfloat16), (256, 0, 192, torch.bfloat16),
                                                         (16, 0, 0, torch.bfloat16), (64, 1, 0, torch.bfloat16),
                                                         (32, 1, 100, torch.bfloat16), (64, 0, 0, torch.float16),
                                                         (48, 0, 0, torch.float16), (96, 0, 128, torch.bfloat16),
                                                         (160, 2, 128, torch.float16)])
def test_paged_decode_equals_contiguous(cuda, bs, variant, chunk_rows, dtype):
    cfg = MLAConfig.deepseek_v2()
    B, cap = 4, (1024 // bs) * bs  # whole blocks (1008 rows for 48-row blocks)
    lens0 = [cap, 1, 700, 0]
    g = torch.Generator().manual_seed(51)
    cache = torch.randn(B, cap, ROW, generator=g).to(dtype).to(cuda)
    pool, table = scatter(cache, bs, 52)
    lens = torch.tensor(lens0, dtype=torch.int32, device=cuda)
    W_UK, W_UV = make_weights(cfg, "bf16", 53, cuda)
    q_nope, q_rope = make_queries((B,), cfg, 54, cuda)
    cos, sin = rope(cap, cfg, cuda)
    # block sizes below a 32-row tile run on the VALU kernel: compare like with like
    var_c = 1 if bs % 32 else variant
    out_c = F.mla_decode(cache, q_nope, q_rope, W_UK, W_UV, cos, sin, cfg, seq_lens=lens, chunk_rows=chunk_rows,
                         kernel_variant=var_c)
    out_p = F.mla_decode(pool, q_nope, q_rope, W_UK, W_UV, cos, sin, cfg, seq_lens=lens, chunk_rows=chunk_rows,
                         kernel_variant=variant, block_table=table, block_size=bs)
    torch.cuda.synchronize()
    assert torch.equal(out_p, out_c), float((out_p - out_c).abs().max())
    if bs == 64 and variant == 0 and dtype == torch.bfloat16:
        d = mo.Dims(5120, 512, 128, 64, 128, 128)
        qa = mo.absorb_q(to_np(q_nope), to_np(W_UK), d)
        kv = to_np(cache)
        packed = np.concatenate([kv[b, :lens0[b]] for b in range(B)])
        offsets = np.concatenate([[0], np.cumsum(lens0)])
        ref = mo.decode_sequences(packed, offsets, qa, to_np(q_rope), to_np(W_UV), to_np(cos), to_np(sin), d)
        assert_close(out_p.cpu().numpy(), ref, "bf16", "paged decode")


def test_paged_mfma_needs_tile_sized_blocks(cuda):
    """block_size 16 has no MFMA kernel (tiles of 32 rows would straddle
    blocks): asking for it explicitly is refused, the default picks the VALU
    kernel (covered above)."""
    cfg = MLAConfig.deepseek_v2()
    cache = torch.zeros(1, 64, ROW, dtype=torch.bfloat16, device=cuda)
    pool, table = scatter(cache, 16, 1, spare=0)
    lens = torch.tensor([64], dtype=torch.int32, device=cuda)
    W_UK, W_UV = make_weights(cfg, "bf16", 2, cuda)
    q_nope, q_rope = make_queries((1,), cfg, 3, cuda)
    cos, sin = rope(64, cfg, cuda)
    with pytest.raises(RuntimeError, match="unsupported"):
        F.mla_decode(pool, q_nope, q_rope, W_UK, W_UV, cos, sin, cfg, seq_lens=lens, kernel_variant=2,
                     block_table=table, block_size=16)


@pytest.mark.parametrize("bs", [16, 64])
def test_paged_append_places_rows_through_the_table(cuda, bs):
    """Three steps of two tokens each into a paged cache: the rows read back
    through the table equal the oracle's contiguous append bit for bit,
    and blocks outside every table keep their 1e4."""
    cfg = MLAConfig.deepseek_v2()
    B, cap = 3, 128
    lens0 = [0, 63, 120]
    g = torch.Generator().manual_seed(61)
    cache = torch.randn(B, cap, ROW, generator=g).to(torch.bfloat16).to(cuda)
    pool, table = scatter(cache, bs, 62)
    used = set(table.flatten().tolist())
    lens = torch.tensor(lens0, dtype=torch.int32, device=cuda)
    kv_np = to_np(cache).reshape(B * cap, ROW)
    lens_np = np.array(lens0)
    status = torch.zeros(1, dtype=torch.int32, device=cuda)
    for step in range(3):
        gg = torch.Generator().manual_seed(70 + step)
        c_t = torch.randn(B, 2, 512, generator=gg)
        k_rope = torch.randn(B, 2, 64, generator=gg)
        F.append_kv(pool, lens, c_t.to(cuda), k_rope.to(cuda), cfg, status=status, block_table=table, block_size=bs)
        kv_np, lens_np, full = mo.append_rows(kv_np, [b * cap for b in range(B)], [cap] * B, lens_np, to_np(c_t),
                                              to_np(k_rope), "bf16")
    torch.cuda.synchronize()
    # sequence 2 (120 + 2*3 = 126 <= 128) fits; nothing was refused
    assert status.item() == 0 and not full
    assert lens.cpu().tolist() == list(lens_np)
    assert np.array_equal(to_np(gather(pool, table, bs)).reshape(B * cap, ROW), kv_np)
    spare = [b for b in range(pool.shape[0] // bs) if b not in used]
    for b in spare:
        assert torch.all(pool[b * bs:(b + 1) * bs] == 1e4)
