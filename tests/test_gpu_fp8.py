"""GPU parity of FP8 E4M3 latent caches (LA_DTYPE_FP8_E4M3, torch.float8_e4m3fn).

The cache values are exactly the fp8 codes' values (oracle fp8_e4m3_decode);
the VALU decode kernel (kernel_variant 1) and the naive path compute in fp32
from them and are held to the fp32 tolerance against the float64 oracle
(tests/conftest.py:assert_close). The default decode runs the MFMA kernel,
which copies the fp8 rows and expands each tile to bf16 in LDS (exactly:
every E4M3 value is a bf16 value), so it is held to the bf16 tolerance, and
must equal that kernel run on a bf16 copy of the cache bit for bit,
contiguous and paged. Appends are byte work: the stored codes must equal the
oracle's encoding (round to nearest even, saturating at +-448) exactly.
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
D = mo.Dims(5120, 512, 128, 64, 128, 128)


def fp8_cache(shape, seed, device):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g).to(torch.float8_e4m3fn).to(device)


def fp8_np(t):
    return mo.fp8_e4m3_decode(t.view(torch.uint8).cpu().numpy()).astype(np.float64)


@pytest.mark.parametrize("variant,tol", [(1, "f32"), (0, "bf16")])
@pytest.mark.parametrize("lens0", [[500, 1, 333], [64, 0, 7]])
def test_fp8_decode_matches_oracle(cuda, lens0, variant, tol):
    cfg = MLAConfig.deepseek_v2()
    B, cap = 3, 500
    kv = fp8_cache((B, cap, ROW), 81, cuda)
    lens = torch.tensor(lens0, dtype=torch.int32, device=cuda)
    W_UK, W_UV = make_weights(cfg, "bf16", 82, cuda)
    q_nope, q_rope = make_queries((B,), cfg, 83, cuda)
    cos, sin = rope(cap, cfg, cuda)
    out = F.mla_decode(kv, q_nope, q_rope, W_UK, W_UV, cos, sin, cfg, seq_lens=lens, kernel_variant=variant)
    torch.cuda.synchronize()
    kv_np = fp8_np(kv)
    packed = np.concatenate([kv_np[b, :lens0[b]] for b in range(B)])
    offsets = np.concatenate([[0], np.cumsum(lens0)])
    qa = mo.absorb_q(to_np(q_nope), to_np(W_UK), D)
    ref = mo.decode_sequences(packed, offsets, qa, to_np(q_rope), to_np(W_UV), to_np(cos), to_np(sin), D)
    assert_close(out.cpu().numpy(), ref, tol, f"fp8 decode {lens0} variant {variant}")


@pytest.mark.parametrize("paged", [False, True])
def test_fp8_mfma_decode_equals_bf16_mfma(cuda, paged):
    """The default fp8 decode (fp8 rows expanded to bf16 in LDS by the MFMA
    kernel) gives exactly what the MFMA kernel gives on a bf16 copy of the
    cache: the expansion is exact and the rest of the path is the same."""
    cfg = MLAConfig.deepseek_v2()
    B, cap, bs = 3, 512, 64
    kv = fp8_cache((B, cap, ROW), 111, cuda)
    lens = torch.tensor([512, 77, 300], dtype=torch.int32, device=cuda)
    W_UK, W_UV = make_weights(cfg, "bf16", 112, cuda)
    q_nope, q_rope = make_queries((B,), cfg, 113, cuda)
    cos, sin = rope(cap, cfg, cuda)
    kw = dict(seq_lens=lens, chunk_rows=128)
    want = F.mla_decode(kv.to(torch.bfloat16), q_nope, q_rope, W_UK, W_UV, cos, sin, cfg, kernel_variant=2, **kw)
    if paged:
        bps = cap // bs
        perm = torch.from_numpy(np.random.RandomState(114).permutation(B * bps).astype(np.int32)).to(cuda)
        pool = torch.empty(B * cap, ROW, dtype=torch.float8_e4m3fn, device=cuda)
        pool.view(torch.uint8).view(B * bps, bs, ROW)[perm.long()] = kv.view(torch.uint8).view(B * bps, bs, ROW)
        got = F.mla_decode(pool, q_nope, q_rope, W_UK, W_UV, cos, sin, cfg, block_table=perm.view(B, bps),
                           block_size=bs, **kw)
    else:
        got = F.mla_decode(kv, q_nope, q_rope, W_UK, W_UV, cos, sin, cfg, **kw)
    torch.cuda.synchronize()
    assert torch.equal(got, want), float((got - want).abs().max())


def test_fp8_naive_matches_oracle(cuda):
    cfg = MLAConfig.deepseek_v2()
    S = 300
    kv = fp8_cache((S, ROW), 91, cuda)
    W_UK, W_UV = make_weights(cfg, "bf16", 92, cuda)
    q_nope, q_rope = make_queries((), cfg, 93, cuda)
    cos, sin = rope(S, cfg, cuda)
    out = F.naive_mla(kv, W_UK, W_UV, q_nope, q_rope, cos, sin, cfg)
    torch.cuda.synchronize()
    ref = mo.naive_mla(fp8_np(kv), to_np(W_UK), to_np(W_UV), to_np(q_nope), to_np(q_rope), to_np(cos), to_np(sin), D)
    assert_close(out.cpu().numpy(), ref, "f32", "fp8 naive")


def test_fp8_append_encodes_like_the_oracle(cuda):
    """f32 rows (some beyond +-448, some at code midpoints) appended into an
    fp8 cache: stored codes equal the oracle's encoding byte for byte, and
    the paged form stores the same bytes through its table."""
    cfg = MLAConfig.deepseek_v2()
    B, cap, T = 2, 64, 3
    g = torch.Generator().manual_seed(101)
    c_t = torch.randn(B, T, 512, generator=g) * 40
    c_t[0, 0, :8] = torch.tensor([500.0, -1e6, 448.0, 464.0, 1.0625, 1.1875, 3 * 2.0 ** -10, 2.0 ** -10])
    k_rope = torch.randn(B, T, 64, generator=g)
    kv = torch.zeros(B, cap, ROW, dtype=torch.float8_e4m3fn, device=cuda)
    lens = torch.tensor([0, 10], dtype=torch.int32, device=cuda)
    F.append_kv(kv, lens, c_t.to(cuda), k_rope.to(cuda), cfg)
    # paged copy of the same empty cache: 2 blocks of 32 rows per sequence, reversed
    pool = torch.zeros(B * cap, ROW, dtype=torch.float8_e4m3fn, device=cuda)
    table = torch.tensor([[3, 2], [1, 0]], dtype=torch.int32, device=cuda)
    lens_p = torch.tensor([0, 10], dtype=torch.int32, device=cuda)
    F.append_kv(pool, lens_p, c_t.to(cuda), k_rope.to(cuda), cfg, block_table=table, block_size=32)
    torch.cuda.synchronize()
    codes = kv.view(torch.uint8).cpu().numpy()
    want = mo.fp8_e4m3_encode(torch.cat([c_t, k_rope], dim=-1).numpy())
    assert np.array_equal(codes[0, 0:T], want[0])
    assert np.array_equal(codes[1, 10:10 + T], want[1])
    assert codes[0, 0, :8].tolist() == [0x7E, 0xFE, 0x7E, 0x7E, 0x38, 0x3A, 0x02, 0x00]
    assert not codes[0, T:].any() and not codes[1, :10].any() and not codes[1, 10 + T:].any()
    p = pool.view(torch.uint8).cpu().numpy()
    assert np.array_equal(p[3 * 32:3 * 32 + T], want[0])          # sequence 0, block 0 -> pool block 3
    assert np.array_equal(p[1 * 32 + 10:1 * 32 + 10 + T], want[1])  # sequence 1, block 0 -> pool block 1
    assert lens.cpu().tolist() == [T, 10 + T] == lens_p.cpu().tolist()


@pytest.mark.parametrize("batched", [False, True])
def test_fp8_fused_entries_match_oracle(cuda, batched):
    """fused_mla_forward / batched_fused_mla_forward (the reference's
    bindings, csrc/bindings.cpp:126-244) over an fp8 cache with bf16 W_UV:
    the workspace they size for that dtype pair must be enough, and the
    result matches the oracle at the bf16 tolerance."""
    cfg = MLAConfig.deepseek_v2()
    S, B = 700, 3
    kv = fp8_cache((S, ROW), 121, cuda)
    _, W_UV = make_weights(cfg, "bf16", 122, cuda)
    g = torch.Generator().manual_seed(123)
    lead = (B,) if batched else ()
    qa = (torch.randn(*lead, 128, 512, generator=g) * 0.5).to(cuda)
    qr = torch.randn(*lead, 128, 64, generator=g).to(cuda)
    cos, sin = rope(S, cfg, cuda)
    fn = F.batched_fused_mla if batched else F.fused_mla
    out = fn(kv, qa, qr, W_UV, cos, sin, cfg)
    torch.cuda.synchronize()
    kv_np = fp8_np(kv)
    if batched:
        ref = mo.batched_absorbed_mla(kv_np, to_np(qa), to_np(qr), to_np(W_UV), to_np(cos), to_np(sin), D)
    else:
        ref = mo.absorbed_mla(kv_np, to_np(qa), to_np(qr), to_np(W_UV), to_np(cos), to_np(sin), D)
    assert_close(out.cpu().numpy(), ref, "bf16", f"fp8 fused batched={batched}")
