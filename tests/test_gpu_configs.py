"""GPU parity at the benchmark configurations' full sizes, called through the C ABI
(``la_mla_decode`` via ctypes, the same call bench.py times) on the inputs bench.py
builds (``bench.build_inputs``: seeded torch generator on the device).

The float64 oracle (absorb, then per-sequence latent attention, then W_UV) runs on
selected sequences at full length; properties that hold at any size cover the rest:

* config 2 (B=1, S=8192): the whole output; also naive decompress-then-attend
  (``tests/test_python.py:26-63`` of the reference) on the same inputs.
* config 3 (B=32, S=8192): 4 sequences against the oracle, and every sequence
  equals a B=1 call on its own cache (batch invariance, the reference's
  ``tests/test_batched.py:68-86`` invariant) within the 16-bit contract.
* config 4 (ragged, B=64, lengths RandomState(0).randint(512, 32769, 64)): the
  shortest, longest and 4 more sequences against the oracle; every sequence equals
  the per-sequence (uniform) call on its own rows.
* config 5 (B=4, S=131072): sequences 0 and 3 against the oracle at full length,
  and a 4096-position slice against the naive path.

Tolerance: bf16 inputs with fp32 accumulation, |d| <= 2e-2 + 1e-2 |ref| elementwise
and 1e-2 normwise (conftest.assert_close).
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

import bench
from conftest import assert_close
from mla_cases import to_np
from oracle import mla_oracle as mo

pytestmark = pytest.mark.gpu


def _dims(cfg) -> mo.Dims:
    return mo.Dims(cfg.d_model, cfg.kv_lora_rank, cfg.qk_nope_head_dim, cfg.qk_rope_head_dim, cfg.num_heads,
                   cfg.v_head_dim)


def _run(inp, lib, capi, variant: int = 0) -> np.ndarray:
    """One la_mla_decode call on the current stream; returns (B, H, dv) float64."""
    cfg = inp["cfg"]
    out = torch.full((inp["B"], cfg.num_heads, cfg.v_head_dim), float("nan"), device=inp["kv"].device)
    a = bench.decode_args(inp, out, capi)
    a.kernel_variant = variant
    ws_bytes = lib.la_mla_decode_workspace_size(ctypes.byref(a))
    assert ws_bytes > 0
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=inp["kv"].device)
    a.workspace = ws.data_ptr()
    a.workspace_bytes = ws_bytes
    st = lib.la_mla_decode(ctypes.byref(a), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert st == 0, lib.la_status_string(st).decode()
    torch.cuda.synchronize()
    return to_np(out)


def _seq_rows(inp, b: int):
    if inp["offsets"] is None:
        S = inp["seq_len"]
        return b * S, (b + 1) * S
    off = inp["offsets"].cpu().numpy()
    return int(off[b]), int(off[b + 1])


def _oracle_seq(inp, b: int, rows: int | None = None) -> np.ndarray:
    """float64 absorbed oracle for sequence b (its first ``rows`` positions)."""
    d = _dims(inp["cfg"])
    lo, hi = _seq_rows(inp, b)
    if rows is not None:
        hi = lo + rows
    kv = to_np(inp["kv"].view(-1, inp["kv"].shape[-1])[lo:hi])
    qa = mo.absorb_q(to_np(inp["q_nope"][b]), to_np(inp["W_UK"]), d)
    acc, _ = mo.absorbed_latent(kv, qa, to_np(inp["q_rope"][b]), to_np(inp["cos"]), to_np(inp["sin"]), d)
    return mo.project_wuv(acc, to_np(inp["W_UV"]), d)


def _single(inp, b: int, rows: int | None = None):
    """Inputs for sequence b alone (optionally its first ``rows`` positions), as a
    uniform B=1 problem over a copy of its rows."""
    lo, hi = _seq_rows(inp, b)
    if rows is not None:
        hi = lo + rows
    one = dict(inp)
    one.update(B=1, seq_len=hi - lo, total=hi - lo, offsets=None, kv=inp["kv"].view(-1, inp["kv"].shape[-1])[lo:hi]
               .contiguous(), q_nope=inp["q_nope"][b:b + 1].contiguous(), q_rope=inp["q_rope"][b:b + 1].contiguous())
    return one


@pytest.fixture(scope="module")
def abi():
    from latent_attn import capi

    return capi.load(), capi


def test_config2_single_sequence(cuda, abi):
    lib, capi = abi
    inp = bench.build_inputs("cfg2", cuda)
    out = _run(inp, lib, capi)
    print("[cfg2] B=1 S=8192 through la_mla_decode", flush=True)
    assert_close(out[0], _oracle_seq(inp, 0), "bf16", "cfg2 vs absorbed oracle")
    d = _dims(inp["cfg"])
    naive = mo.naive_mla(to_np(inp["kv"]), to_np(inp["W_UK"]), to_np(inp["W_UV"]), to_np(inp["q_nope"][0]),
                         to_np(inp["q_rope"][0]), to_np(inp["cos"]), to_np(inp["sin"]), d)
    assert_close(out[0], naive, "bf16", "cfg2 vs naive decompress-then-attend")


def test_config2_merge_halves_repeat_bitwise(cuda, abi):
    """At B = 1 the full-row merge would launch 128 workgroups for 256 CUs, so
    the launch merges each latent half in its own workgroup and both add into
    the output (zeroed by the absorb kernel) with float atomics. Two addends
    onto zero give fl(a + b) in either order: repeated calls are bitwise equal."""
    lib, capi = abi
    inp = bench.build_inputs("cfg2", cuda)
    out = torch.empty(1, inp["cfg"].num_heads, inp["cfg"].v_head_dim, device=cuda)
    info = capi.PlanInfo()
    assert lib.la_mla_decode_plan(ctypes.byref(bench.decode_args(inp, out, capi)), ctypes.byref(info)) == 0
    assert info.merge == capi.LA_PLAN_MERGE_MFMA_HALVES, info.merge  # the path this test is about
    outs = [_run(inp, lib, capi) for _ in range(4)]
    print("[cfg2] four calls, merge over latent halves", flush=True)
    for o in outs[1:]:
        assert np.array_equal(o, outs[0])
    assert_close(outs[0][0], _oracle_seq(inp, 0), "bf16", "cfg2 (latent-half merge) vs absorbed oracle")


def test_config2_plan_keeps_partials_below_cache(cuda, abi):
    """At B = 1 the MFMA split plan gives every chunk at least ceil(Hq*512/576)
    rows (128 at Hq = 128), so the fp16 partial rows it writes (Hq x 1 KB per
    chunk) stay below the chunk's cache bytes: the workspace (16-bit q_prep,
    partials, their scales, maxima and log-sum-exps) is bounded by the cache
    bytes plus q_prep plus 16 B per partial row. Cutting 8,192 rows into one
    chunk per CU (64 rows each) would need about twice the cache bytes."""
    lib, capi = abi
    inp = bench.build_inputs("cfg2", cuda)
    cfg = inp["cfg"]
    out = torch.empty(1, cfg.num_heads, cfg.v_head_dim, device=cuda)
    a = bench.decode_args(inp, out, capi)
    ws = lib.la_mla_decode_workspace_size(ctypes.byref(a))
    S, H = inp["seq_len"], cfg.num_heads
    cache_bytes = S * (cfg.kv_lora_rank + cfg.qk_rope_head_dim) * 2
    q_prep = 128 * 576 * 2
    chunks_max = S // 128                      # the plan's shortest chunk
    bound = q_prep + chunks_max * H * (cfg.kv_lora_rank * 2 + 16) + 4 * 256
    print(f"[cfg2 plan] workspace {ws} B, bound {bound} B, cache {cache_bytes} B", flush=True)
    assert 0 < ws <= bound
    assert ws - q_prep <= cache_bytes
    # the explicit 64-row override still works and needs the larger workspace
    a.chunk_rows = 64
    assert lib.la_mla_decode_workspace_size(ctypes.byref(a)) > cache_bytes


def _al(x):
    return (x + 255) // 256 * 256


def _mfma_workspace(B, Hq, slots):
    """Workspace of an MFMA plan whose queries become the attention kernel's
    16-bit rows: [q_prep (B, Hq padded to 32, 576) 16-bit] [partials
    (slots * Hq, 512) fp16] [2 scales + 1 maximum fp32 per partial row]
    [log-sum-exp fp32 per partial row], each region 256-B aligned."""
    return (_al(B * (-(-Hq // 32) * 32) * 576 * 2) + _al(slots * Hq * 512 * 2) + _al(slots * Hq * 3 * 4) +
            _al(slots * Hq * 4))


# Hand-computed plans on a 256-CU MI355X (one 128-head group per chunk unless
# noted): about one workgroup per CU, chunks rounded up to 64 rows and at
# least 128 rows for a 128-head group (its 128 fp16 partial rows, 128 KB,
# stay below the 16-bit cache bytes it streams, 114 rows); slots = chunks +
# sequences - 1; the latent-half merge when the full-row merge would have
# fewer than 256 workgroups (8 x ceil(128 / 8) x ceil(query rows / 16)).
#   name: (chunk_rows, num_chunks, num_slots, head_groups, merge)
_HALVES, _FULL = 3, 2
PLANS_256 = {
    # 8,192 rows / 256 = 32 -> 128-row floor: 64 chunks; 1 query row: 128 merge workgroups
    "cfg2": (128, 64, 64, 1, _HALVES),
    # 262,144 / 256 = 1,024; 32 rows -> 256 merge workgroups
    "cfg3": (1024, 256, 287, 1, _FULL),
    # 1,033,074 ragged rows / 256 = 4,035.4 -> 4,096: 253 chunks, + 63 slots; 64 rows -> 512
    "cfg4": (4096, 253, 316, 1, _FULL),
    # 524,288 / 256 = 2,048; 4 rows -> 128 merge workgroups
    "cfg5": (2048, 256, 259, 1, _HALVES),
}


@pytest.mark.parametrize("name", ["cfg2", "cfg3", "cfg4", "cfg5"])
def test_mfma_plan_at_the_benchmark_configs(cuda, abi, name):
    """The split plan on the benchmark configurations against hand-computed
    values (la_mla_decode_plan), and its workspace."""
    lib, capi = abi
    ncu = torch.cuda.get_device_properties(cuda).multi_processor_count
    if ncu != 256:
        pytest.skip(f"hand-computed plans assume 256 CUs, device has {ncu}")
    inp = bench.build_inputs(name, cuda)
    cfg = inp["cfg"]
    out = torch.empty(inp["B"], cfg.num_heads, cfg.v_head_dim, device=cuda)
    a = bench.decode_args(inp, out, capi)
    info = capi.PlanInfo()
    assert lib.la_mla_decode_plan(ctypes.byref(a), ctypes.byref(info)) == 0
    got = (info.chunk_rows, info.num_chunks, info.num_slots, info.head_groups, info.merge)
    print(f"[plan {name}] {got}, workspace {info.workspace_bytes} B", flush=True)
    assert info.attention == capi.LA_PLAN_ATTENTION_MFMA and info.absorb == capi.LA_PLAN_ABSORB_MFMA_QPREP
    assert got == PLANS_256[name]
    assert info.workspace_bytes == _mfma_workspace(inp["B"], cfg.num_heads, info.num_slots)
    assert info.workspace_bytes == lib.la_mla_decode_workspace_size(ctypes.byref(a))
    if name == "cfg2":
        # an FP8 cache: the floor counts rows, so the same chunks (its partials
        # may reach twice the fp8 cache bytes); and the explicit 64-row
        # override still works, with the larger workspace
        a.kv_dtype = capi.LA_DTYPE_FP8_E4M3
        assert lib.la_mla_decode_plan(ctypes.byref(a), ctypes.byref(info)) == 0
        assert (info.chunk_rows, info.num_chunks) == (128, 64)
        a.kv_dtype = capi.LA_DTYPE_BF16
        a.chunk_rows = 64
        assert lib.la_mla_decode_plan(ctypes.byref(a), ctypes.byref(info)) == 0
        assert (info.chunk_rows, info.num_chunks) == (64, 128)
        assert info.workspace_bytes > 8192 * 1152  # partials above the cache bytes


@pytest.mark.parametrize("batch,seq_len,want", [
    # the reference's batched entry (B queries over one shared cache, Hq = 128 B):
    # B = 16 at 2,048 rows: 16 head groups -> 256 / 16 = 16 chunks of 128 rows
    # (the 128-row floor of one group), 16 query rows -> 128 merge workgroups
    (16, 2048, (128, 16, 16, 16, _HALVES)),
    # B = 64 at 8,192 rows: 64 groups -> 4 chunks of 2,048 rows, 64 rows -> 512
    (64, 8192, (2048, 4, 4, 64, _FULL)),
    # B = 1 at 512 rows: 4 chunks of the 128-row floor
    (1, 512, (128, 4, 4, 1, _HALVES)),
])
def test_mfma_plan_for_the_shared_cache_entry(cuda, abi, batch, seq_len, want):
    """la_batched_fused_mla's plan: the row floor applies per 128-head group
    (each group's workgroup writes its own 128 partial rows), not to all
    128 B heads at once, which made 1,856-row chunks and 32 workgroups at
    B = 16."""
    lib, capi = abi
    ncu = torch.cuda.get_device_properties(cuda).multi_processor_count
    if ncu != 256:
        pytest.skip(f"hand-computed plans assume 256 CUs, device has {ncu}")
    a = capi.DecodeArgs()
    fake = 0x10000
    a.kv_cache, a.kv_dtype, a.total_rows, a.num_seqs, a.seq_len = fake, capi.LA_DTYPE_F16, seq_len, 1, seq_len
    a.queries_per_seq, a.q_absorbed, a.q_rope = batch, fake, fake
    a.W_UV, a.w_uv_dtype, a.rope_cos, a.rope_sin, a.rope_rows, a.output = fake, capi.LA_DTYPE_F16, fake, fake, 0, fake
    from latent_attn import MLAConfig
    a.cfg = capi.config(MLAConfig.deepseek_v2())
    info = capi.PlanInfo()
    assert lib.la_mla_decode_plan(ctypes.byref(a), ctypes.byref(info)) == 0
    got = (info.chunk_rows, info.num_chunks, info.num_slots, info.head_groups, info.merge)
    print(f"[plan shared B={batch} S={seq_len}] {got}", flush=True)
    assert info.attention == capi.LA_PLAN_ATTENTION_MFMA and info.absorb == capi.LA_PLAN_ABSORB_NONE
    assert got == want


@pytest.mark.parametrize("seq_len, mfma", [((1 << 30) - 32, True), ((1 << 30) + 32, False)])
def test_mfma_plan_needs_a_31_bit_uniform_row_space(cuda, abi, seq_len, mfma):
    """The MFMA kernels find a uniform sequence by a 32-bit division of the
    row index, so la_mla_decode keeps them to row spaces below 2^31 rows (two
    sequences of 2^30 - 32 rows: MFMA; of 2^30 + 32: not, the VALU kernel or
    LA_ERROR_NOT_SUPPORTED). The plan query touches no cache memory."""
    lib, capi = abi
    a = capi.DecodeArgs()
    fake = 0x10000
    a.kv_cache, a.kv_dtype, a.total_rows, a.num_seqs, a.seq_len = fake, capi.LA_DTYPE_BF16, 2 * seq_len, 2, seq_len
    a.queries_per_seq, a.q_absorbed, a.q_rope = 1, fake, fake
    a.W_UV, a.w_uv_dtype, a.rope_cos, a.rope_sin, a.rope_rows, a.output = fake, capi.LA_DTYPE_BF16, fake, fake, 8192, fake
    from latent_attn import MLAConfig
    a.cfg = capi.config(MLAConfig.deepseek_v2())
    info = capi.PlanInfo()
    st = lib.la_mla_decode_plan(ctypes.byref(a), ctypes.byref(info))
    print(f"[plan rows={2 * seq_len}] status {st} attention {info.attention}", flush=True)
    if mfma:
        assert st == 0 and info.attention == capi.LA_PLAN_ATTENTION_MFMA
    else:
        assert st == capi.LA_ERROR_NOT_SUPPORTED or (st == 0 and info.attention != capi.LA_PLAN_ATTENTION_MFMA)


def test_config3_batched_uniform(cuda, abi):
    lib, capi = abi
    inp = bench.build_inputs("cfg3", cuda)
    out = _run(inp, lib, capi)
    print("[cfg3] B=32 S=8192 through la_mla_decode", flush=True)
    assert np.isfinite(out).all()
    for b in (0, 9, 22, 31):
        assert_close(out[b], _oracle_seq(inp, b), "bf16", f"cfg3 seq {b} vs oracle")
    for b in range(inp["B"]):
        one = _run(_single(inp, b), lib, capi)
        assert_close(out[b], one[0], "bf16", f"cfg3 seq {b}: batched vs single call")


def test_config4_ragged(cuda, abi):
    lib, capi = abi
    inp = bench.build_inputs("cfg4", cuda)
    lens = np.asarray(inp["lens"])
    assert lens.min() >= 512 and lens.max() <= 32768 and len(lens) == 64
    out = _run(inp, lib, capi)
    print(f"[cfg4] ragged B=64 total={inp['total']} through la_mla_decode", flush=True)
    assert np.isfinite(out).all()
    picks = sorted({int(lens.argmin()), int(lens.argmax()), 0, 17, 40, 63})
    for b in picks:
        assert_close(out[b], _oracle_seq(inp, b), "bf16", f"cfg4 seq {b} (len {lens[b]}) vs oracle")
    for b in range(inp["B"]):
        one = _run(_single(inp, b), lib, capi)
        assert_close(out[b], one[0], "bf16", f"cfg4 seq {b}: ragged vs per-sequence call")


def test_config5_long_context(cuda, abi):
    lib, capi = abi
    inp = bench.build_inputs("cfg5", cuda)
    out = _run(inp, lib, capi)
    print("[cfg5] B=4 S=131072 through la_mla_decode", flush=True)
    assert np.isfinite(out).all()
    for b in (0, 3):
        assert_close(out[b], _oracle_seq(inp, b), "bf16", f"cfg5 seq {b} vs oracle (131072 positions)")
    # 4096-position slice of sequence 1 against the naive decompress-then-attend path
    d = _dims(inp["cfg"])
    sl = _single(inp, 1, rows=4096)
    o_sl = _run(sl, lib, capi)
    naive = mo.naive_mla(to_np(sl["kv"]), to_np(inp["W_UK"]), to_np(inp["W_UV"]), to_np(inp["q_nope"][1]),
                         to_np(inp["q_rope"][1]), to_np(inp["cos"][:4096]), to_np(inp["sin"][:4096]), d,
                         dtype=np.float32)
    assert_close(o_sl[0], naive, "bf16", "cfg5 4096-position slice vs fp32 naive")
