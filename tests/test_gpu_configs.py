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


def _plan_workspace(B, total, Hq, ncu, chunk_rows=0):
    """Workspace of the MFMA split plan (q_nope absorbed into 16-bit queries):
    about one workgroup per CU, chunks of at least ceil(Hq*512/576) rows
    rounded up to 64; slots = chunks + sequences - 1; regions 256-B aligned:
    [q_prep (B, Hq padded to 32, 576) 16-bit] [partials (slots*Hq, 512) fp16]
    [scales (2) and maxima (1) fp32 per partial row] [log-sum-exps fp32]."""
    def al(x):
        return (x + 255) // 256 * 256

    if chunk_rows:
        L = chunk_rows
    else:
        chunks = max(1, ncu // ((Hq + 127) // 128))
        L = -(-total // chunks)
        L = max(L, -(-(Hq * 512) // 576))
        L = max(-(-L // 64) * 64, 64)
    n = -(-total // L)
    slots = n + B - 1
    q_prep = al(B * (-(-Hq // 32) * 32) * 576 * 2)
    return q_prep + al(slots * Hq * 512 * 2) + al(slots * Hq * 3 * 4) + al(slots * Hq * 4), L, n


@pytest.mark.parametrize("name", ["cfg2", "cfg3", "cfg4", "cfg5"])
def test_mfma_plan_at_the_benchmark_configs(cuda, abi, name):
    """The split plan on the benchmark configurations, pinned by its workspace:
    one workgroup per CU where the rows allow (config 3: 256 chunks of 1,024
    rows, config 5: 256 of 2,048, config 4: 253 chunks over the ragged rows),
    and at B = 1 the 128-row floor that keeps the partial rows below the
    cache bytes (64 chunks)."""
    lib, capi = abi
    inp = bench.build_inputs(name, cuda)
    cfg = inp["cfg"]
    out = torch.empty(inp["B"], cfg.num_heads, cfg.v_head_dim, device=cuda)
    a = bench.decode_args(inp, out, capi)
    ncu = torch.cuda.get_device_properties(cuda).multi_processor_count
    want, L, n = _plan_workspace(inp["B"], int(inp["total"]), cfg.num_heads, ncu)
    got = lib.la_mla_decode_workspace_size(ctypes.byref(a))
    print(f"[plan {name}] {ncu} CUs: {n} chunks of {L} rows, workspace {got} B", flush=True)
    assert got == want
    if name in ("cfg3", "cfg5"):
        assert n == ncu


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
