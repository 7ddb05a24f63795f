"""GPU check of la_mla_decode_noalloc, the allocation-free variant of
la_mla_decode (static per-GPU device scratch instead of a workspace), called
through the C ABI (ctypes).

Two calls in a row, the second with a smaller input (fewer, ragged
sequences over a different cache, so it reuses the scratch the first call
left behind): each output must equal la_mla_decode's on the same arguments
with a caller workspace bit for bit (the same kernels on the same plan). A
step whose workspace exceeds the scratch is refused with
LA_ERROR_WORKSPACE before any device work.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from mla_cases import make_cache, make_queries, make_weights, rope

from latent_attn import MLAConfig, capi

pytestmark = pytest.mark.gpu


def _args(kv, offsets, seq_len, q_nope, q_rope, W_UK, W_UV, cos, sin, out, cfg):
    a = capi.DecodeArgs()
    a.kv_cache, a.kv_dtype, a.total_rows = kv.data_ptr(), capi.LA_DTYPE_BF16, kv.shape[0]
    a.num_seqs = q_nope.shape[0]
    if offsets is None:
        a.seq_len = seq_len
    else:
        a.seq_offsets = offsets.data_ptr()
    a.queries_per_seq = 1
    a.q_nope, a.W_UK, a.w_uk_dtype = q_nope.data_ptr(), W_UK.data_ptr(), capi.LA_DTYPE_BF16
    a.q_rope = q_rope.data_ptr()
    a.W_UV, a.w_uv_dtype = W_UV.data_ptr(), capi.LA_DTYPE_BF16
    a.rope_cos, a.rope_sin, a.rope_rows = cos.data_ptr(), sin.data_ptr(), cos.shape[0]
    a.output = out.data_ptr()
    a.cfg = capi.config(cfg)
    return a


def _both(lib, a, out, stream):
    """(la_mla_decode with a torch workspace, la_mla_decode_noalloc) outputs."""
    need = lib.la_mla_decode_workspace_size(ctypes.byref(a))
    assert 0 < need <= lib.la_mla_decode_noalloc_max_bytes()
    ws = torch.empty(need, dtype=torch.uint8, device=out.device)
    a.workspace, a.workspace_bytes = ws.data_ptr(), need
    assert lib.la_mla_decode(ctypes.byref(a), ctypes.c_void_p(stream)) == capi.LA_SUCCESS
    torch.cuda.synchronize()
    want = out.clone()
    out.fill_(float("nan"))
    a.workspace, a.workspace_bytes = None, 0
    st = lib.la_mla_decode_noalloc(ctypes.byref(a), ctypes.c_void_p(stream))
    assert st == capi.LA_SUCCESS, lib.la_status_string(st)
    torch.cuda.synchronize()
    return want, out.clone()


def test_noalloc_equals_workspace_decode_twice(cuda):
    lib = capi.load()
    cfg = MLAConfig.deepseek_v2()
    stream = torch.cuda.current_stream().cuda_stream
    W_UK, W_UV = make_weights(cfg, "bf16", 201, cuda)
    # call 1: 8 sequences x 2048 positions
    B, S = 8, 2048
    print(f"[noalloc] call 1: B={B} S={S}", flush=True)
    kv = make_cache((B * S,), cfg, "bf16", 202, cuda)
    q_nope, q_rope = make_queries((B,), cfg, 203, cuda)
    cos, sin = rope(S, cfg, cuda)
    out = torch.empty(B, 128, 128, device=cuda)
    want, got = _both(lib, _args(kv, None, S, q_nope, q_rope, W_UK, W_UV, cos, sin, out, cfg), out, stream)
    assert torch.isfinite(want).all()
    assert torch.equal(got, want), float((got - want).abs().max())
    # call 2, smaller: 3 ragged sequences (one empty) over another cache
    lens = [700, 0, 333]
    print(f"[noalloc] call 2: lens={lens}", flush=True)
    offsets = torch.tensor(np.concatenate([[0], np.cumsum(lens)]).astype(np.int32), device=cuda)
    kv2 = make_cache((sum(lens),), cfg, "bf16", 204, cuda)
    q_nope2, q_rope2 = make_queries((3,), cfg, 205, cuda)
    out2 = torch.empty(3, 128, 128, device=cuda)
    want2, got2 = _both(lib, _args(kv2, offsets, 0, q_nope2, q_rope2, W_UK, W_UV, cos, sin, out2, cfg), out2, stream)
    assert torch.equal(got2, want2), float((got2 - want2).abs().max())
    assert not want2[1].any()  # the empty sequence's heads are zero


def test_noalloc_refuses_a_step_beyond_its_scratch(cuda):
    """B=64 x 65536 positions x 8 queries needs more than the scratch: refused before any
    launch (the cache pointer is never read)."""
    lib = capi.load()
    cfg = MLAConfig.deepseek_v2()
    a = capi.DecodeArgs()
    fake = 0x10000
    a.kv_cache, a.kv_dtype, a.total_rows = fake, capi.LA_DTYPE_BF16, 64 * 65536
    a.num_seqs, a.seq_len, a.queries_per_seq = 64, 65536, 8
    a.q_nope, a.W_UK, a.w_uk_dtype = fake, fake, capi.LA_DTYPE_BF16
    a.q_rope, a.W_UV, a.w_uv_dtype = fake, fake, capi.LA_DTYPE_BF16
    a.rope_cos = a.rope_sin = fake
    a.output = fake
    a.cfg = capi.config(cfg)
    assert lib.la_mla_decode_workspace_size(ctypes.byref(a)) > lib.la_mla_decode_noalloc_max_bytes()
    assert lib.la_mla_decode_noalloc(ctypes.byref(a), None) == capi.LA_ERROR_WORKSPACE


def test_noalloc_under_hip_graph_capture(cuda):
    """la_mla_decode_noalloc captured into a HIP graph (torch.cuda.graph on a
    side stream) after one eager warm-up call (which looks up the scratch
    address and sets the kernels' attributes: the only non-stream HIP calls on
    the path). Every replay, with eager work and a synchronisation between
    replays (a la_mla_decode call with a caller workspace, and the output
    refilled with NaN), equals the eager la_mla_decode output bit for bit.
    Nothing on this path records a memset (the latent-half merge's output is
    zeroed by the absorb kernel)."""
    lib = capi.load()
    cfg = MLAConfig.deepseek_v2()
    stream = torch.cuda.current_stream().cuda_stream
    W_UK, W_UV = make_weights(cfg, "bf16", 211, cuda)
    B, S = 8, 2048
    kv = make_cache((B * S,), cfg, "bf16", 212, cuda)
    q_nope, q_rope = make_queries((B,), cfg, 213, cuda)
    cos, sin = rope(S, cfg, cuda)
    out = torch.empty(B, 128, 128, device=cuda)
    a = _args(kv, None, S, q_nope, q_rope, W_UK, W_UV, cos, sin, out, cfg)
    want, got = _both(lib, a, out, stream)  # eager reference and the warm-up noalloc call
    assert torch.equal(got, want)
    side = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    print("[noalloc] capturing into a HIP graph", flush=True)
    with torch.cuda.graph(g, stream=side):
        st = lib.la_mla_decode_noalloc(ctypes.byref(a), ctypes.c_void_p(side.cuda_stream))
    assert st == capi.LA_SUCCESS, lib.la_status_string(st)
    need = lib.la_mla_decode_workspace_size(ctypes.byref(a))
    ws = torch.empty(need, dtype=torch.uint8, device=cuda)
    other = torch.empty_like(out)
    b = _args(kv, None, S, q_nope, q_rope, W_UK, W_UV, cos, sin, other, cfg)
    b.workspace, b.workspace_bytes = ws.data_ptr(), need
    for r in range(4):
        out.fill_(float("nan"))
        assert lib.la_mla_decode(ctypes.byref(b), ctypes.c_void_p(stream)) == capi.LA_SUCCESS  # eager work
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        print(f"[noalloc] replay {r}", flush=True)
        assert torch.equal(out, want), (r, float((out - want).abs().max()))
        assert torch.equal(other, want)
