#!/usr/bin/env python3
"""Benchmark of the MLA decode hot path on one MI355X.

A step = one decode step of BASELINE.json's headline workload (config 3):
B=32 sequences x 8192 cached positions, H=128, d_c=512, d_R=64, bf16 latent
cache, fp32 accumulation, one query token per sequence:
    q_abs = q_nope . W_UK  ->  split-KV latent attention (MFMA kernel)
    ->  log-sum-exp combine + W_UV projection.
All inputs are resident in HBM before timing. The step is launched through the
C ABI (la_mla_decode) on one stream; HIP events bracket the K timed steps.
K further steps then time the attention kernel alone (an event pair recorded
around it by hipExtLaunchKernelGGL in each step) for the roofline line; those
events add dispatch gaps, so they stay out of the K timed steps.

Prints ONE JSON line. ``value`` is microseconds per decode step (lower is
better); ``latent_cache_GBps`` is the whole-step cache read rate; ``roofline``
is the attention kernel's algorithmic latent-cache bytes (1152 B per sequence
position, one pass) over its measured duration against 8 TB/s.
``append_kernel_us`` is one device-side cache append (la_append_kv: one new
bf16 row per sequence of the batch at its length, plus the query's RoPE),
averaged over back-to-back calls; it is not part of the decode step.
``cpu_baseline`` times this repo's CPU restatement of the reference path
(oracle/, numpy float32 absorbed math) on a bounded sample of the same
workload, extrapolated to one step.
"""

from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "latent-attn_amd"))
sys.path.insert(0, ROOT)

CONFIGS = {
    # name: (batch, seq_len or None for ragged, description)
    "cfg2": dict(batch=1, seq_len=8192, desc="DeepSeek-V2 single-sequence decode B=1 S=8192"),
    "cfg3": dict(batch=32, seq_len=8192, desc="batched uniform decode B=32 S=8192"),
    "cfg4": dict(batch=64, seq_len=None, desc="ragged decode B=64 len U[512,32768] seed 0"),
    "cfg5": dict(batch=4, seq_len=131072, desc="long-context decode B=4 S=131072"),
}
HBM_PEAK_GBPS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0
BYTES_PER_POS = 1152  # (512 + 64) * 2, one pass over the latent cache


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def hip_runtime():
    hip = ctypes.CDLL("libamdhip64.so.7")
    hip.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
    hip.hipEventCreateWithFlags.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_uint]
    hip.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    hip.hipEventSynchronize.argtypes = [ctypes.c_void_p]
    hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
    hip.hipEventDestroy.argtypes = [ctypes.c_void_p]
    return hip


# hipEventDisableSystemFence (hip_runtime_api.h): the event only records a timestamp, without
# the system-scope release (L2 write-back + invalidate) a default event performs; a default
# event pair around the attention kernel adds ~12 us of such fences to every step.
HIP_EVENT_DISABLE_SYSTEM_FENCE = 0x20000000


def new_event(hip, timing_only: bool = False):
    e = ctypes.c_void_p()
    if timing_only:
        assert hip.hipEventCreateWithFlags(ctypes.byref(e), HIP_EVENT_DISABLE_SYSTEM_FENCE) == 0
    else:
        assert hip.hipEventCreate(ctypes.byref(e)) == 0
    return e


def elapsed_ms(hip, a, b) -> float:
    t = ctypes.c_float()
    assert hip.hipEventElapsedTime(ctypes.byref(t), a, b) == 0
    return t.value


def build_inputs(cfg_name: str, device, seed: int = 0):
    import numpy as np
    import torch

    from latent_attn import MLAConfig, build_rope_tables

    spec = CONFIGS[cfg_name]
    cfg = MLAConfig.deepseek_v2()
    B = spec["batch"]
    g = torch.Generator(device=device).manual_seed(seed)
    row = cfg.kv_lora_rank + cfg.qk_rope_head_dim
    if spec["seq_len"] is None:
        lens = np.random.RandomState(seed).randint(512, 32769, B)
        offsets = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
        total = int(offsets[-1])
        max_len = int(lens.max())
    else:
        lens = np.full(B, spec["seq_len"])
        offsets = None
        total = B * spec["seq_len"]
        max_len = spec["seq_len"]
    kv = torch.randn(total, row, generator=g, device=device, dtype=torch.float32).to(torch.bfloat16)
    std = 1.0 / math.sqrt(cfg.kv_lora_rank)
    W_UK = (torch.randn(cfg.num_heads * cfg.qk_nope_head_dim, cfg.kv_lora_rank, generator=g, device=device) * std)
    W_UV = (torch.randn(cfg.num_heads * cfg.v_head_dim, cfg.kv_lora_rank, generator=g, device=device) * std)
    W_UK, W_UV = W_UK.to(torch.bfloat16), W_UV.to(torch.bfloat16)
    q_nope = torch.randn(B, cfg.num_heads, cfg.qk_nope_head_dim, generator=g, device=device)
    q_rope = torch.randn(B, cfg.num_heads, cfg.qk_rope_head_dim, generator=g, device=device)
    cos, sin = build_rope_tables(max_len, cfg.qk_rope_head_dim, device=device)
    off_t = torch.from_numpy(offsets).to(device) if offsets is not None else None
    return dict(cfg=cfg, B=B, lens=lens, total=total, kv=kv, W_UK=W_UK, W_UV=W_UV, q_nope=q_nope,
                q_rope=q_rope, cos=cos.contiguous(), sin=sin.contiguous(), offsets=off_t, max_len=max_len,
                seq_len=spec["seq_len"])


def decode_args(inp, out, capi):
    a = capi.DecodeArgs()
    a.kv_cache = inp["kv"].data_ptr()
    a.kv_dtype = capi.LA_DTYPE_BF16
    a.total_rows = inp["total"]
    a.num_seqs = inp["B"]
    if inp["offsets"] is None:
        a.seq_len = inp["seq_len"]
    else:
        a.seq_offsets = inp["offsets"].data_ptr()
    a.queries_per_seq = 1
    a.q_nope = inp["q_nope"].data_ptr()
    a.W_UK = inp["W_UK"].data_ptr()
    a.w_uk_dtype = capi.LA_DTYPE_BF16
    a.q_rope = inp["q_rope"].data_ptr()
    a.W_UV = inp["W_UV"].data_ptr()
    a.w_uv_dtype = capi.LA_DTYPE_BF16
    a.rope_cos = inp["cos"].data_ptr()
    a.rope_sin = inp["sin"].data_ptr()
    a.rope_rows = inp["cos"].shape[0]
    a.output = out.data_ptr()
    a.cfg = capi.config(inp["cfg"])
    return a


def decode_call(lib, a, stream, ev_b=None, ev_e=None, repeat: int = 0, what: str = "") -> None:
    """One decode step: la_mla_decode, or la_mla_decode_profiled when events
    bracket the attention kernel (launched `repeat` times back to back)."""
    if ev_b is None and ev_e is None and repeat <= 1:
        st = lib.la_mla_decode(ctypes.byref(a), ctypes.c_void_p(stream))
    else:
        st = lib.la_mla_decode_profiled(ctypes.byref(a), ctypes.c_void_p(stream), ev_b, ev_e, repeat)
    if st != 0:
        raise RuntimeError(f"la_mla_decode{what}: {lib.la_status_string(st).decode()} hip={lib.la_last_hip_error()}")


def time_append(lib, hip, capi, inp, stream, calls: int = 100) -> float:
    """Microseconds per la_append_kv call: one bf16 row per sequence of the
    batch appended at its length into a capacity cache (B, calls + 8, 576),
    with the query's q_rope rotated for that position; calls back to back
    on the GPU between one event pair (after 4 untimed calls)."""
    import torch

    cfg, B = inp["cfg"], inp["B"]
    dev = inp["kv"].device
    row = cfg.kv_lora_rank + cfg.qk_rope_head_dim
    cap = calls + 8
    kv = torch.zeros(B, cap, row, dtype=torch.bfloat16, device=dev)
    lens = torch.zeros(B, dtype=torch.int32, device=dev)
    g = torch.Generator(device=dev).manual_seed(1)
    c_t = torch.randn(B, 1, cfg.kv_lora_rank, generator=g, device=dev).to(torch.bfloat16)
    k_rope = torch.randn(B, 1, cfg.qk_rope_head_dim, generator=g, device=dev).to(torch.bfloat16)
    q = inp["q_rope"].clone()
    status = torch.zeros(1, dtype=torch.int32, device=dev)
    a = capi.AppendArgs()
    a.kv_cache, a.kv_dtype, a.total_rows = kv.data_ptr(), capi.LA_DTYPE_BF16, B * cap
    a.num_seqs, a.seq_capacity, a.seq_lens = B, cap, lens.data_ptr()
    a.tokens_per_seq, a.c_t, a.k_rope, a.src_dtype = 1, c_t.data_ptr(), k_rope.data_ptr(), capi.LA_DTYPE_BF16
    a.q_rope, a.queries_per_seq = q.data_ptr(), 1
    a.rope_cos, a.rope_sin, a.rope_rows = inp["cos"].data_ptr(), inp["sin"].data_ptr(), inp["cos"].shape[0]
    a.status, a.cfg = status.data_ptr(), capi.config(cfg)

    def call():
        st = lib.la_append_kv(ctypes.byref(a), ctypes.c_void_p(stream))
        if st != 0:
            raise RuntimeError(f"la_append_kv: {lib.la_status_string(st).decode()}")

    for _ in range(4):
        call()
    t0, t1 = new_event(hip), new_event(hip)
    torch.cuda.synchronize()
    # A short spin kernel holds the stream while the host enqueues the calls
    # (~10 us of host time each), so the event pair times the appends back to
    # back on the GPU rather than the host's launch rate.
    torch.cuda._sleep(4_000_000)
    hip.hipEventRecord(t0, ctypes.c_void_p(stream))
    for _ in range(calls):
        call()
    hip.hipEventRecord(t1, ctypes.c_void_p(stream))
    hip.hipEventSynchronize(t1)
    us = elapsed_ms(hip, t0, t1) * 1e3 / calls
    hip.hipEventDestroy(t0)
    hip.hipEventDestroy(t1)
    assert status.item() == 0 and int(lens[0].item()) == calls + 4, "append bench overflowed its cache"
    return us


def time_paged(lib, hip, capi, inp, out, ws, stream, bs: int = 64, steps: int = 100) -> dict:
    """The same decode step over a paged copy of the cache: every sequence's
    rows in blocks of `bs` rows scattered over a pool by a fixed permutation,
    read through a block table with device lengths (la_decode_args.block_table).
    Step time over `steps` steps (after 20 untimed steps and a 50-ms clock
    settle) and the attention kernel's time (10 x 10 back-to-back launches),
    as for the contiguous line."""
    import numpy as np
    import torch

    B, S = inp["B"], inp["seq_len"]
    dev = inp["kv"].device
    bps = S // bs
    perm = torch.from_numpy(np.random.RandomState(7).permutation(B * bps).astype(np.int32)).to(dev)
    pool = torch.empty_like(inp["kv"])
    pool.view(B * bps, bs, -1)[perm.long()] = inp["kv"].view(B * bps, bs, -1)
    table = perm.view(B, bps).contiguous()
    lens = torch.full((B,), S, dtype=torch.int32, device=dev)
    a = decode_args(inp, out, capi)
    a.kv_cache = pool.data_ptr()
    a.seq_len = 0
    a.seq_lens = lens.data_ptr()
    a.block_table, a.block_size, a.blocks_per_seq = table.data_ptr(), bs, bps
    need = lib.la_mla_decode_workspace_size(ctypes.byref(a))
    assert 0 < need <= ws.numel()
    a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel()

    def step(ev_b=None, ev_e=None, repeat=0):
        decode_call(lib, a, stream, ev_b, ev_e, repeat, " (paged)")

    for _ in range(20):
        step()
    settle_clocks(step, 50)
    t0, t1 = new_event(hip), new_event(hip)
    torch.cuda.synchronize()
    hip.hipEventRecord(t0, ctypes.c_void_p(stream))
    for _ in range(steps):
        step()
    hip.hipEventRecord(t1, ctypes.c_void_p(stream))
    hip.hipEventSynchronize(t1)
    us_step = elapsed_ms(hip, t0, t1) * 1e3 / steps
    evs = [(new_event(hip, True), new_event(hip, True)) for _ in range(10)]
    for b, e in evs:
        step(b, e, 10)
    torch.cuda.synchronize()
    kern = sorted(elapsed_ms(hip, b, e) / 10 for b, e in evs)
    for ev in (t0, t1, *[x for pair in evs for x in pair]):
        hip.hipEventDestroy(ev)
    kern_us = sum(kern) / len(kern) * 1e3
    return {"step_us": round(us_step, 2), "attn_kernel_us": round(kern_us, 2),
            "frac_of_8TBps": round(int(inp["total"]) * BYTES_PER_POS / (kern_us * 1e-6) / 1e9 / HBM_PEAK_GBPS, 4)}


def time_fp8(lib, hip, capi, inp, out, stream, steps: int = 100) -> dict:
    """The same decode step over an FP8 E4M3 copy of the cache (576 B per
    position, half the bytes; the MFMA kernel copies the fp8 rows and expands
    them to bf16 in LDS): microseconds per step over `steps` steps (after 20
    untimed steps and a 50-ms clock settle), the attention kernel's time (10 x 10 back-to-back launches), and the
    latent-cache rates against 8 TB/s at 576 B per position."""
    import torch

    kv8 = inp["kv"].to(torch.float8_e4m3fn)
    a = decode_args(inp, out, capi)
    a.kv_cache, a.kv_dtype = kv8.data_ptr(), capi.LA_DTYPE_FP8_E4M3
    need = lib.la_mla_decode_workspace_size(ctypes.byref(a))
    ws8 = torch.empty(need, dtype=torch.uint8, device=kv8.device)
    a.workspace, a.workspace_bytes = ws8.data_ptr(), need

    def step(ev_b=None, ev_e=None, repeat=0):
        decode_call(lib, a, stream, ev_b, ev_e, repeat, " (fp8)")

    for _ in range(20):
        step()
    settle_clocks(step, 50)
    t0, t1 = new_event(hip), new_event(hip)
    torch.cuda.synchronize()
    hip.hipEventRecord(t0, ctypes.c_void_p(stream))
    for _ in range(steps):
        step()
    hip.hipEventRecord(t1, ctypes.c_void_p(stream))
    hip.hipEventSynchronize(t1)
    us = elapsed_ms(hip, t0, t1) * 1e3 / steps
    hip.hipEventDestroy(t0)
    hip.hipEventDestroy(t1)

    kern = time_attention(hip, step)
    kern_us = sum(kern) / len(kern) * 1e3
    fp8_bytes = int(inp["total"]) * BYTES_PER_POS // 2
    return {"step_us": round(us, 2), "attn_kernel_us": round(kern_us, 2),
            "cache_frac_of_8TBps": round(fp8_bytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBPS, 4),
            "attn_frac_of_8TBps": round(fp8_bytes / (kern_us * 1e-6) / 1e9 / HBM_PEAK_GBPS, 4)}


def time_fp16(lib, hip, capi, inp, out, stream, steps: int = 100) -> dict:
    """The same decode step with the reference's contract dtype: an fp16 copy
    of the cache and fp16 W_UK / W_UV (the reference binding accepts float16
    only, csrc/bindings.cpp:28-33), timed like the fp8 leg."""
    import torch

    kv16 = inp["kv"].to(torch.float16)
    wuk16, wuv16 = inp["W_UK"].to(torch.float16), inp["W_UV"].to(torch.float16)
    a = decode_args(inp, out, capi)
    a.kv_cache, a.kv_dtype = kv16.data_ptr(), capi.LA_DTYPE_F16
    a.W_UK, a.w_uk_dtype = wuk16.data_ptr(), capi.LA_DTYPE_F16
    a.W_UV, a.w_uv_dtype = wuv16.data_ptr(), capi.LA_DTYPE_F16
    need = lib.la_mla_decode_workspace_size(ctypes.byref(a))
    ws16 = torch.empty(need, dtype=torch.uint8, device=kv16.device)
    a.workspace, a.workspace_bytes = ws16.data_ptr(), need

    def step(ev_b=None, ev_e=None, repeat=0):
        decode_call(lib, a, stream, ev_b, ev_e, repeat, " (fp16)")

    for _ in range(20):
        step()
    settle_clocks(step, 50)
    us = time_steps(hip, step, stream, steps) * 1e3
    kern = time_attention(hip, step)
    kern_us = sum(kern) / len(kern) * 1e3
    cache_bytes = int(inp["total"]) * BYTES_PER_POS
    return {"step_us": round(us, 2), "attn_kernel_us": round(kern_us, 2),
            "attn_frac_of_8TBps": round(cache_bytes / (kern_us * 1e-6) / 1e9 / HBM_PEAK_GBPS, 4)}


def reference_entry_legs(lib, capi, hip, dev, stream) -> dict:
    """The reference's own launch entry points over the reference's own
    benchmark matrix, fp16 cache and weights (its contract dtype), DeepSeek-V2
    dims (DeepSeek-V3 has the same attention shapes: only d_model differs),
    pre-absorbed fp32 queries:
      * la_fused_mla (launch_fused_mla): one query token at kv_len 512, 2048,
        8192 and 32768 (reference benchmarks/bench_latency.cu:252-271);
      * la_batched_fused_mla (launch_batched_fused_mla): B query tokens over
        one shared cache, B in {1, 4, 16, 64} x kv_len {2048, 8192}
        (reference benchmarks/bench_throughput.py:86-93).
    Each entry: microseconds per call (50 calls back to back on the GPU, a
    spin kernel holding the stream while the host enqueues them, after 10
    untimed calls), tokens/s, and the attention kernel's time (the same
    arguments through la_mla_decode_profiled, 10 x 10 back-to-back launches)
    with its fraction of 8 TB/s on the cache bytes read once (kv_len x 1152 B;
    a shared cache is read by every 128-head group, the extra reads hit L2)."""
    import torch

    from latent_attn import MLAConfig, build_rope_tables

    cfg = MLAConfig.deepseek_v2()
    row = cfg.kv_lora_rank + cfg.qk_rope_head_dim
    g = torch.Generator(device=dev).manual_seed(3)
    std = 1.0 / math.sqrt(cfg.kv_lora_rank)
    W_UV = (torch.randn(cfg.num_heads * cfg.v_head_dim, cfg.kv_lora_rank, generator=g, device=dev) * std).half()
    c_cfg = capi.config(cfg)

    def leg(entry: str, S: int, B: int) -> dict:
        kv = torch.randn(S, row, generator=g, device=dev).half()
        qa = torch.randn(B, cfg.num_heads, cfg.kv_lora_rank, generator=g, device=dev) * std
        qr = torch.randn(B, cfg.num_heads, cfg.qk_rope_head_dim, generator=g, device=dev)
        cos, sin = build_rope_tables(S, cfg.qk_rope_head_dim, device=dev)
        cos, sin = cos.contiguous(), sin.contiguous()
        out = torch.empty(B, cfg.num_heads, cfg.v_head_dim, device=dev)
        need = lib.la_fused_mla_workspace_size_dt(S, B, ctypes.byref(c_cfg), capi.LA_DTYPE_F16, capi.LA_DTYPE_F16)
        ws = torch.empty(max(need, 1), dtype=torch.uint8, device=dev)
        vp = ctypes.c_void_p

        def call():
            if entry == "la_fused_mla":
                st = lib.la_fused_mla(vp(kv.data_ptr()), capi.LA_DTYPE_F16, S, vp(qa.data_ptr()), vp(qr.data_ptr()),
                                      vp(W_UV.data_ptr()), capi.LA_DTYPE_F16, vp(cos.data_ptr()), vp(sin.data_ptr()),
                                      vp(out.data_ptr()), ctypes.byref(c_cfg), vp(ws.data_ptr()), need, vp(stream))
            else:
                st = lib.la_batched_fused_mla(vp(kv.data_ptr()), capi.LA_DTYPE_F16, S, B, vp(qa.data_ptr()),
                                              vp(qr.data_ptr()), vp(W_UV.data_ptr()), capi.LA_DTYPE_F16,
                                              vp(cos.data_ptr()), vp(sin.data_ptr()), vp(out.data_ptr()),
                                              ctypes.byref(c_cfg), vp(ws.data_ptr()), need, vp(stream))
            if st != 0:
                raise RuntimeError(f"{entry}: {lib.la_status_string(st).decode()}")

        for _ in range(10):
            call()
        t0, t1 = new_event(hip), new_event(hip)
        torch.cuda.synchronize()
        torch.cuda._sleep(8_000_000)
        hip.hipEventRecord(t0, ctypes.c_void_p(stream))
        for _ in range(50):
            call()
        hip.hipEventRecord(t1, ctypes.c_void_p(stream))
        hip.hipEventSynchronize(t1)
        us = elapsed_ms(hip, t0, t1) * 1e3 / 50
        hip.hipEventDestroy(t0)
        hip.hipEventDestroy(t1)
        # the same arguments as the entry point builds them (one shared cache,
        # B query tokens per sequence), for the attention kernel's own time
        a = capi.DecodeArgs()
        a.kv_cache, a.kv_dtype, a.total_rows = kv.data_ptr(), capi.LA_DTYPE_F16, S
        a.num_seqs, a.seq_len, a.queries_per_seq = 1, S, B
        a.q_absorbed, a.q_rope = qa.data_ptr(), qr.data_ptr()
        a.W_UV, a.w_uv_dtype = W_UV.data_ptr(), capi.LA_DTYPE_F16
        a.rope_cos, a.rope_sin, a.rope_rows = cos.data_ptr(), sin.data_ptr(), S
        a.output, a.cfg = out.data_ptr(), c_cfg
        a.workspace, a.workspace_bytes = ws.data_ptr(), need
        kern = time_attention(hip, lambda b=None, e=None, r=0: decode_call(lib, a, stream, b, e, r, f" ({entry})"))
        kern_us = sum(kern) / len(kern) * 1e3
        return {"kv_len": S, "batch": B, "us_per_call": round(us, 2), "tokens_per_s": round(B / (us * 1e-6), 1),
                "attn_kernel_us": round(kern_us, 2),
                "attn_frac_of_8TBps": round(S * BYTES_PER_POS / (kern_us * 1e-6) / 1e9 / HBM_PEAK_GBPS, 4)}

    res = {"dtype": "fp16 cache and weights, fp32 queries", "model": "DeepSeek-V2 dims (128 heads, 512 + 64)",
           "la_fused_mla": [leg("la_fused_mla", S, 1) for S in (512, 2048, 8192, 32768)],
           "la_batched_fused_mla": [leg("la_batched_fused_mla", S, B) for B in (1, 4, 16, 64) for S in (2048, 8192)]}
    torch.cuda.empty_cache()
    return res


def time_layer(hip, inp, stream, calls: int = 20) -> dict:
    """LatentAttentionLayer.forward_batch (DeepSeek-V2 dims, fp32 parameters
    as in the reference module) for one token per sequence over the
    workload's cache: microseconds per call over `calls` calls between one
    event pair, against the HBM time of its algorithmic bytes (fp32 weights
    W_Q_absorbed, W_Q_rope, W_O, fp16 W_UV, the latent cache)."""
    import torch

    from latent_attn import LatentAttentionLayer

    cfg, B = inp["cfg"], inp["B"]
    dev = inp["kv"].device
    torch.manual_seed(0)
    layer = LatentAttentionLayer(cfg, max_seq_len=inp["max_len"]).to(dev)
    x = torch.randn(B, cfg.d_model, device=dev)
    kv = inp["kv"] if inp["offsets"] is not None else inp["kv"].view(B, inp["seq_len"], -1)
    run = lambda: layer.forward_batch(x, kv, seq_offsets=inp["offsets"])
    for _ in range(3):
        run()
    t0, t1 = new_event(hip), new_event(hip)
    torch.cuda.synchronize()
    hip.hipEventRecord(t0, ctypes.c_void_p(stream))
    for _ in range(calls):
        run()
    hip.hipEventRecord(t1, ctypes.c_void_p(stream))
    hip.hipEventSynchronize(t1)
    us = elapsed_ms(hip, t0, t1) * 1e3 / calls
    hip.hipEventDestroy(t0)
    hip.hipEventDestroy(t1)
    wbytes = 4 * (layer.W_Q_absorbed.numel() + layer.W_Q_rope.numel() + layer.W_O.numel()) + 2 * layer.W_UV.numel()
    total = wbytes + int(inp["total"]) * BYTES_PER_POS
    return {"us": round(us, 1), "algorithmic_bytes": total, "hbm_frac": round(total / (us * 1e-6) / 1e9 / HBM_PEAK_GBPS, 4)}


def measured_traffic(config: str):
    """HBM bytes per attention-kernel launch measured with rocprofv3
    (FETCH_SIZE + WRITE_SIZE, scaled by a copy of known size), read from the
    committed profile summary for this workload; None if there is none."""
    path = os.path.join(ROOT, "profiles", f"decode_mfma_{config}_traffic.json")
    try:
        with open(path) as f:
            return json.load(f)["hbm_bytes_per_launch"]
    except (OSError, KeyError, ValueError):
        return None


def host_info() -> dict:
    """The host's logical CPU count, CPU model and numpy's thread-pool size."""
    try:
        from threadpoolctl import threadpool_info

        threads = max([i.get("num_threads", 1) for i in threadpool_info()] or [1])
    except Exception:  # pragma: no cover
        threads = os.cpu_count() or 1
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                if ln.startswith("model name"):
                    model = ln.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"os_cpu_count": os.cpu_count(), "cpu_model": model, "numpy_threads": int(threads)}


def cpu_time_path(inp, kind: str, budget_s: float, max_pos: int = 0):
    """Seconds of the oracle's float32 `kind` path ("naive": the reference's
    PyTorch decompress-then-attend math, tests/test_python.py:26-63, oracle
    naive_mla; "absorbed": the reference kernel's algorithm,
    src/fused_mla.cu:218-267, oracle absorb_q + absorbed_latent +
    project_wuv) on the workload's sequences one at a time until budget_s,
    each cut to its first max_pos positions when max_pos > 0. Returns
    (seconds, sequences, positions)."""
    import numpy as np

    from oracle import mla_oracle as mo

    cfg = inp["cfg"]
    d = mo.Dims(cfg.d_model, cfg.kv_lora_rank, cfg.qk_nope_head_dim, cfg.qk_rope_head_dim, cfg.num_heads,
                cfg.v_head_dim)
    W_UK = inp["W_UK"].float().cpu().numpy()
    W_UV = inp["W_UV"].float().cpu().numpy()
    cos = inp["cos"].cpu().numpy()
    sin = inp["sin"].cpu().numpy()
    lens = [int(x) for x in inp["lens"]]
    offs = np.concatenate([[0], np.cumsum(lens)])
    done_pos, done_seq, spent = 0, 0, 0.0
    while spent < budget_s and done_seq < inp["B"]:
        b = done_seq
        n = lens[b] if max_pos <= 0 else min(lens[b], max_pos)
        kv = inp["kv"][offs[b]:offs[b] + n].float().cpu().numpy()
        qn = inp["q_nope"][b].cpu().numpy()
        qr = inp["q_rope"][b].cpu().numpy()
        t0 = time.perf_counter()
        if kind == "naive":
            mo.naive_mla(kv, W_UK, W_UV, qn, qr, cos, sin, d, dtype=np.float32)
        else:
            qa = mo.absorb_q(qn, W_UK, d, dtype=np.float32)
            acc, _ = mo.absorbed_latent(kv, qa, qr, cos, sin, d, dtype=np.float32)
            mo.project_wuv(acc, W_UV, d, dtype=np.float32)
        spent += time.perf_counter() - t0
        done_pos += n
        done_seq += 1
    return spent, done_seq, done_pos


def cpu_baseline(inp, budget_s: float = 10.0):
    """CPU baseline on the box's host cores: the oracle's float32 naive and
    absorbed paths (cpu_time_path) on whole sequences of the workload until
    ~budget_s each, extrapolated by positions to one step (all B sequences)."""
    total_pos = int(sum(int(x) for x in inp["lens"]))
    host = host_info()
    n_s, n_seq, n_pos = cpu_time_path(inp, "naive", budget_s)
    a_s, a_seq, a_pos = cpu_time_path(inp, "absorbed", budget_s)
    return {
        "value": round(n_s / n_pos * total_pos * 1e6, 1),
        "unit": "us/step",
        "cores": host["numpy_threads"],
        "kind": "port",
        "sample": f"{n_seq} of {inp['B']} sequences ({n_pos} positions) through oracle/mla_oracle.py naive_mla "
                  f"(the reference's PyTorch decompress-then-attend math) in float32, extrapolated by positions",
        "host": host,
        "absorbed": {"value": round(a_s / a_pos * total_pos * 1e6, 1), "unit": "us/step",
                     "sample": f"{a_seq} of {inp['B']} sequences ({a_pos} positions) through the absorbed "
                               f"float32 path (absorb_q, absorbed_latent, project_wuv)"},
    }


def cpu_baseline_configs(dev, budget_s: float = 4.0) -> dict:
    """The CPU paths on the other configurations (same seeded inputs as their
    GPU legs, same host threads): the absorbed float32 path on configs 2, 4
    and 5, the naive float32 path on config 2 and on the first 4,096
    positions of config 5's first sequence, each extrapolated by positions to
    one step of its configuration."""
    import torch

    res = {}
    for name, kinds in (("cfg2", ("absorbed", "naive")), ("cfg4", ("absorbed",)), ("cfg5", ("absorbed", "naive"))):
        inp = build_inputs(name, dev)
        total_pos = int(sum(int(x) for x in inp["lens"]))
        leg = {}
        for kind in kinds:
            cut = 4096 if (name == "cfg5" and kind == "naive") else 0
            sec, nseq, npos = cpu_time_path(inp, kind, budget_s, cut)
            key = kind if not cut else "naive_slice_4096"
            leg[key] = {"us_per_step": round(sec / npos * total_pos * 1e6, 1),
                        "sample": f"{nseq} sequence(s), {npos} positions" + (
                            f" (the first {cut} of a {int(inp['lens'][0])}-position sequence)" if cut else "")}
        res[name] = leg
        del inp
        torch.cuda.empty_cache()
    return res


class Stepper:
    """One decode step of a workload through la_mla_decode on `stream`, with
    the workspace sized by la_mla_decode_workspace_size."""

    def __init__(self, lib, capi, inp, stream, variant: int = 0):
        import torch

        self.lib, self.stream = lib, stream
        cfg = inp["cfg"]
        self.out = torch.empty(inp["B"], cfg.num_heads, cfg.v_head_dim, device=inp["kv"].device, dtype=torch.float32)
        self.a = decode_args(inp, self.out, capi)
        self.a.kernel_variant = variant
        need = lib.la_mla_decode_workspace_size(ctypes.byref(self.a))
        assert need > 0
        self.ws = torch.empty(need, dtype=torch.uint8, device=inp["kv"].device)
        self.a.workspace, self.a.workspace_bytes = self.ws.data_ptr(), need

    def __call__(self, ev_b=None, ev_e=None, repeat=0):
        decode_call(self.lib, self.a, self.stream, ev_b, ev_e, repeat)


def settle_clocks(step, min_ms: float) -> dict:
    """Clock-settle phase, separate from --warmup: steps in batches of 20
    until at least min_ms of wall time has passed with the GPU busy. The
    MI355X's clocks take ~100 steps of this load to reach their loaded
    steady state; timing before that reads up to ~20 % slow."""
    import torch

    n, t0 = 0, time.perf_counter()
    while (time.perf_counter() - t0) * 1e3 < min_ms:
        for _ in range(20):
            step()
        torch.cuda.synchronize()
        n += 20
    return {"steps": n, "ms": round((time.perf_counter() - t0) * 1e3, 1)}


def time_steps(hip, step, stream, K: int) -> float:
    """Milliseconds per step over K back-to-back steps between one event pair."""
    import torch

    t0, t1 = new_event(hip), new_event(hip)
    torch.cuda.synchronize()
    hip.hipEventRecord(t0, ctypes.c_void_p(stream))
    for _ in range(K):
        step()
    hip.hipEventRecord(t1, ctypes.c_void_p(stream))
    hip.hipEventSynchronize(t1)
    ms = elapsed_ms(hip, t0, t1) / K
    hip.hipEventDestroy(t0)
    hip.hipEventDestroy(t1)
    return ms


def time_attention(hip, step, calls: int = 10, repeat: int = 10) -> list:
    """Attention-kernel milliseconds per launch: `calls` steps, each running
    the attention kernel `repeat` times back to back (la_mla_decode_profiled) between
    one fence-free event pair on the launch stream. An event pair around a
    single launch also times its dispatch (~5 us; in a step that dispatch
    overlaps the previous kernel), while back-to-back launches overlap their
    dispatches like the kernels of a step do, so the per-launch time agrees
    with the profiler's kernel duration."""
    import torch

    evs = [(new_event(hip, True), new_event(hip, True)) for _ in range(calls)]
    for b, e in evs:
        step(b, e, repeat)
    torch.cuda.synchronize()
    ms = sorted(elapsed_ms(hip, b, e) / repeat for b, e in evs)
    for b, e in evs:
        hip.hipEventDestroy(b)
        hip.hipEventDestroy(e)
    return ms


def time_ceiling(lib, hip, a, stream, cache_bytes: int, calls: int = 10, repeat: int = 10) -> dict:
    """Streaming ceiling of the attention kernel's copy schedule
    (la_stream_ceiling): its grid and every wave's HBM->LDS copies per tile,
    no compute, into a ring of 3 tile buffers (the kernel's: one tile in
    flight at its end-of-iteration wait) or 4 (the deepest 160 KB of LDS
    holds). Microseconds per launch over `calls` x `repeat` back-to-back
    launches between fence-free event pairs, and the cache rate."""
    import torch

    res = {}
    for ring in (3, 4):
        for _ in range(3):
            st = lib.la_stream_ceiling(ctypes.byref(a), ring, ctypes.c_void_p(stream), None, None, 1)
            if st != 0:
                raise RuntimeError(f"la_stream_ceiling: {lib.la_status_string(st).decode()}")
        evs = [(new_event(hip, True), new_event(hip, True)) for _ in range(calls)]
        for b, e in evs:
            assert lib.la_stream_ceiling(ctypes.byref(a), ring, ctypes.c_void_p(stream), b, e, repeat) == 0
        torch.cuda.synchronize()
        us = sum(elapsed_ms(hip, b, e) / repeat for b, e in evs) / calls * 1e3
        for b, e in evs:
            hip.hipEventDestroy(b)
            hip.hipEventDestroy(e)
        gbps = cache_bytes / (us * 1e-6) / 1e9
        res[f"ring{ring}"] = {"us": round(us, 2), "cache_GBps": round(gbps, 1),
                              "frac_of_8TBps": round(gbps / HBM_PEAK_GBPS, 4)}
    return res


def time_mall_cold(hip, step, stream, dev, steps: int = 30, flush_mib: int = 1024) -> dict:
    """Per-step times with one fence-free event pair around each step, once
    with a device copy of flush_mib MiB between steps (it sweeps the 256 MB
    infinity cache and every L2, so weights, queries, tables and the cache all
    come from HBM: MALL-cold) and once back to back with the same events
    (steady state). Both include the event pair's dispatch gap, so compare
    them with each other, not with `value`."""
    import torch

    src = torch.empty(flush_mib << 20, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    res = {}
    for cold in (True, False):
        evs = [(new_event(hip, True), new_event(hip, True)) for _ in range(steps)]
        for b, e in evs:
            if cold:
                dst.copy_(src)
            hip.hipEventRecord(b, ctypes.c_void_p(stream))
            step()
            hip.hipEventRecord(e, ctypes.c_void_p(stream))
        torch.cuda.synchronize()
        us = [elapsed_ms(hip, b, e) * 1e3 for b, e in evs]
        for b, e in evs:
            hip.hipEventDestroy(b)
            hip.hipEventDestroy(e)
        us.sort()
        n = len(us)
        res["cold" if cold else "warm"] = {"mean_us": round(sum(us) / n, 2), "median_us": round(us[n // 2], 2),
                                           "p10_us": round(us[n // 10], 2), "p90_us": round(us[(9 * n) // 10], 2)}
    del src, dst
    return {"flush_mib": flush_mib, "steps": steps, **res}


def step_bytes(inp, ws_bytes: int, ms_step: float) -> dict:
    """Algorithmic HBM bytes of one step beside the latent cache (the
    secondary total): both weight matrices, queries in and outputs out, the
    RoPE table rows the longest sequence reads, and the workspace's query and
    partial regions (the partials written once by the attention kernel and read
    once by the merge, the 16-bit queries written by the absorb kernel and read
    by the attention kernel)."""
    cfg = inp["cfg"]
    B, H = inp["B"], cfg.num_heads
    lens = inp["lens"]
    b = {
        "cache": int(inp["total"]) * BYTES_PER_POS,
        "weights": 2 * H * cfg.kv_lora_rank * (cfg.qk_nope_head_dim + cfg.v_head_dim),
        "queries_and_output": 4 * B * H * (cfg.qk_nope_head_dim + cfg.qk_rope_head_dim + cfg.v_head_dim),
        "rope_tables": 2 * 4 * int(max(lens)) * (cfg.qk_rope_head_dim // 2),
        "workspace_written_and_read": 2 * int(ws_bytes),
    }
    b["total"] = sum(b.values())
    b["total_GBps"] = round(b["total"] / (ms_step * 1e-3) / 1e9, 1)
    return b


def config_leg(lib, capi, hip, name: str, dev, stream, steps: int = 50) -> dict:
    """One configuration besides the headline one: microseconds per step,
    tokens/s, the whole-step latent-cache rate, and the attention kernel's
    time and fraction of 8 TB/s on its algorithmic cache bytes."""
    import torch

    inp = build_inputs(name, dev)
    step = Stepper(lib, capi, inp, stream)
    settle_clocks(step, 30)
    ms = time_steps(hip, step, stream, steps)
    kern = time_attention(hip, step)
    kern_ms = sum(kern) / len(kern)
    cache_bytes = int(inp["total"]) * BYTES_PER_POS
    leg = {
        "workload": CONFIGS[name]["desc"],
        "total_positions": int(inp["total"]),
        "step_us": round(ms * 1e3, 2),
        "tokens_per_s": round(inp["B"] / (ms * 1e-3), 1),
        "latent_cache_GBps": round(cache_bytes / (ms * 1e-3) / 1e9, 1),
        "attn_kernel_us": round(kern_ms * 1e3, 2),
        "attn_frac_of_8TBps": round(cache_bytes / (kern_ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4),
    }
    del step, inp
    torch.cuda.empty_cache()
    return leg


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=200)
    # Declared separately from --warmup: steps run for at least this long
    # before the timed region so the GPU clocks reach their loaded state.
    ap.add_argument("--settle-ms", type=float, default=200.0)
    ap.add_argument("--config", default="cfg3", choices=sorted(CONFIGS))
    ap.add_argument("--legs", default="cfg2,cfg4,cfg5",
                    help="comma-separated other configurations timed after the headline one ('' for none)")
    ap.add_argument("--no-mall-cold", action="store_true")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-fp8", action="store_true",
                    help="skip the leg over an FP8 E4M3 copy of the cache")
    ap.add_argument("--no-fp16", action="store_true",
                    help="skip the leg over an fp16 copy of the cache and weights (the reference's dtype)")
    ap.add_argument("--no-reference-legs", action="store_true",
                    help="skip la_fused_mla / la_batched_fused_mla over the reference's benchmark matrix")
    ap.add_argument("--layer", action="store_true",
                    help="also time LatentAttentionLayer.forward_batch (fp32 projections, 1.8 GB of weights) "
                         "on the same batch and cache")
    ap.add_argument("--variant", type=int, default=0, help="0 auto, 1 VALU kernel, 2 MFMA kernel")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="only run 3 device-to-device copies of MIB MiB (the known-size kernel that scales "
                         "rocprofv3 FETCH_SIZE / WRITE_SIZE into bytes) and exit")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); this build runs on a single MI355X "
              "and has no multi-GPU path.", file=sys.stderr)
        sys.exit(2)

    import torch

    from latent_attn import capi

    device = torch.device("cuda:0")
    if args.calibrate_copy > 0:
        n = args.calibrate_copy << 20
        src = torch.ones(n, dtype=torch.uint8, device=device)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"calibrate_copy_bytes_read": n, "bytes_written": n, "launches": 3}), flush=True)
        return
    lib = capi.load()
    hip = hip_runtime()
    log(f"[bench] building inputs for {args.config}")
    inp = build_inputs(args.config, device)
    cfg = inp["cfg"]
    B = inp["B"]
    stream = torch.cuda.current_stream().cuda_stream
    step = Stepper(lib, capi, inp, stream, args.variant)
    torch.cuda.synchronize()

    log(f"[bench] warmup {args.warmup}")
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    log(f"[bench] clock settle {args.settle_ms} ms")
    settle = settle_clocks(step, args.settle_ms)

    K = args.steps
    log(f"[bench] timing {K} steps")
    ms_step = time_steps(hip, step, stream, K)
    log("[bench] timing the attention kernel: 10 x 10 launches")
    kern_ms = time_attention(hip, step)
    kern_avg = sum(kern_ms) / len(kern_ms)
    us_step = ms_step * 1e3
    log("[bench] streaming ceiling of the copy schedule")
    ceiling = time_ceiling(lib, hip, step.a, stream, int(inp["total"]) * BYTES_PER_POS) if inp["offsets"] is None else None
    log("[bench] append / paged legs")
    append_us = time_append(lib, hip, capi, inp, stream)
    paged = time_paged(lib, hip, capi, inp, step.out, step.ws, stream) if inp["offsets"] is None else None
    layer = time_layer(hip, inp, stream) if args.layer else None
    fp8 = time_fp8(lib, hip, capi, inp, step.out, stream) if not args.no_fp8 and inp["offsets"] is None else None
    fp16 = time_fp16(lib, hip, capi, inp, step.out, stream) if not args.no_fp16 else None
    mall = None
    if not args.no_mall_cold:
        log("[bench] MALL-cold leg")
        mall = time_mall_cold(hip, step, stream, device)

    total_pos = int(inp["total"])
    cache_bytes = total_pos * BYTES_PER_POS
    flops_attn = total_pos * 2 * cfg.num_heads * (cfg.kv_lora_rank + cfg.qk_rope_head_dim + cfg.kv_lora_rank)
    achieved_gbps = cache_bytes / (kern_avg * 1e-3) / 1e9
    line = {
        "metric": "µs/decode step + achieved latent-cache HBM GB/s, H=128 d_c=512, B=32 seq=8K",
        "value": round(us_step, 2),
        "unit": "us/step",
        "n_gpus": 1,
        "steps": K,
        "warmup": args.warmup,
        "clock_settle": settle,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": CONFIGS[args.config]["desc"],
            "batch": B,
            "seq_len": inp["seq_len"] if inp["seq_len"] else "ragged",
            "total_positions": total_pos,
            "num_heads": cfg.num_heads,
            "kv_lora_rank": cfg.kv_lora_rank,
            "qk_rope_head_dim": cfg.qk_rope_head_dim,
            "cache_dtype": "bf16",
            "accumulate": "fp32",
            "kernel_variant": args.variant,
        },
        "tokens_per_s": round(B / (ms_step * 1e-3), 1),
        "latent_cache_GBps": round(cache_bytes / (ms_step * 1e-3) / 1e9, 1),
        "step_bytes": step_bytes(inp, step.ws.numel(), ms_step),
        "attn_kernel_us": round(kern_avg * 1e3, 2),
        "attn_kernel_us_min_max": [round(kern_ms[0] * 1e3, 2), round(kern_ms[-1] * 1e3, 2)],
        "mfma_frac_of_bf16_peak": round(flops_attn / (kern_avg * 1e-3) / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4),
        "append_kernel_us": round(append_us, 2),
        **({"paged_block64": paged} if paged else {}),
        **({"mall_cold": mall} if mall else {}),
        **({"layer_forward_batch": layer} if layer else {}),
        **({"fp8_cache": fp8} if fp8 else {}),
        **({"fp16_cache": fp16} if fp16 else {}),
        **({"stream_ceiling": ceiling} if ceiling else {}),
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved_gbps, 1),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(achieved_gbps / HBM_PEAK_GBPS, 4),
            "traffic": measured_traffic(args.config),
        },
    }
    legs = [c for c in args.legs.split(",") if c and c != args.config]
    if legs:
        del step, inp
        torch.cuda.empty_cache()
        line["other_configs"] = {}
        for c in legs:
            log(f"[bench] leg {c}")
            line["other_configs"][c] = config_leg(lib, capi, hip, c, device, stream)
        inp = build_inputs(args.config, device) if not args.no_cpu_baseline else None
    if not args.no_reference_legs:
        log("[bench] reference entry points (la_fused_mla, la_batched_fused_mla)")
        line["reference_entry_points"] = reference_entry_legs(lib, capi, hip, device, stream)
    if not args.no_cpu_baseline:
        log("[bench] cpu baseline")
        line["cpu_baseline"] = cpu_baseline(inp)
        if legs:
            log("[bench] cpu baseline, other configurations")
            line["cpu_baseline"]["other_configs"] = cpu_baseline_configs(device)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
