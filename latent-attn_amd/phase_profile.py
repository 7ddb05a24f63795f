"""Phase timings of the decode step's kernels, from the phase-timing build.

``python latent-attn_amd/build.py --phase-stamps`` compiles the library with
-DLA_PHASE_STAMPS into ``_build/phase/`` (kernels that record clock stamps at
their phase boundaries; the shipped library has none of them). This script
loads that build, runs decode steps of the benchmark workloads on cuda:0 and
prints, per workload:

* the attention kernel (``decode_mfma_kernel``): shader-clock cycles per wave
  of each phase, mean and max over the waves of all workgroups, for two
  launches: the 10th of 10 identical launches back to back, and the launch
  inside a normal step (after the absorb kernel); and the mean cycles per
  tile of each part of a loop iteration (barrier, QK phase, PV phase, wait
  for the iteration's copies), summed over the iterations and divided by
  their number;
* the absorb and merge + projection kernels: wave 0 of each block on the
  device's constant 100 MHz clock (common to all XCDs), so the block start
  spread and every phase are in microseconds on one time line.

The in-step tables come from the last of ``STEPS_IN_A_ROW`` steps launched
back to back. A step launched onto an idle GPU (after a host synchronize)
starts its first kernel's blocks XCD by XCD, up to ~4 us apart, while the
XCDs wake; back to back, as in the benchmark, every block starts within
~0.3 us.

The stamps wait for the scalar data path (it drains the wave's LDS queue),
so the instrumented kernels run a few per cent slower than the shipped ones;
the breakdown, not the total, is the result.

Usage: ``python latent-attn_amd/phase_profile.py [--configs cfg3,cfg2,b1s512]``.
"""

from __future__ import annotations

import argparse
import ctypes
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
STEPS_IN_A_ROW = 5
ROOT = os.path.dirname(HERE)
sys.path[:0] = [ROOT, HERE]

ATTN_PHASES = [
    "entry -> segment set up",
    "segment barrier",
    "Q loads issued",
    "Q issued -> tile 0 landed",
    "RoPE of tile 0",
    "iteration -1 (QK(0), softmax(0))",
    "loop t >= 0",
    "loop end -> staging barrier",
    "staging + partial stores issued",
    "stores complete",
]
TILE_PARTS = [
    "barrier (from the iteration's start)",
    "QK(t+1): 36 score MFMAs, 11 copies of tile t+2, partner P and first value reads",
    "PV(t): 32 value MFMAs, softmax(t+1), RoPE of tile t+2, P publication",
    "wait for the iteration's copies",
]
ABSORB_PHASES = ["issue loads", "wait data, LDS stores", "barrier", "MFMAs", "stores complete"]
MERGE_PHASES = ["issue W_UV loads", "merge (wave 0)", "other waves + LDS sums", "projection MFMAs", "stores complete"]


def load_phase_lib():
    from latent_attn import capi

    import build

    if not os.path.exists(build.PHASE_LIB):
        raise SystemExit(f"{build.PHASE_LIB} not built: run `python latent-attn_amd/build.py --phase-stamps`")
    capi._lib = None
    capi.LIB_PATH = build.PHASE_LIB
    lib = capi.load()
    lib.la_phase_attn_stamps.restype = ctypes.c_int
    lib.la_phase_attn_stamps.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int]
    lib.la_phase_side_stamps.restype = ctypes.c_int
    lib.la_phase_side_stamps.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_int, ctypes.c_int]
    return capi, lib


SLOTS = 16  # kStampSlots in la_mfma.hip


def attn_table(lib, blocks: int):
    import numpy as np

    buf = (ctypes.c_ulonglong * (4 * SLOTS * blocks))()
    assert lib.la_phase_attn_stamps(buf, blocks, 0) == 0
    full = np.frombuffer(buf, dtype=np.uint64).reshape(blocks, 4, SLOTS).astype(np.int64)
    full = full[full[:, 0, 10] > 0]  # workgroups that ran to the end
    a = full[:, :, :11]
    d = np.diff(a, axis=2)
    total = a[:, :, 10] - a[:, :, 0]
    n = np.maximum(full[:, :, 15], 1)
    per_tile = full[:, :, 11:15] / n[:, :, None]  # (workgroups, waves, 4 parts)
    return len(a), total, d, per_tile


def side_table(lib, kind: int, blocks: int):
    import numpy as np

    buf = (ctypes.c_ulonglong * (8 * blocks))()
    assert lib.la_phase_side_stamps(kind, buf, blocks, 0) == 0
    a = np.frombuffer(buf, dtype=np.uint64).reshape(blocks, 8).astype(np.int64)[:, :6]
    a = a[a[:, 5] > 0]
    return a


def pct(x, q):
    import numpy as np

    return float(np.percentile(x, q))


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--configs", default="cfg3,cfg2,b1s512")
    args = ap.parse_args()

    import numpy as np
    import torch

    import bench
    from latent_attn import MLAConfig

    capi, lib = load_phase_lib()
    dev = torch.device("cuda:0")
    hip = bench.hip_runtime()
    stream = torch.cuda.current_stream().cuda_stream
    print(f"phase-timing build: {capi.LIB_PATH}", flush=True)
    for name in args.configs.split(","):
        if name == "b1s512":
            inp = bench.build_inputs("cfg2", dev)
            S = 512
            g = torch.Generator(device=dev).manual_seed(3)
            kv = torch.randn(S, 576, generator=g, device=dev).to(torch.bfloat16)
            inp.update(kv=kv, total=S, seq_len=S, lens=np.array([S]))
            label = "B=1 x 512 positions"
        else:
            inp = bench.build_inputs(name, dev)
            label = bench.CONFIGS[name]["desc"]
        for k in (0, 1):
            assert lib.la_phase_side_stamps(k, None, 0, 1) == 0
        step = bench.Stepper(lib, capi, inp, stream)
        info = capi.PlanInfo()
        assert lib.la_mla_decode_plan(ctypes.byref(step.a), ctypes.byref(info)) == capi.LA_SUCCESS
        ablocks = 8 * ((info.num_chunks * info.head_groups + 7) // 8)
        for _ in range(30):
            step()
        bench.settle_clocks(step, 100)
        torch.cuda.synchronize()
        print(f"\n## {name}: {label} (chunks of {info.chunk_rows} rows x {info.num_chunks}, "
              f"{ablocks} attention workgroups)", flush=True)
        # attention kernel, 10th of 10 identical launches, then inside a step
        assert lib.la_phase_attn_stamps(None, 0, 1) == 0
        kern = bench.time_attention(hip, step)
        torch.cuda.synchronize()
        rows = {}
        rows["back to back"] = attn_table(lib, ablocks)
        for _ in range(STEPS_IN_A_ROW):  # every launch rewrites the stamps: the last step's remain
            step()
        torch.cuda.synchronize()
        rows["in a step"] = attn_table(lib, ablocks)
        print(f"\nattention kernel (instrumented), back to back: {np.median(kern) * 1e3:.2f} us per launch", flush=True)
        print("\n| phase (cycles per wave) | back to back: mean | max | in a step: mean | max |")
        print("|---|---|---|---|---|")
        for i, ph in enumerate(ATTN_PHASES):
            b, s = rows["back to back"][2][:, :, i], rows["in a step"][2][:, :, i]
            print(f"| {ph} | {b.mean():.0f} | {b.max():.0f} | {s.mean():.0f} | {s.max():.0f} |")
        tb, ts = rows["back to back"][1], rows["in a step"][1]
        print(f"| total | {tb.mean():.0f} | {tb.max():.0f} | {ts.mean():.0f} | {ts.max():.0f} |")
        print("\n| loop iteration part (cycles per tile, mean over waves) | back to back | in a step |")
        print("|---|---|---|")
        pb, ps = rows["back to back"][3], rows["in a step"][3]
        for i, part in enumerate(TILE_PARTS):
            print(f"| {part} | {pb[:, :, i].mean():.0f} | {ps[:, :, i].mean():.0f} |")
        print(f"| iteration | {pb.sum(axis=2).mean():.0f} | {ps.sum(axis=2).mean():.0f} |")
        # absorb and merge of that step
        for kind, kname, phases in ((0, "absorb", ABSORB_PHASES), (1, "merge + projection", MERGE_PHASES)):
            a = side_table(lib, kind, 8192)
            if len(a) == 0:
                continue
            t0 = a[:, 0].min()
            us = lambda v: v * 10 / 1000.0  # 100 MHz ticks
            start = us(a[:, 0] - t0)
            end = us(a[:, 5] - t0)
            d = us(np.diff(a, axis=1))
            print(f"\n{kname} kernel (instrumented, in the same step): {len(a)} blocks, first start to last end "
                  f"{us(a[:, 5].max() - t0):.2f} us")
            print("\n| phase (us, wave 0 of each block) | p10 | p50 | p90 | max |")
            print("|---|---|---|---|---|")
            print(f"| block start after the first | {pct(start, 10):.2f} | {pct(start, 50):.2f} | {pct(start, 90):.2f} | {start.max():.2f} |")
            for i, ph in enumerate(phases):
                print(f"| {ph} | {pct(d[:, i], 10):.2f} | {pct(d[:, i], 50):.2f} | {pct(d[:, i], 90):.2f} | {d[:, i].max():.2f} |")
            print(f"| block end after the first start | {pct(end, 10):.2f} | {pct(end, 50):.2f} | {pct(end, 90):.2f} | {end.max():.2f} |")
        sys.stdout.flush()
        del step, inp
        torch.cuda.empty_cache()


if __name__ == "__main__":
    main()
