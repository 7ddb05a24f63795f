"""CPU checks of the C ABI and the torch extension's argument validation.

No kernels run here: only symbol export, ABI constants, argument rejection
(which happens before any HIP call) and the extension's input checks, which
mirror the reference's TORCH_CHECKs (reference csrc/bindings.cpp:28-40,
147-152, 208-221).
"""

from __future__ import annotations

import ctypes

import pytest
import torch

from latent_attn import MLAConfig, capi
from latent_attn import functional as F


def test_library_exports_header_symbols():
    lib = capi.load()
    names = capi.header_symbols()
    assert {"la_mla_decode", "la_fused_mla", "la_batched_fused_mla", "la_absorb_q", "la_append_kv"} <= set(names)
    for n in names:
        assert hasattr(lib, n), n
    assert lib.la_abi_version() == 4


def test_ctypes_structs_match_the_header(tmp_path):
    """The ctypes mirrors of la_decode_args / la_append_args have the C
    header's size and field offsets (a C program compiled with gcc prints
    them)."""
    import os
    import shutil
    import subprocess

    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc not available")
    REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    structs = {"la_decode_args": capi.DecodeArgs, "la_append_args": capi.AppendArgs,
               "la_plan_info": capi.PlanInfo}
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "latent_attn.h"', "int main(void) {"]
    for cname, py in structs.items():
        lines.append(f'  printf("{cname} size %zu\\n", sizeof({cname}));')
        for f, _ in py._fields_:
            lines.append(f'  printf("{cname} {f} %zu\\n", offsetof({cname}, {f}));')
    lines += ["  return 0;", "}"]
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines) + "\n")
    exe = tmp_path / "layout"
    subprocess.run([gcc, "-I" + os.path.join(REPO, "include"), str(src), "-o", str(exe)], check=True)
    got = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split("\n")
    want = []
    for cname, py in structs.items():
        want.append(f"{cname} size {ctypes.sizeof(py)}")
        want += [f"{cname} {f} {getattr(py, f).offset}" for f, _ in py._fields_]
    assert [l for l in got if l] == want


def _append_args(**kw):
    a = capi.AppendArgs()
    a.cfg = capi.config(MLAConfig.deepseek_v2())
    a.kv_dtype = capi.LA_DTYPE_BF16
    a.src_dtype = capi.LA_DTYPE_F32
    a.num_seqs = 2
    a.seq_capacity = 8
    a.total_rows = 16
    a.tokens_per_seq = 1
    fake = 0x1000
    a.kv_cache = a.seq_lens = a.c_t = a.k_rope = fake
    for k, v in kw.items():
        setattr(a, k, v)
    return a


@pytest.mark.parametrize("field,value", [
    ("num_seqs", -1),
    ("tokens_per_seq", -1),
    ("seq_capacity", 9),        # 2 * 9 rows do not fit in total_rows = 16
    ("kv_dtype", 7),
    ("src_dtype", 5),
    ("seq_lens", 0),
    ("kv_cache", 0),
    ("c_t", 0),
    ("k_rope", 0),
    ("rope_rows", -1),
    ("q_rope", 0x2000),         # query rotation without tables
])
def test_append_rejects_bad_arguments(field, value):
    lib = capi.load()
    a = _append_args(**{field: value})
    assert lib.la_append_kv(ctypes.byref(a), None) == capi.LA_ERROR_INVALID_VALUE


def test_append_rejects_more_queries_than_tokens():
    lib = capi.load()
    a = _append_args(q_rope=0x2000, rope_cos=0x3000, rope_sin=0x3000, queries_per_seq=2)
    assert lib.la_append_kv(ctypes.byref(a), None) == capi.LA_ERROR_INVALID_VALUE
    a = _append_args(q_rope=0x2000, rope_cos=0x3000, rope_sin=0x3000, queries_per_seq=0)
    assert lib.la_append_kv(ctypes.byref(a), None) == capi.LA_ERROR_INVALID_VALUE
    assert lib.la_append_kv(None, None) == capi.LA_ERROR_INVALID_VALUE


def test_append_empty_batch_is_a_no_op():
    lib = capi.load()
    a = _append_args(num_seqs=0, total_rows=0, kv_cache=0, seq_lens=0)
    assert lib.la_append_kv(ctypes.byref(a), None) == capi.LA_SUCCESS


def test_status_strings():
    lib = capi.load()
    assert lib.la_status_string(capi.LA_SUCCESS) == b"success"
    assert lib.la_status_string(capi.LA_ERROR_INVALID_VALUE) == b"invalid value"
    assert lib.la_status_string(capi.LA_ERROR_WORKSPACE) == b"workspace too small"
    assert lib.la_status_string(99) == b"unknown status"


def _args(**kw):
    a = capi.DecodeArgs()
    a.cfg = capi.config(MLAConfig.deepseek_v2())
    a.kv_dtype = capi.LA_DTYPE_BF16
    a.w_uv_dtype = capi.LA_DTYPE_BF16
    a.w_uk_dtype = capi.LA_DTYPE_BF16
    a.num_seqs = 1
    a.queries_per_seq = 1
    a.seq_len = 16
    a.total_rows = 16
    fake = 0x1000
    a.kv_cache = a.q_rope = a.W_UV = a.rope_cos = a.rope_sin = a.output = a.q_absorbed = fake
    for k, v in kw.items():
        setattr(a, k, v)
    return a


@pytest.mark.parametrize("field,value", [
    ("queries_per_seq", 0),
    ("num_seqs", -1),
    ("seq_len", -3),
    ("total_rows", 8),          # uniform sequences need num_seqs*seq_len rows
    ("kv_dtype", 7),
    ("q_absorbed", 0),          # neither q_nope nor q_absorbed
    ("q_nope", 0x2000),         # both q_nope and q_absorbed
    ("chunk_rows", -1),
    ("kernel_variant", 5),
    ("q_rope", 0),
    ("output", 0),
])
def test_decode_rejects_bad_arguments(field, value):
    lib = capi.load()
    a = _args(**{field: value})
    assert lib.la_mla_decode(ctypes.byref(a), None) == capi.LA_ERROR_INVALID_VALUE


def test_profiled_decode_rejects_a_negative_repeat():
    """la_mla_decode_profiled checks its repeat count before any device work
    (and, like la_mla_decode, every descriptor field)."""
    lib = capi.load()
    a = _args()
    assert lib.la_mla_decode_profiled(ctypes.byref(a), None, None, None, -1) == capi.LA_ERROR_INVALID_VALUE
    a = _args(queries_per_seq=0)
    assert lib.la_mla_decode_profiled(ctypes.byref(a), None, None, None, 10) == capi.LA_ERROR_INVALID_VALUE


def test_plan_query_without_a_gfx950_device():
    """la_mla_decode_plan reports the plan la_mla_decode would run. Without a
    gfx950 device (this host) the MFMA attention kernel is not selectable:
    the VALU kernel's plan aims at 4 workgroups per CU (256 CUs assumed) over
    one workgroup per query head. Config 3's shape (32 sequences x 8,192 rows,
    128 heads): 1,024 / 128 = 8 chunks of 32,768 rows, 8 + 32 - 1 = 39 slots
    per head; fp32 partials, merged and projected on the MFMA merge; q_nope
    absorbed on the MFMA absorb kernel into fp32 queries."""
    lib = capi.load()
    a = _args(num_seqs=32, seq_len=8192, total_rows=32 * 8192, q_absorbed=0, q_nope=0x2000, W_UK=0x3000)
    info = capi.PlanInfo()
    assert lib.la_mla_decode_plan(ctypes.byref(a), ctypes.byref(info)) == capi.LA_SUCCESS
    assert (info.attention, info.chunk_rows, info.num_chunks, info.num_slots, info.head_groups) == (
        capi.LA_PLAN_ATTENTION_VALU, 32768, 8, 39, 128)
    assert (info.merge, info.absorb) == (capi.LA_PLAN_MERGE_MFMA, capi.LA_PLAN_ABSORB_MFMA)
    al = lambda x: (x + 255) // 256 * 256
    want = al(32 * 128 * 512 * 4) + al(39 * 128 * 512 * 4) + al(39 * 128 * 4)  # q_abs, fp32 partials, lse
    assert info.workspace_bytes == want == lib.la_mla_decode_workspace_size(ctypes.byref(a))
    # pre-absorbed queries: no absorb step; an empty batch: an empty plan
    b = _args(num_seqs=32, seq_len=8192, total_rows=32 * 8192)
    assert lib.la_mla_decode_plan(ctypes.byref(b), ctypes.byref(info)) == capi.LA_SUCCESS
    assert info.absorb == capi.LA_PLAN_ABSORB_NONE
    e = _args(num_seqs=0)
    assert lib.la_mla_decode_plan(ctypes.byref(e), ctypes.byref(info)) == capi.LA_SUCCESS
    assert (info.attention, info.num_chunks, info.workspace_bytes) == (0, 0, 0)
    assert lib.la_mla_decode_plan(ctypes.byref(_args(queries_per_seq=0)), ctypes.byref(info)) == \
        capi.LA_ERROR_INVALID_VALUE
    assert lib.la_mla_decode_plan(ctypes.byref(a), None) == capi.LA_ERROR_INVALID_VALUE


def test_stream_ceiling_rejects_bad_arguments():
    """la_stream_ceiling (the copies-only measurement of the attention
    kernel's copy schedule) checks its ring depth, repeat count and
    descriptor before any device work."""
    lib = capi.load()
    a = _args()
    for ring in (0, 2, 5):
        assert lib.la_stream_ceiling(ctypes.byref(a), ring, None, None, None, 1) == capi.LA_ERROR_INVALID_VALUE
    assert lib.la_stream_ceiling(ctypes.byref(a), 3, None, None, None, -1) == capi.LA_ERROR_INVALID_VALUE
    a = _args(queries_per_seq=0)
    assert lib.la_stream_ceiling(ctypes.byref(a), 3, None, None, None, 1) == capi.LA_ERROR_INVALID_VALUE


def test_decode_rejects_bad_config():
    lib = capi.load()
    a = _args()
    a.cfg.qk_rope_head_dim = 63  # odd: rotate-half needs pairs
    assert lib.la_mla_decode(ctypes.byref(a), None) == capi.LA_ERROR_INVALID_VALUE
    a = _args()
    a.cfg.num_heads = 0
    assert lib.la_mla_decode(ctypes.byref(a), None) == capi.LA_ERROR_INVALID_VALUE
    assert lib.la_mla_decode(None, None) == capi.LA_ERROR_INVALID_VALUE


def test_empty_batch_is_a_no_op():
    lib = capi.load()
    a = _args(num_seqs=0, total_rows=0)
    assert lib.la_mla_decode(ctypes.byref(a), None) == capi.LA_SUCCESS


def test_absorb_rejects_bad_arguments():
    lib = capi.load()
    cfg = capi.config(MLAConfig.deepseek_v2())
    assert lib.la_absorb_q(None, None, 2, None, -1, ctypes.byref(cfg), None) == capi.LA_ERROR_INVALID_VALUE
    assert lib.la_absorb_q(None, None, 2, None, 0, ctypes.byref(cfg), None) == capi.LA_SUCCESS
    assert lib.la_absorb_q(0x10, 0x10, 9, 0x10, 1, ctypes.byref(cfg), None) == capi.LA_ERROR_INVALID_VALUE


# ---- torch extension checks (CPU tensors never reach the library) ----------

def _fused_inputs(dtype=torch.float16, S=8, nh=4):
    cfg = MLAConfig(5120, 512, 128, 64, nh, 128)
    kv = torch.zeros(S, 576, dtype=dtype)
    qa = torch.zeros(nh, 512)
    qr = torch.zeros(nh, 64)
    W = torch.zeros(nh * 128, 512, dtype=dtype)
    c = torch.zeros(S, 32)
    return cfg, kv, qa, qr, W, c


def test_extension_requires_device_tensors():
    cfg, kv, qa, qr, W, c = _fused_inputs()
    with pytest.raises(RuntimeError, match="kv_cache must be on CUDA"):
        F.fused_mla(kv, qa, qr, W, c, c, cfg)


def test_extension_dtype_and_layout_messages():
    cfg, kv, qa, qr, W, c = _fused_inputs()
    with pytest.raises(RuntimeError, match="kv_cache must be float16, bfloat16, float32 or float8_e4m3fn"):
        F.fused_mla(kv.to(torch.int32), qa, qr, W, c, c, cfg)
    with pytest.raises(RuntimeError, match="kv_cache must be contiguous"):
        F.fused_mla(kv.t(), qa, qr, W, c, c, cfg)


def test_config_validation_messages():
    """MLAConfig.validate raises like src/mla_config.cuh:35-40 (the extension
    raises the same ValueError after its tensor checks; see the GPU tests)."""
    with pytest.raises(ValueError, match="MLA dims must be positive"):
        MLAConfig(5120, 0, 128, 64, 4, 128).validate()
    with pytest.raises(ValueError, match="num_heads and v_head_dim must be positive"):
        MLAConfig(5120, 512, 128, 64, 0, 128).validate()
    MLAConfig.deepseek_v2().validate()


def test_batched_rejects_2d_queries():
    cfg, kv, qa, qr, W, c = _fused_inputs()
    with pytest.raises(RuntimeError):
        F.batched_fused_mla(kv, qa, qr, W, c, c, cfg)


def test_functional_signatures_match_reference():
    import inspect

    assert list(inspect.signature(F.fused_mla).parameters) == [
        "kv_cache", "q_absorbed", "q_rope", "W_UV", "rope_cos", "rope_sin", "cfg"]
    assert list(inspect.signature(F.naive_mla).parameters) == [
        "kv_cache", "W_UK", "W_UV", "q_nope", "q_rope", "rope_cos", "rope_sin", "cfg"]
    assert list(inspect.signature(F.batched_fused_mla).parameters) == [
        "kv_cache", "q_absorbed", "q_rope", "W_UV", "rope_cos", "rope_sin", "cfg"]
    assert MLAConfig.deepseek_v2() == MLAConfig(5120, 512, 128, 64, 128, 128)
    assert MLAConfig.deepseek_v3() == MLAConfig(7168, 512, 128, 64, 128, 128)
    assert MLAConfig.deepseek_v2().bytes_per_kv_entry() == 1152


def test_cpp_dropin_header_compiles_and_links(tmp_path):
    """include/{mla_config,fused_mla,fused_mla_batched}.cuh under the
    reference's own header names: reference-style aggregate initialisation of
    FusedMLAParams / BatchedFusedMLAParams (src/fused_mla.cuh:11-34,
    src/fused_mla_batched.cuh:7-30) compiles with HIP types and links against
    the library; the workspace query runs on the host."""
    import os
    import shutil
    import subprocess

    REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    gxx = shutil.which("g++")
    if gxx is None or not os.path.isdir("/opt/rocm/include/hip"):
        pytest.skip("g++ or HIP headers not available")
    src = tmp_path / "dropin.cpp"
    src.write_text(
        '#include "fused_mla.cuh"\n'
        '#include "fused_mla_batched.cuh"\n'
        '#include "mla_config.cuh"\n'
        "int main() {\n"
        "  MLAConfig cfg = MLAConfig::deepseek_v2();\n"
        "  cfg.validate();\n"
        "  FusedMLAParams p{nullptr, 16, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, &cfg};\n"
        "  BatchedFusedMLAParams b{nullptr, 16, 2, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, &cfg};\n"
        "  if (p.kv_dtype != LA_DTYPE_F16 || b.batch_size != 2) return 2;\n"
        "  if (launch_fused_mla(FusedMLAParams{}) != hipErrorInvalidValue) return 3;\n"
        "  MLAConfig c2 = MLAConfig::deepseek_v3();\n"
        "  FusedMLAParams q; q.cfg = nullptr;\n"
        "  if (launch_fused_mla(q) != hipErrorInvalidValue) return 4;\n"
        "  BatchedFusedMLAParams bq; bq.cfg = &c2; bq.batch_size = 0;\n"
        "  __half* base = reinterpret_cast<__half*>(0x1000);\n"
        "  LatentKVCache cache(base, 4, c2);\n"
        "  if (cache.entry_stride != 576 || cache.current_len != 0 || cache.row(2) != base + 2 * 576) return 5;\n"
        "  // one dtype pair never needs more than the largest over all pairs\n"
        "  const la_mla_config cc = c2.c_abi();\n"
        "  if (fused_mla_workspace_size(16, 2, c2, LA_DTYPE_BF16, LA_DTYPE_BF16) >\n"
        "      la_fused_mla_workspace_size(16, 2, &cc)) return 6;\n"
        "  return fused_mla_workspace_size(16, 2, cfg) > 0 ? 0 : 1;\n"
        "}\n")
    libdir = os.path.join(REPO, "latent-attn_amd", "latent_attn")
    exe = tmp_path / "dropin"
    subprocess.run([gxx, "-std=c++17", "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include",
                    "-I" + os.path.join(REPO, "include"), str(src), "-o", str(exe), "-L" + libdir,
                    "-llatent_attn_hip", "-Wl,-rpath," + libdir], check=True)
    assert subprocess.run([str(exe)]).returncode == 0


def test_naive_rejects_bad_arguments_and_sizes_its_workspace():
    lib = capi.load()
    cfg = capi.config(MLAConfig.deepseek_v2())
    f = 0x1000
    ok = [f, capi.LA_DTYPE_BF16, 16, f, capi.LA_DTYPE_BF16, f, capi.LA_DTYPE_BF16, f, f, f, f, f]
    for i, bad in [(1, 9), (2, -1), (3, 0), (4, 7), (5, 0), (7, 0), (8, 0), (9, 0), (10, 0), (11, 0)]:
        args = list(ok)
        args[i] = bad
        assert lib.la_naive_mla(*args, ctypes.byref(cfg), None, 0, None) == capi.LA_ERROR_INVALID_VALUE, i
    # too small a caller workspace is refused before any launch
    assert lib.la_naive_mla(*ok, ctypes.byref(cfg), 0x2000, 16, None) == capi.LA_ERROR_WORKSPACE
    # fp32 K_nope (S, H*dn), V (S, H*dv) and scores (H, S), each 256-B aligned
    S = 1000
    up = lambda x: (x + 255) // 256 * 256
    want = up(S * 128 * 128 * 4) + up(S * 128 * 128 * 4) + up(S * 128 * 4)
    assert lib.la_naive_mla_workspace_size(S, ctypes.byref(cfg)) == want
    assert lib.la_naive_mla_workspace_size(-1, ctypes.byref(cfg)) == 0


@pytest.mark.parametrize("field,value", [
    ("block_size", 0),
    ("blocks_per_seq", 0),
    ("seq_lens", 0),            # a paged cache needs device lengths
    ("seq_offsets", 0x3000),    # block tables and packed offsets exclude each other
    ("total_rows", 100),        # the pool is whole blocks
    ("total_rows", 0),          # a pool without a block: no row to clamp a table entry into
])
def test_decode_rejects_bad_paged_arguments(field, value):
    lib = capi.load()
    a = _args(block_table=0x2000, block_size=64, blocks_per_seq=2, seq_lens=0x2100, total_rows=128, seq_len=0)
    setattr(a, field, value)
    assert lib.la_mla_decode(ctypes.byref(a), None) == capi.LA_ERROR_INVALID_VALUE


def test_append_rejects_bad_paged_arguments():
    lib = capi.load()
    for field, value in (("block_size", 0), ("blocks_per_seq", -1), ("seq_offsets", 0x3000), ("total_rows", 100),
                         ("total_rows", 0)):
        a = _append_args(block_table=0x2000, block_size=64, blocks_per_seq=2, total_rows=256)
        setattr(a, field, value)
        assert lib.la_append_kv(ctypes.byref(a), None) == capi.LA_ERROR_INVALID_VALUE, field
