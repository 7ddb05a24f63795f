"""ctypes view of the C ABI in include/latent_attn.h (liblatent_attn_hip.so).

This is the binding a Python caller without the torch extension would use:
plain integers for device pointers and the stream. ``load()`` raises if the
library is missing; there is no fallback.
"""

from __future__ import annotations

import ctypes
import os

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "liblatent_attn_hip.so")

LA_SUCCESS, LA_ERROR_INVALID_VALUE, LA_ERROR_NOT_SUPPORTED, LA_ERROR_WORKSPACE, LA_ERROR_HIP = range(5)
LA_DTYPE_F32, LA_DTYPE_F16, LA_DTYPE_BF16, LA_DTYPE_FP8_E4M3 = range(4)


class MlaConfig(ctypes.Structure):
    _fields_ = [
        ("d_model", ctypes.c_int32),
        ("kv_lora_rank", ctypes.c_int32),
        ("qk_nope_head_dim", ctypes.c_int32),
        ("qk_rope_head_dim", ctypes.c_int32),
        ("num_heads", ctypes.c_int32),
        ("v_head_dim", ctypes.c_int32),
    ]


class DecodeArgs(ctypes.Structure):
    _fields_ = [
        ("kv_cache", ctypes.c_void_p),
        ("kv_dtype", ctypes.c_int32),
        ("total_rows", ctypes.c_int64),
        ("num_seqs", ctypes.c_int32),
        ("seq_len", ctypes.c_int32),
        ("seq_offsets", ctypes.c_void_p),
        ("queries_per_seq", ctypes.c_int32),
        ("q_nope", ctypes.c_void_p),
        ("W_UK", ctypes.c_void_p),
        ("w_uk_dtype", ctypes.c_int32),
        ("q_absorbed", ctypes.c_void_p),
        ("q_rope", ctypes.c_void_p),
        ("W_UV", ctypes.c_void_p),
        ("w_uv_dtype", ctypes.c_int32),
        ("rope_cos", ctypes.c_void_p),
        ("rope_sin", ctypes.c_void_p),
        ("rope_rows", ctypes.c_int64),
        ("output", ctypes.c_void_p),
        ("cfg", MlaConfig),
        ("workspace", ctypes.c_void_p),
        ("workspace_bytes", ctypes.c_size_t),
        ("chunk_rows", ctypes.c_int32),
        ("kernel_variant", ctypes.c_int32),
        ("seq_lens", ctypes.c_void_p),
        ("block_table", ctypes.c_void_p),
        ("block_size", ctypes.c_int32),
        ("blocks_per_seq", ctypes.c_int32),
    ]


class AppendArgs(ctypes.Structure):
    _fields_ = [
        ("kv_cache", ctypes.c_void_p),
        ("kv_dtype", ctypes.c_int32),
        ("total_rows", ctypes.c_int64),
        ("num_seqs", ctypes.c_int32),
        ("seq_capacity", ctypes.c_int32),
        ("seq_offsets", ctypes.c_void_p),
        ("seq_lens", ctypes.c_void_p),
        ("tokens_per_seq", ctypes.c_int32),
        ("c_t", ctypes.c_void_p),
        ("k_rope", ctypes.c_void_p),
        ("src_dtype", ctypes.c_int32),
        ("q_rope", ctypes.c_void_p),
        ("queries_per_seq", ctypes.c_int32),
        ("rope_cos", ctypes.c_void_p),
        ("rope_sin", ctypes.c_void_p),
        ("rope_rows", ctypes.c_int64),
        ("status", ctypes.c_void_p),
        ("cfg", MlaConfig),
        ("block_table", ctypes.c_void_p),
        ("block_size", ctypes.c_int32),
        ("blocks_per_seq", ctypes.c_int32),
    ]


class PlanInfo(ctypes.Structure):
    _fields_ = [
        ("attention", ctypes.c_int32),
        ("chunk_rows", ctypes.c_int32),
        ("num_chunks", ctypes.c_int32),
        ("num_slots", ctypes.c_int32),
        ("head_groups", ctypes.c_int32),
        ("merge", ctypes.c_int32),
        ("absorb", ctypes.c_int32),
        ("workspace_bytes", ctypes.c_size_t),
    ]


LA_PLAN_ATTENTION_VALU, LA_PLAN_ATTENTION_MFMA = 1, 2
LA_PLAN_MERGE_VALU, LA_PLAN_MERGE_MFMA, LA_PLAN_MERGE_MFMA_HALVES = 1, 2, 3
LA_PLAN_ABSORB_NONE, LA_PLAN_ABSORB_VALU, LA_PLAN_ABSORB_MFMA, LA_PLAN_ABSORB_MFMA_QPREP = 0, 1, 2, 3

_lib = None


def load() -> ctypes.CDLL:
    """Load the library once and declare the prototypes."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"{LIB_PATH} not built; run `python latent-attn_amd/build.py`")
    lib = ctypes.CDLL(LIB_PATH)
    vp, i32, sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t
    cfgp = ctypes.POINTER(MlaConfig)
    lib.la_status_string.restype = ctypes.c_char_p
    lib.la_status_string.argtypes = [i32]
    lib.la_last_hip_error.restype = i32
    lib.la_last_hip_error.argtypes = []
    lib.la_abi_version.restype = i32
    lib.la_abi_version.argtypes = []
    lib.la_mla_decode_workspace_size.restype = sz
    lib.la_mla_decode_workspace_size.argtypes = [ctypes.POINTER(DecodeArgs)]
    lib.la_mla_decode.restype = i32
    lib.la_mla_decode.argtypes = [ctypes.POINTER(DecodeArgs), vp]
    lib.la_mla_decode_noalloc.restype = i32
    lib.la_mla_decode_noalloc.argtypes = [ctypes.POINTER(DecodeArgs), vp]
    lib.la_mla_decode_profiled.restype = i32
    lib.la_mla_decode_profiled.argtypes = [ctypes.POINTER(DecodeArgs), vp, vp, vp, ctypes.c_int32]
    lib.la_mla_decode_noalloc_max_bytes.restype = sz
    lib.la_mla_decode_noalloc_max_bytes.argtypes = []
    lib.la_mla_decode_plan.restype = i32
    lib.la_mla_decode_plan.argtypes = [ctypes.POINTER(DecodeArgs), ctypes.POINTER(PlanInfo)]
    lib.la_stream_ceiling.restype = i32
    lib.la_stream_ceiling.argtypes = [ctypes.POINTER(DecodeArgs), ctypes.c_int32, vp, vp, vp, ctypes.c_int32]
    lib.la_fused_mla.restype = i32
    lib.la_fused_mla.argtypes = [vp, i32, i32, vp, vp, vp, i32, vp, vp, vp, cfgp, vp, sz, vp]
    lib.la_batched_fused_mla.restype = i32
    lib.la_batched_fused_mla.argtypes = [vp, i32, i32, i32, vp, vp, vp, i32, vp, vp, vp, cfgp, vp, sz, vp]
    lib.la_fused_mla_workspace_size.restype = sz
    lib.la_fused_mla_workspace_size.argtypes = [i32, i32, cfgp]
    lib.la_fused_mla_workspace_size_dt.restype = sz
    lib.la_fused_mla_workspace_size_dt.argtypes = [i32, i32, cfgp, i32, i32]
    lib.la_absorb_q.restype = i32
    lib.la_absorb_q.argtypes = [vp, vp, i32, vp, i32, cfgp, vp]
    lib.la_naive_mla.restype = i32
    lib.la_naive_mla.argtypes = [vp, i32, i32, vp, i32, vp, i32, vp, vp, vp, vp, vp, cfgp, vp, sz, vp]
    lib.la_naive_mla_workspace_size.restype = sz
    lib.la_naive_mla_workspace_size.argtypes = [i32, cfgp]
    lib.la_append_kv.restype = i32
    lib.la_append_kv.argtypes = [ctypes.POINTER(AppendArgs), vp]
    _lib = lib
    return lib


def header_symbols() -> list[str]:
    """Function names declared in include/latent_attn.h."""
    import re

    hdr = os.path.join(os.path.dirname(os.path.dirname(os.path.dirname(LIB_PATH))), "include", "latent_attn.h")
    text = open(hdr).read()
    return sorted(set(re.findall(r"^\w[\w\s\*]*?\b(la_\w+)\s*\(", text, flags=re.M)))


def config(cfg) -> MlaConfig:
    return MlaConfig(cfg.d_model, cfg.kv_lora_rank, cfg.qk_nope_head_dim, cfg.qk_rope_head_dim, cfg.num_heads,
                     cfg.v_head_dim)
