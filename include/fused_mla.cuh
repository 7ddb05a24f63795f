// Drop-in for the reference's src/fused_mla.cuh (paths relative to the
// reference repo): FusedMLAParams (:11-34) and launch_fused_mla (:51) in the
// global namespace with HIP types, as a header-only layer over the C ABI of
// latent_attn.h (link with liblatent_attn_hip.so).
//
// Field names and order match the reference, so code that fills the struct
// field by field or by aggregate initialisation compiles unchanged (with HIP
// types). Appended fields, all defaulted, select the cache / weight dtype
// (the reference is fp16 only; bf16, fp32 and, for the cache, FP8 E4M3 are
// accepted) and an optional caller workspace (size: fused_mla_workspace_size).
// The reference's device helpers latent_dot / rope_score_correction
// (:37-49) belong to its kernel, not to the launch API, and have no
// counterpart. The launch is asynchronous on `stream`; the return value
// reports argument and launch errors, like the reference's cudaGetLastError()
// return (src/fused_mla.cu:295).
#pragma once

#include "mla_config.cuh"

struct FusedMLAParams {
  const __half* kv_cache;   // (seq_len, kv_lora_rank + qk_rope_head_dim); see kv_dtype
  int seq_len;
  const float* q_absorbed;  // (num_heads, kv_lora_rank) fp32
  const float* q_rope;      // (num_heads, qk_rope_head_dim) fp32, already rotated
  const __half* W_UV;       // (num_heads * v_head_dim, kv_lora_rank); see w_uv_dtype
  const float* rope_cos;    // (seq_len, qk_rope_head_dim / 2) fp32
  const float* rope_sin;
  float* output;            // (num_heads, v_head_dim) fp32
  const MLAConfig* cfg;
  // extensions (defaulted)
  int kv_dtype = LA_DTYPE_F16;    // la_dtype of kv_cache
  int w_uv_dtype = LA_DTYPE_F16;  // la_dtype of W_UV
  void* workspace = nullptr;      // >= fused_mla_workspace_size(...) bytes; null: allocated stream-ordered
  size_t workspace_bytes = 0;
};

// C-ABI status -> hipError_t.
inline hipError_t la_to_hip_error(int status) {
  switch (status) {
    case LA_SUCCESS: return hipSuccess;
    case LA_ERROR_NOT_SUPPORTED: return hipErrorNotSupported;
    case LA_ERROR_HIP: return static_cast<hipError_t>(la_last_hip_error());
    default: return hipErrorInvalidValue;  // LA_ERROR_INVALID_VALUE, LA_ERROR_WORKSPACE
  }
}

// Workspace bytes for a cache / weight dtype pair (batch_size 1 for
// launch_fused_mla).
inline size_t fused_mla_workspace_size(int seq_len, int batch_size, const MLAConfig& cfg, int kv_dtype = LA_DTYPE_F16,
                                       int w_uv_dtype = LA_DTYPE_F16) {
  const la_mla_config c = cfg.c_abi();
  return la_fused_mla_workspace_size_dt(seq_len, batch_size, &c, kv_dtype, w_uv_dtype);
}

inline hipError_t launch_fused_mla(const FusedMLAParams& p, hipStream_t stream = 0) {
  if (!p.cfg) return hipErrorInvalidValue;
  const la_mla_config c = p.cfg->c_abi();
  return la_to_hip_error(la_fused_mla(p.kv_cache, p.kv_dtype, p.seq_len, p.q_absorbed, p.q_rope, p.W_UV,
                                      p.w_uv_dtype, p.rope_cos, p.rope_sin, p.output, &c, p.workspace,
                                      p.workspace_bytes, static_cast<void*>(stream)));
}
