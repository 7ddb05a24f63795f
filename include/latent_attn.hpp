// C++ drop-in for the reference's launch API, as a header-only layer over the C ABI
// of latent_attn.h (link with liblatent_attn_hip.so).
//
//   reference                                          here
//   MLAConfig               src/mla_config.cuh:7-41    latent_attn::MLAConfig
//   FusedMLAParams          src/fused_mla.cuh:11-34    latent_attn::FusedMLAParams
//   launch_fused_mla        src/fused_mla.cuh:51       latent_attn::launch_fused_mla
//   BatchedFusedMLAParams   src/fused_mla_batched.cuh:7-30
//                                                      latent_attn::BatchedFusedMLAParams
//   launch_batched_fused_mla src/fused_mla_batched.cuh:35
//                                                      latent_attn::launch_batched_fused_mla
//
// Field names and order match the reference, so aggregate initialisation written for it
// compiles unchanged (with HIP types). Appended fields (all defaulted) select the cache /
// weight dtype (the reference is fp16 only) and an optional caller workspace; without one
// the call allocates it stream-ordered (hipMallocAsync / hipFreeAsync on `stream`).
// Launches are asynchronous on `stream`; the return value reports argument errors and launch
// errors, like the reference's cudaGetLastError() return (src/fused_mla.cu:295).
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <cstddef>
#include <stdexcept>

#include "latent_attn.h"

namespace latent_attn {

struct MLAConfig {
  int d_model;
  int kv_lora_rank;      // d_c
  int qk_nope_head_dim;  // d_n
  int qk_rope_head_dim;  // d_R
  int num_heads;
  int v_head_dim;

  static MLAConfig deepseek_v2() { return {5120, 512, 128, 64, 128, 128}; }
  static MLAConfig deepseek_v3() { return {7168, 512, 128, 64, 128, 128}; }

  // Bytes per packed cache row [c_t | k_rope] in a 16-bit cache.
  int bytes_per_kv_entry() const { return (kv_lora_rank + qk_rope_head_dim) * 2; }
  size_t kv_cache_bytes(int seq_len) const { return static_cast<size_t>(seq_len) * bytes_per_kv_entry(); }

  // Same checks and messages as the reference (src/mla_config.cuh:35-40).
  void validate() const {
    if (kv_lora_rank <= 0 || qk_nope_head_dim <= 0 || qk_rope_head_dim <= 0)
      throw std::invalid_argument("MLA dims must be positive");
    if (num_heads <= 0 || v_head_dim <= 0) throw std::invalid_argument("num_heads and v_head_dim must be positive");
  }

  la_mla_config c_abi() const {
    return la_mla_config{d_model, kv_lora_rank, qk_nope_head_dim, qk_rope_head_dim, num_heads, v_head_dim};
  }
};

struct FusedMLAParams {
  const __half* kv_cache;  // (seq_len, kv_lora_rank + qk_rope_head_dim); see kv_dtype
  int seq_len;
  const float* q_absorbed;  // (num_heads, kv_lora_rank) fp32
  const float* q_rope;      // (num_heads, qk_rope_head_dim) fp32, already rotated
  const __half* W_UV;       // (num_heads * v_head_dim, kv_lora_rank); see w_uv_dtype
  const float* rope_cos;    // (seq_len, qk_rope_head_dim / 2) fp32
  const float* rope_sin;
  float* output;            // (num_heads, v_head_dim) fp32
  const MLAConfig* cfg;
  // extensions (defaulted)
  int kv_dtype = LA_DTYPE_F16;    // LA_DTYPE_F16 / LA_DTYPE_BF16 / LA_DTYPE_F32
  int w_uv_dtype = LA_DTYPE_F16;
  void* workspace = nullptr;      // >= fused_mla_workspace_size(seq_len, 1, *cfg) bytes, or null
  size_t workspace_bytes = 0;
};

struct BatchedFusedMLAParams {
  const __half* kv_cache;  // shared cache (seq_len, kv_lora_rank + qk_rope_head_dim)
  int seq_len;
  int batch_size;
  const float* q_absorbed;  // (batch_size, num_heads, kv_lora_rank) fp32
  const float* q_rope;      // (batch_size, num_heads, qk_rope_head_dim) fp32
  const __half* W_UV;
  const float* rope_cos;
  const float* rope_sin;
  float* output;            // (batch_size, num_heads, v_head_dim) fp32
  const MLAConfig* cfg;
  // extensions (defaulted)
  int kv_dtype = LA_DTYPE_F16;
  int w_uv_dtype = LA_DTYPE_F16;
  void* workspace = nullptr;
  size_t workspace_bytes = 0;
};

// C-ABI status -> hipError_t.
inline hipError_t to_hip_error(int status) {
  switch (status) {
    case LA_SUCCESS: return hipSuccess;
    case LA_ERROR_NOT_SUPPORTED: return hipErrorNotSupported;
    case LA_ERROR_HIP: return static_cast<hipError_t>(la_last_hip_error());
    default: return hipErrorInvalidValue;  // LA_ERROR_INVALID_VALUE, LA_ERROR_WORKSPACE
  }
}

inline size_t fused_mla_workspace_size(int seq_len, int batch_size, const MLAConfig& cfg) {
  const la_mla_config c = cfg.c_abi();
  return la_fused_mla_workspace_size(seq_len, batch_size, &c);
}

inline hipError_t launch_fused_mla(const FusedMLAParams& p, hipStream_t stream = 0) {
  if (!p.cfg) return hipErrorInvalidValue;
  const la_mla_config c = p.cfg->c_abi();
  return to_hip_error(la_fused_mla(p.kv_cache, p.kv_dtype, p.seq_len, p.q_absorbed, p.q_rope, p.W_UV, p.w_uv_dtype,
                                   p.rope_cos, p.rope_sin, p.output, &c, p.workspace, p.workspace_bytes,
                                   static_cast<void*>(stream)));
}

inline hipError_t launch_batched_fused_mla(const BatchedFusedMLAParams& p, hipStream_t stream = 0) {
  if (!p.cfg) return hipErrorInvalidValue;
  const la_mla_config c = p.cfg->c_abi();
  return to_hip_error(la_batched_fused_mla(p.kv_cache, p.kv_dtype, p.seq_len, p.batch_size, p.q_absorbed, p.q_rope,
                                           p.W_UV, p.w_uv_dtype, p.rope_cos, p.rope_sin, p.output, &c, p.workspace,
                                           p.workspace_bytes, static_cast<void*>(stream)));
}

}  // namespace latent_attn
