// Drop-in for the reference's src/fused_mla_batched.cuh (paths relative to
// the reference repo): BatchedFusedMLAParams (:7-30) and
// launch_batched_fused_mla (:35) in the global namespace with HIP types, over
// the C ABI of latent_attn.h. Same conventions as fused_mla.cuh: reference
// fields in reference order, then defaulted dtype / workspace extensions.
#pragma once

#include "fused_mla.cuh"

struct BatchedFusedMLAParams {
  const __half* kv_cache;   // shared cache (seq_len, kv_lora_rank + qk_rope_head_dim)
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

inline hipError_t launch_batched_fused_mla(const BatchedFusedMLAParams& p, hipStream_t stream = 0) {
  if (!p.cfg) return hipErrorInvalidValue;
  const la_mla_config c = p.cfg->c_abi();
  return la_to_hip_error(la_batched_fused_mla(p.kv_cache, p.kv_dtype, p.seq_len, p.batch_size, p.q_absorbed,
                                              p.q_rope, p.W_UV, p.w_uv_dtype, p.rope_cos, p.rope_sin, p.output, &c,
                                              p.workspace, p.workspace_bytes, static_cast<void*>(stream)));
}
