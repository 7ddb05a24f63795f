// Drop-in for the reference's src/mla_config.cuh (paths relative to the
// reference repo): MLAConfig (:7-41) and LatentKVCache (:45-92) in the global
// namespace with HIP types, over the C ABI of latent_attn.h (link with
// liblatent_attn_hip.so).
//
// Field names, order and member functions match the reference, so code written
// against it compiles after its CUDA runtime calls are ported to HIP.
// LatentKVCache::append_host keeps the reference's contract (host row in,
// "KV cache full" when full, returns after the row is in the cache) but
// writes the row with the library's device-side append (la_append_kv):
// the row is staged in stream-ordered device memory and appended by the
// append kernel, instead of two host-to-device copies into the row.
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>

#include "latent_attn.h"

struct MLAConfig {
  int d_model;
  int kv_lora_rank;      // d_c: compressed KV latent dimension
  int qk_nope_head_dim;  // per-head non-RoPE key/query dim
  int qk_rope_head_dim;  // per-head RoPE key/query dim (d_R)
  int num_heads;
  int v_head_dim;

  // DeepSeek-V2 / V3 MLA shapes (reference src/mla_config.cuh:16-24)
  static MLAConfig deepseek_v2() { return {5120, 512, 128, 64, 128, 128}; }
  static MLAConfig deepseek_v3() { return {7168, 512, 128, 64, 128, 128}; }

  // Bytes per packed cache row [c_t | k_rope] in a 16-bit cache.
  int bytes_per_kv_entry() const { return (kv_lora_rank + qk_rope_head_dim) * (int)sizeof(__half); }
  size_t kv_cache_bytes(int seq_len) const { return static_cast<size_t>(seq_len) * bytes_per_kv_entry(); }

  // Same conditions and messages as the reference (src/mla_config.cuh:35-40).
  void validate() const {
    if (kv_lora_rank <= 0 || qk_nope_head_dim <= 0 || qk_rope_head_dim <= 0)
      throw std::invalid_argument("MLA dims must be positive");
    if (num_heads <= 0 || v_head_dim <= 0) throw std::invalid_argument("num_heads and v_head_dim must be positive");
  }

  la_mla_config c_abi() const {
    return la_mla_config{d_model, kv_lora_rank, qk_nope_head_dim, qk_rope_head_dim, num_heads, v_head_dim};
  }
};

// Packed per-position latent cache [c_t (kv_lora_rank) | k_rope (qk_rope_head_dim)],
// fp16, caller-owned device memory of max_seq_len rows.
struct LatentKVCache {
  __half* data;      // device pointer, (max_seq_len, kv_lora_rank + qk_rope_head_dim)
  int max_seq_len;
  int entry_stride;  // kv_lora_rank + qk_rope_head_dim
  int current_len;   // filled positions

  LatentKVCache(__half* device_ptr, int max_len, const MLAConfig& cfg)
      : data(device_ptr), max_seq_len(max_len), entry_stride(cfg.kv_lora_rank + cfg.qk_rope_head_dim),
        current_len(0) {}

  // Appends one position from host memory: c_t (kv_lora_rank) and the
  // un-rotated k_rope_t (qk_rope_head_dim), fp16. Returns once the row is in
  // the cache (the reference synchronizes the stream too). Throws
  // std::runtime_error("KV cache full") when full, like the reference, and
  // std::runtime_error naming the failing call on a HIP or library error.
  void append_host(const __half* c_t, const __half* k_rope_t, const MLAConfig& cfg, hipStream_t stream = 0) {
    if (current_len >= max_seq_len) throw std::runtime_error("KV cache full");
    const size_t dc = (size_t)cfg.kv_lora_rank, dr = (size_t)cfg.qk_rope_head_dim;
    // staging: [c_t | k_rope] fp16, then the int32 length, 16-B aligned
    const size_t row_bytes = (dc + dr) * sizeof(__half);
    const size_t len_off = (row_bytes + 15) / 16 * 16;
    char* stage = nullptr;
    check(hipMallocAsync(reinterpret_cast<void**>(&stage), len_off + 16, stream), "hipMallocAsync");
    const int32_t len = current_len;
    hipError_t e = hipMemcpyAsync(stage, c_t, dc * sizeof(__half), hipMemcpyHostToDevice, stream);
    if (e == hipSuccess)
      e = hipMemcpyAsync(stage + dc * sizeof(__half), k_rope_t, dr * sizeof(__half), hipMemcpyHostToDevice, stream);
    if (e == hipSuccess) e = hipMemcpyAsync(stage + len_off, &len, sizeof(len), hipMemcpyHostToDevice, stream);
    int st = LA_SUCCESS;
    if (e == hipSuccess) {
      la_append_args a{};
      a.kv_cache = data;
      a.kv_dtype = LA_DTYPE_F16;
      a.total_rows = max_seq_len;
      a.num_seqs = 1;
      a.seq_capacity = max_seq_len;
      a.seq_lens = reinterpret_cast<int32_t*>(stage + len_off);
      a.tokens_per_seq = 1;
      a.c_t = stage;                                // (1, 1, dc) fp16
      a.k_rope = stage + dc * sizeof(__half);       // (1, 1, dr) fp16
      a.src_dtype = LA_DTYPE_F16;
      a.cfg = cfg.c_abi();
      st = la_append_kv(&a, static_cast<void*>(stream));
    }
    // the host copies above read the caller's memory and &len: finish them
    // (and the append) before returning, as the reference does
    const hipError_t f = hipFreeAsync(stage, stream);
    const hipError_t s = hipStreamSynchronize(stream);
    check(e, "hipMemcpyAsync");
    if (st != LA_SUCCESS) throw std::runtime_error(std::string("la_append_kv: ") + la_status_string(st));
    check(f, "hipFreeAsync");
    check(s, "hipStreamSynchronize");
    ++current_len;
  }

  // Device accessor: pointers into the packed buffer for position pos.
  __device__ void get(int pos, int kv_lora_rank, const __half*& c_t_out, const __half*& k_rope_out) const {
    const __half* base = data + (size_t)pos * entry_stride;
    c_t_out = base;
    k_rope_out = base + kv_lora_rank;
  }

  // Packed row pos.
  __device__ __host__ const __half* row(int pos) const { return data + (size_t)pos * entry_stride; }
  __device__ __host__ __half* row(int pos) { return data + (size_t)pos * entry_stride; }

 private:
  static void check(hipError_t e, const char* what) {
    if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
  }
};
