// Device-side latent-cache append with query RoPE (la_append_kv).
//
// Replaces LatentKVCache::append_host (paths relative to the reference repo,
// src/mla_config.cuh:57-72), which copies one host row into the cache with two
// host-to-device copies and a stream synchronize per token and keeps the
// length on the host. Here one launch appends tokens_per_seq rows to every
// sequence of a batch, the lengths live in device memory, and nothing waits on
// the host, so a decode step (append -> absorb -> attend -> project) is one
// stream-ordered sequence of kernels.
//
// Rows are stored as the reference's cache holds them: [c_t | k_rope] with
// k_rope not rotated (the attention rotates keys by position,
// src/fused_mla.cu:34-54). The reference never rotates the query; this kernel
// rotates q_rope for the query's own position with the same rotate-half
// pairing (i, i + dR/2) and the same tables (src/fused_mla.cu:43-51), so
// callers no longer pre-rotate it.
#include "la_internal.hpp"

#include <algorithm>

namespace la {
namespace {

constexpr int kAppendThreads = 1024;

__device__ inline void store_any(void* base, int dtype, int64_t i, float v) {
  if (dtype == LA_DTYPE_BF16) reinterpret_cast<__hip_bfloat16*>(base)[i] = __float2bfloat16(v);
  else if (dtype == LA_DTYPE_F16) reinterpret_cast<__half*>(base)[i] = __float2half(v);
  else if (dtype == LA_DTYPE_FP8_E4M3) reinterpret_cast<uint8_t*>(base)[i] = f32_to_fp8(v);
  else reinterpret_cast<float*>(base)[i] = v;
}

typedef float f32x4 __attribute__((ext_vector_type(4)));

// One workgroup per sequence. Thread 0 reads the sequence's length and checks
// the room in its region; after a barrier every thread copies (and converts)
// its share of the new rows and rotates its share of the query pairs; after a
// second barrier (all reads of the old length done) thread 0 stores the new
// length. A sequence without room is left untouched and raises *status.
// Index arithmetic is 32-bit (the launcher bounds the per-sequence counts).
// The rotation takes four consecutive pairs per thread with 16-B loads when
// dR/2 is a multiple of 4 (every query row and table row is then 16-B
// aligned; the launcher checks the base pointers), one pair otherwise. With
// up to 1024 groups per sequence (128 heads x 8 groups of a 64-wide rope
// dimension) every thread has one group, so a sequence costs one memory round
// trip for its loads and one for its stores.
__global__ __launch_bounds__(kAppendThreads) void append_kernel(AppendProblem p) {
  const int s = blockIdx.x;
  __shared__ int64_t first_row;  // row of the first new token, -1 = no room
  __shared__ int old_len;
  if (threadIdx.x == 0) {
    // paged: a virtual region of blocks_per_seq blocks (rows are mapped below)
    const int64_t start = p.block_table ? 0 : p.offsets ? (int64_t)p.offsets[s] : (int64_t)s * p.capacity;
    const int64_t end = p.block_table ? (int64_t)p.blocks_per_seq * p.block_size
                        : p.offsets   ? (int64_t)p.offsets[s + 1]
                                      : start + p.capacity;
    const int len = p.lens[s];
    const bool ok = start >= 0 && start <= end && (p.block_table || end <= p.total_rows) && len >= 0 &&
                    (int64_t)len + p.tokens <= end - start;
    first_row = ok ? start + len : -1;
    old_len = len;
    if (!ok && p.status) *p.status = 1;
  }
  __syncthreads();
  const int64_t row0 = first_row;
  const int len = old_len;
  if (row0 < 0) return;

  const int row = p.dc + p.dR;
  const int n = p.tokens * row;
  const int64_t tok0 = (int64_t)s * p.tokens;
  for (int i = threadIdx.x; i < n; i += kAppendThreads) {
    const int t = i / row;
    const int c = i - t * row;
    const float v = c < p.dc ? load_any(p.c_t, p.src_dtype, (tok0 + t) * p.dc + c)
                             : load_any(p.k_rope, p.src_dtype, (tok0 + t) * p.dR + (c - p.dc));
    int64_t dst = row0 + t;
    if (p.block_table) {  // position len + t of sequence s in the pool (block id clamped into it)
      const int64_t pos = (int64_t)len + t;
      int64_t b = p.block_table[(int64_t)s * p.blocks_per_seq + pos / p.block_size];
      b = b < 0 ? 0 : (b >= p.pool_blocks ? p.pool_blocks - 1 : b);
      dst = b * p.block_size + pos % p.block_size;
    }
    store_any(p.kv, p.kv_dtype, dst * row + c, v);
  }

  if (p.q_rope) {
    // query j of this sequence is the token at position len + tokens - qps + j
    const int half = p.dR >> 1;
    float* const qs = p.q_rope + (int64_t)s * p.qps * p.nh * p.dR;
    const int pos_base = len + p.tokens - p.qps;
    if ((half & 3) == 0) {
      const int quads = half >> 2;
      const int nq = p.qps * p.nh * quads;
      for (int i = threadIdx.x; i < nq; i += kAppendThreads) {
        const int qr = i / quads;  // j * nh + h
        const int e = 4 * (i - qr * quads);
        int64_t pos = pos_base + qr / p.nh;
        if (p.rope_rows > 0 && pos >= p.rope_rows) pos = p.rope_rows - 1;
        f32x4* q0 = reinterpret_cast<f32x4*>(qs + (int64_t)qr * p.dR + e);
        f32x4* q1 = reinterpret_cast<f32x4*>(qs + (int64_t)qr * p.dR + e + half);
        const f32x4 x = *q0, y = *q1;
        const f32x4 cs = *reinterpret_cast<const f32x4*>(p.rope_cos + pos * half + e);
        const f32x4 sn = *reinterpret_cast<const f32x4*>(p.rope_sin + pos * half + e);
        *q0 = x * cs - y * sn;
        *q1 = x * sn + y * cs;
      }
    } else {
      const int nq = p.qps * p.nh * half;
      for (int i = threadIdx.x; i < nq; i += kAppendThreads) {
        const int qr = i / half;
        const int e = i - qr * half;
        int64_t pos = pos_base + qr / p.nh;
        if (p.rope_rows > 0 && pos >= p.rope_rows) pos = p.rope_rows - 1;
        float* q = qs + (int64_t)qr * p.dR;
        const float x = q[e], y = q[e + half];
        const float cs = p.rope_cos[pos * half + e], sn = p.rope_sin[pos * half + e];
        q[e] = x * cs - y * sn;
        q[e + half] = x * sn + y * cs;
      }
    }
  }
  __syncthreads();
  if (threadIdx.x == 0) p.lens[s] = len + p.tokens;
}

}  // namespace

hipError_t launch_append(const AppendProblem& p, hipStream_t stream) {
  if (p.num_seqs == 0) return hipSuccess;
  hipLaunchKernelGGL(append_kernel, dim3((unsigned)p.num_seqs), dim3(kAppendThreads), 0, stream, p);
  return hipGetLastError();
}

}  // namespace la
