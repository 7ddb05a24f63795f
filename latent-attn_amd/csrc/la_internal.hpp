// Internal types shared by the HIP kernels and the C-ABI layer of
// liblatent_attn_hip.so. Not installed; the public ABI is include/latent_attn.h.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_bf16.h>
#include <hip/hip_fp16.h>
#include <cstddef>
#include <cstdint>

#include "latent_attn.h"

namespace la {

// log2(e): scores are kept in base-2 units so the softmax uses v_exp_f32 (2^x).
constexpr float kLog2e = 1.4426950408889634f;

// One decode step, fully resolved on the host. Passed to kernels by value.
//
// Sequences: sequence s owns rows [seq_begin(s), seq_begin(s+1)) of the packed
// cache; RoPE positions are row - seq_begin(s). Each sequence carries Hq query
// heads = queries_per_seq * nh; query row (s, hq) reads q_abs[(s*Hq + hq)*dc].
//
// Split-KV plan: the flat row space is cut into num_chunks chunks of
// chunk_len rows. The piece of chunk c that falls in sequence s is one
// "segment"; it writes partial slot (c + s): part_o[(slot*Hq + hq)*dc + i]
// (normalised by its own softmax sum) and part_lse[slot*Hq + hq] (base-2
// log-sum-exp of the scaled scores). Slots are unique because a sequence's
// chunks form a contiguous range that starts no earlier than where the
// previous sequence's range ends; num_slots = num_chunks + num_seqs - 1.
// q_prep layout of the MFMA path ("operand order"). The query rows of each
// sequence are padded to a multiple of 32 (qprep_rows_per_seq) and cut into
// blocks of 32 rows (qrow = s * qprep_rows_per_seq(Hq) + hq). Block b stores,
// for k-step kk (16 elements of the 576-element row) and lane l = r + 32 g,
// the 8 elements Q[32 b + r][16 kk + 8 g .. +8] at element 512 kk + 8 l: the
// attention kernel's B operand of k-step kk is one coalesced 1 KB load.
constexpr int kQPrepRow = 576;  // kv_lora_rank 512 + qk_rope_head_dim 64
__host__ __device__ inline int qprep_rows_per_seq(int Hq) { return (Hq + 31) & ~31; }
__host__ __device__ inline int64_t qprep_index(int64_t qrow, int c) {
  return (qrow >> 5) * (32 * kQPrepRow) + 512 * (c >> 4) + 8 * ((qrow & 31) + 32 * ((c >> 3) & 1)) + (c & 7);
}

struct DecodeProblem {
  const void* kv;
  int kv_dtype;
  int row_elems;  // dc + dR
  int64_t total_rows;
  int num_seqs;
  int seq_len;            // used when offsets == nullptr
  const int32_t* offsets; // device, num_seqs + 1, or nullptr
  const int32_t* lens;    // device, num_seqs, or nullptr: filled rows of each region
  // paged cache (block_table != nullptr): kv is a pool of pool_blocks blocks
  // of block_size rows; the row space above is virtual (sequence s owns
  // [s * seq_len, (s+1) * seq_len), seq_len = blocks_per_seq * block_size),
  // position pos of sequence s lives in pool row paged_row(p, s, pos)
  const int32_t* block_table;  // device, num_seqs * blocks_per_seq
  int block_size;
  int blocks_per_seq;
  int64_t pool_blocks;
  // paged MFMA kernel (block_size % 32 == 0): 32-row tiles per block and the
  // multiplier that divides by it, q / tile_per_block = (mulhi(q, tpb_magic)
  // + q) >> tpb_shift for q < 2^31 (set by set_tile_divisor); pool_last =
  // pool_blocks - 1, capped at INT32_MAX (table entries are int32)
  uint32_t tile_per_block, tpb_magic;
  int tpb_shift;
  int pool_last;
  int qps;                // query tokens per sequence
  int nh;                 // weight heads
  int Hq;                 // query heads per sequence = qps * nh
  const float* q_abs;     // (num_seqs*Hq, dc) f32
  const float* q_rope;    // (num_seqs*Hq, dR) f32
  void* q_prep;           // MFMA path: [q_abs | q_rope] * scale_log2 in the MFMAs' 16-bit
                          // type, operand-order layout (qprep_index), written by
                          // launch_prep_q or the absorb kernel
  const void* W_UV;
  int wuv_dtype;
  const float* rope_cos;
  const float* rope_sin;
  int64_t rope_rows;      // 0 = unchecked
  float* out;             // (num_seqs*Hq, dv)
  int dc, dR, dv;
  float scale_log2;       // softmax scale * log2(e)
  // plan
  int chunk_len;
  int num_chunks;
  int num_slots;
  float* part_o;       // fp32 rows O / l, or (part_f16) fp16 rows, see below
  float* part_lse;     // base-2 log-sum-exp m + log2(l) of the slot's scores
  // part_f16 (MFMA kernel): part_o row (slot, hq) holds the unnormalised
  // numerator N = sum_pos 2^(s_pos - m) V_pos as fp16 N * 2^-e, with e chosen
  // per half row (columns 0..255, 256..511) so every value is below 1;
  // part_scale[2 row + half] = 2^e and part_m[row] = m. O / l = N / l with
  // 1 / l = 2^(m - lse).
  int part_f16;
  float* part_scale;
  float* part_m;
};

// One scalar load from each 64-B scalar-cache line of a DecodeProblem kernel
// argument (fields at 0x1c, 0x60, 0xa0 and 0xc4 of the 248-B struct; the
// int after it shares the last line), issued together at kernel start. The
// compiler loads every other field where it is first used, after branches on
// earlier ones; at kernel start the lines are cold, so each such round costs
// a full memory round trip (about 700 cycles), and the attention kernel's
// prologue took six of them before its first copy went out. With the lines
// warmed in one round, those loads hit the scalar cache.
__device__ inline void warm_kernarg_lines(const DecodeProblem& p) {
  asm volatile("" ::"s"(p.seq_len), "s"(p.Hq), "s"(p.rope_rows), "s"(p.num_chunks));
}
static_assert(offsetof(DecodeProblem, seq_len) < 64 && offsetof(DecodeProblem, Hq) / 64 == 1 &&
                  offsetof(DecodeProblem, rope_rows) / 64 == 2 && offsetof(DecodeProblem, num_chunks) / 64 == 3 &&
                  sizeof(DecodeProblem) + 4 <= 256,
              "warm_kernarg_lines touches every 64-B line of the arguments");

// Partial row (slot, hq) element i as fp32 O / l.
__device__ inline float load_part(const DecodeProblem& p, int64_t row, int i) {
  if (p.part_f16)
    return (float)reinterpret_cast<const _Float16*>(p.part_o)[row * p.dc + i] * p.part_scale[2 * row + (i >= 256)] *
           exp2f(p.part_m[row] - p.part_lse[row]);
  return p.part_o[row * p.dc + i];
}

// First row of sequence s, clamped into [0, total_rows] so that malformed
// offsets can give wrong answers but never out-of-bounds reads.
__device__ inline int64_t seq_begin(const DecodeProblem& p, int s) {
  const int64_t b = p.offsets ? (int64_t)p.offsets[s] : (int64_t)s * p.seq_len;
  return b < 0 ? 0 : (b > p.total_rows ? p.total_rows : b);
}

// End of sequence s's rows: the end of its region, or, with per-sequence
// lengths, its first row plus its length clamped into the region (the rows
// past it are unfilled capacity and belong to no sequence).
__device__ inline int64_t seq_end(const DecodeProblem& p, int s) {
  const int64_t region_end = seq_begin(p, s + 1);
  if (!p.lens) return region_end;
  const int64_t b = seq_begin(p, s);
  const int64_t l = p.lens[s];
  return l <= 0 ? b : (b + l < region_end ? b + l : region_end);
}

// Division by an invariant d >= 1 with a multiply (Granlund & Montgomery,
// "Division by invariant integers using multiplication", PLDI 1994, the
// round-up multiplier): l = ceil(log2 d), m = floor(2^32 (2^l - d) / d) + 1,
// then q / d = (floor(q m / 2^32) + q) >> l for every q < 2^31 (the sum fits
// in 32 bits there).
inline void set_tile_divisor(DecodeProblem& p, uint32_t d) {
  int l = 0;
  while ((1ull << l) < d) ++l;
  p.tile_per_block = d;
  p.tpb_shift = l;
  p.tpb_magic = (uint32_t)((((1ull << l) - d) << 32) / d + 1);
}

// Pool row of position pos of sequence s in a paged cache. Block ids are
// clamped into the pool: a malformed table gives wrong rows, never an
// out-of-bounds access. Requires pos < blocks_per_seq * block_size.
__device__ inline int64_t paged_row(const DecodeProblem& p, int s, int64_t pos) {
  int64_t b = p.block_table[(int64_t)s * p.blocks_per_seq + pos / p.block_size];
  b = b < 0 ? 0 : (b >= p.pool_blocks ? p.pool_blocks - 1 : b);
  return b * p.block_size + pos % p.block_size;
}

// RoPE table row of in-sequence position pos.
__device__ inline int64_t rope_row(const DecodeProblem& p, int64_t pos) {
  return (p.rope_rows > 0 && pos >= p.rope_rows) ? p.rope_rows - 1 : pos;
}

// Sequence whose row range contains row r: the largest s with
// seq_begin(s) <= r (empty sequences are skipped because their successor has
// the same begin). Requires seq_begin(0) <= r < seq_begin(num_seqs).
__device__ inline int find_seq(const DecodeProblem& p, int64_t r) {
  if (!p.offsets) return (int)(r / p.seq_len);
  int lo = 0, hi = p.num_seqs - 1;
  while (lo < hi) {
    int mid = (lo + hi + 1) >> 1;
    if ((int64_t)p.offsets[mid] <= r) lo = mid;
    else hi = mid - 1;
  }
  return lo;
}

// OCP FP8 E4M3 (e4m3fn) latent-cache element: sign, 4 exponent bits (bias
// 7), 3 mantissa bits; exponent 0 is subnormal (m * 2^-9), 0x7F / 0xFF NaN.
struct fp8e4m3 {
  uint8_t bits;
};
__device__ inline float fp8_to_f32(uint32_t c) {
  const uint32_t e = (c >> 3) & 15, m = c & 7;
  float v;
  if (e == 15 && m == 7) v = __builtin_nanf("");
  else if (e == 0) v = (float)m * 0x1p-9f;
  else v = __builtin_amdgcn_ldexpf(1.f + (float)m * 0.125f, (int)e - 7);
  return (c & 0x80) ? -v : v;
}
// Round to nearest even, saturating at +-448 (the largest finite value);
// NaN stays NaN.
__device__ inline uint8_t f32_to_fp8(float x) {
  const uint32_t b = __builtin_bit_cast(uint32_t, x);
  const uint32_t s = (b >> 24) & 0x80;
  const float a = __builtin_fabsf(x);
  if (a != a) return (uint8_t)(s | 0x7F);
  if (a >= 448.f) return (uint8_t)(s | 0x7E);
  if (a < 0x1p-6f) return (uint8_t)(s | (uint32_t)__builtin_rintf(a * 512.f));  // subnormal; 8 = 2^-6
  const uint32_t ab = __builtin_bit_cast(uint32_t, a);
  uint32_t e = ((ab >> 23) & 0xFF) - 127 + 7;  // 1 .. 15
  uint32_t m = (ab >> 20) & 7;
  const uint32_t rem = ab & 0xFFFFF;
  if (rem > 0x80000 || (rem == 0x80000 && (m & 1))) ++m;
  if (m == 8) {
    m = 0;
    ++e;
  }
  const uint32_t c = (e << 3) | m;
  return (uint8_t)(s | (c > 0x7E ? 0x7E : c));
}

template <typename T>
__device__ inline float to_f32(T v);
template <>
__device__ inline float to_f32<float>(float v) { return v; }
template <>
__device__ inline float to_f32<__half>(__half v) { return __half2float(v); }
template <>
__device__ inline float to_f32<__hip_bfloat16>(__hip_bfloat16 v) { return __bfloat162float(v); }
template <>
__device__ inline float to_f32<fp8e4m3>(fp8e4m3 v) { return fp8_to_f32(v.bits); }

// Load element i of a weight matrix whose dtype is only known at run time
// (uniform across the launch, so the switch does not diverge).
__device__ inline float load_any(const void* base, int dtype, int64_t i) {
  if (dtype == LA_DTYPE_BF16) return __bfloat162float(reinterpret_cast<const __hip_bfloat16*>(base)[i]);
  if (dtype == LA_DTYPE_F16) return __half2float(reinterpret_cast<const __half*>(base)[i]);
  if (dtype == LA_DTYPE_FP8_E4M3) return fp8_to_f32(reinterpret_cast<const uint8_t*>(base)[i]);
  return reinterpret_cast<const float*>(base)[i];
}

__device__ inline float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

__device__ inline float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// One la_append_kv call, resolved on the host (la_append.hip).
struct AppendProblem {
  void* kv;
  int kv_dtype;
  int64_t total_rows;
  int num_seqs;
  int capacity;            // region rows per sequence when offsets == nullptr
  const int32_t* offsets;  // device, num_seqs + 1, or nullptr
  int32_t* lens;           // device, num_seqs
  int tokens;
  const void* c_t;
  const void* k_rope;
  int src_dtype;
  float* q_rope;           // nullptr = no query rotation
  int qps;
  int nh;
  const float* rope_cos;
  const float* rope_sin;
  int64_t rope_rows;
  int32_t* status;
  int dc, dR;
  // paged cache (block_table != nullptr): as in DecodeProblem; capacity =
  // blocks_per_seq * block_size, kv a pool of pool_blocks blocks
  const int32_t* block_table;
  int block_size;
  int blocks_per_seq;
  int64_t pool_blocks;
};

// One la_naive_mla call (la_naive.hip): a single query over one cache.
struct NaiveProblem {
  const void* kv;
  int kv_dtype;
  int S;
  const void* W_UK;
  int wuk_dtype;
  const void* W_UV;
  int wuv_dtype;
  const float* q_nope;
  const float* q_rope;
  const float* rope_cos;
  const float* rope_sin;
  int64_t rope_rows;
  float* out;
  int nh, dn, dR, dc, dv;
  float scale;
  float* Kn;      // workspace: (S, nh*dn) fp32
  float* V;       // workspace: (S, nh*dv) fp32
  float* scores;  // workspace: (nh, S) fp32
};

// ---- host launchers (one per kernel family) -------------------------------

// Decompress-then-attend (la_naive.hip).
size_t naive_workspace_bytes(int64_t S, int nh, int dn, int dv);
hipError_t launch_naive(NaiveProblem p, void* workspace, hipStream_t stream);

// Device-side cache append + query RoPE.
hipError_t launch_append(const AppendProblem& p, hipStream_t stream);

// VALU split-KV decode: any dtype, kv_lora_rank <= 1024, qk_rope_head_dim <= 256.
hipError_t launch_decode_generic(const DecodeProblem& p, hipStream_t stream);
bool generic_supported(const DecodeProblem& p);

// MFMA split-KV decode for 16-bit and FP8 E4M3 caches with kv_lora_rank 512,
// qk_rope_head_dim 64.
// ev_begin / ev_end (optional) are recorded at the kernel's start and end.
hipError_t launch_decode_mfma(const DecodeProblem& p, hipStream_t stream, hipEvent_t ev_begin = nullptr,
                              hipEvent_t ev_end = nullptr);
bool mfma_supported(const DecodeProblem& p);
// The attention kernel's grid and copy schedule with no compute (a
// streaming-ceiling measurement); ring = 3 or 4 tile buffers. 16-bit
// contiguous caches.
hipError_t launch_stream_copies(const DecodeProblem& p, int ring, hipStream_t stream);
int mfma_heads_per_group();
int mfma_max_chunk_rows();
// Fills p.q_prep from p.q_abs and p.q_rope (MFMA path only).
// zero_out (optional): zero_n floats zeroed for a latent-half merge.
hipError_t launch_prep_q(const DecodeProblem& p, hipStream_t stream, float* zero_out = nullptr, int64_t zero_n = 0);

// log-sum-exp combine of the partial slots + W_UV projection into p.out.
hipError_t launch_combine_project(const DecodeProblem& p, hipStream_t stream);

// MFMA versions for 16-bit weights (la_proj.hip).
bool absorb_mfma_supported(int w_dtype, int nh, int dn, int dc);
// out_mode 0: out = q_abs (fp32). 1 / 2: out = q_prep (bf16 / fp16) =
// [q_abs | q_rope] * scale in the operand-order layout, as prep_q_kernel
// writes it; token t is query t % qps of sequence t / qps (qps = tokens per
// sequence, used by modes 1 / 2 only).
// zero_out (optional): zero_n floats the kernel zeroes, for a merge that adds
// its latent halves into the output.
hipError_t launch_absorb_mfma(const float* q_nope, const void* W_UK, int w_dtype, void* out, int out_mode,
                              const float* q_rope, float scale, int dR, int tokens, int nh, int dn, int dc, int qps,
                              hipStream_t stream, float* zero_out = nullptr, int64_t zero_n = 0);
bool project_mfma_supported(const DecodeProblem& p);
// Workgroups of the full-row merge + projection launch.
int merge_project_blocks(const DecodeProblem& p);
// Merge of the split partials and W_UV projection in one kernel (the merged
// rows stay in LDS: no workspace). halves: one workgroup per latent half,
// which adds its product into p.out with atomics: p.out must be zero (fp16
// partials only).
hipError_t launch_combine_project_mfma(const DecodeProblem& p, hipStream_t stream, bool halves = false);

// q_abs = q_nope . W_UK per head.
hipError_t launch_absorb(const float* q_nope, const void* W_UK, int w_dtype, float* q_abs, int tokens, int nh, int dn,
                         int dc, hipStream_t stream);

}  // namespace la
