// MFMA kernels for the two small contractions around the attention kernel,
// for 16-bit weights (bf16 or fp16):
//
//   absorb:   q_abs[t,h,c] = sum_i q_nope[t,h,i] * W_UK[h*dn + i, c]
//             (reference tests/test_correctness.cu:29-46, tests/test_python.py:97-99)
//   project:  out[t,h,j]   = sum_c O[t,h,c] * W_UV[h*dv + j, c], where O is the
//             log-sum-exp merge of the split-KV partial slots
//             (reference src/fused_mla.cu:255-267: normalise, then W_UV)
//
// absorb runs v_mfma_f32_32x32x16 with 32 query tokens as M, the projection
// v_mfma_f32_16x16x32 with 16 query rows as M. The fp32 operand (q_nope, or
// the merged O) is split into a 16-bit high part and a 16-bit residual
// (hi = rn(x), lo = rn(x - hi)); two MFMAs accumulate W*hi + W*lo in fp32, so
// the result keeps ~16 bits of the fp32 operand instead of 8 (bf16) or 11
// (fp16). For fp16 the residual is pre-multiplied by 2^11 (and its product by
// 2^-11) so it stays in the normal range.
//
// absorb:  one block of 512 threads per (32-token block, head, 128-column
//          block), XCD-ordered; all 8 waves load W_UK[h][:, 128-col block]
//          (128 x 128) into LDS and one q k-step each, then waves 0..3 run
//          the MFMAs, wave w on 32 columns; the B operand (8 consecutive
//          rows i per lane) comes from ds_read_b64_tr_b16.
// merge + project: merge_project_kernel, one block of 8 waves per (weight
//          head, 16 query rows): the log-sum-exp merge of the partial slots
//          into LDS, then the W_UV projection of the merged rows. With fewer
//          such blocks than CUs (a few query rows), merge_project_half_kernel
//          splits each over the two latent halves, which add into the output
//          (zeroed earlier in the same call by the kernel that writes the
//          attention kernel's 16-bit queries).
#include "la_internal.hpp"

#include <type_traits>

namespace la {

// Phase-timing build only (-DLA_PHASE_STAMPS, see la_mfma.hip): wave 0 of
// every block of the absorb and merge + projection kernels records the
// device's constant-rate clock (s_memrealtime, 100 MHz, common to all XCDs)
// at 6 points and writes them at exit. Absorb: 0 entry, 1 loads issued, 2
// operands in LDS, 3 past the barrier, 4 MFMAs done, 5 stores complete.
// Merge: 0 entry, 1 W_UV loads issued, 2 this wave's merge done, 3 every
// wave's merge in LDS, 4 projection done, 5 stores complete.
#ifdef LA_PHASE_STAMPS
constexpr int kSideStampBlocks = 8192;
__device__ unsigned long long g_side_stamps[2][kSideStampBlocks * 8];
#define LA_RSTAMP(i)                                                               \
  do {                                                                             \
    unsigned long long t_;                                                         \
    asm volatile("s_memrealtime %0\n\ts_waitcnt lgkmcnt(0)" : "=s"(t_)::"memory"); \
    stamps_[i] = t_;                                                               \
  } while (0)
#define LA_RSTAMP_DECL unsigned long long stamps_[8] = {}
#define LA_RSTAMP_WRITE(kind)                                                                            \
  do {                                                                                                   \
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");                                                     \
    LA_RSTAMP(5);                                                                                        \
    if (threadIdx.x == 0 && blockIdx.x < kSideStampBlocks)                                               \
      for (int i_ = 0; i_ < 6; ++i_) g_side_stamps[kind][(size_t)blockIdx.x * 8 + i_] = stamps_[i_];     \
  } while (0)
#else
#define LA_RSTAMP(i) ((void)0)
#define LA_RSTAMP_DECL ((void)0)
#define LA_RSTAMP_WRITE(kind) ((void)0)
#endif

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef short i16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void;

template <typename WT>
struct Mma;

template <>
struct Mma<__hip_bfloat16> {
  typedef bf16x8 vec;
  typedef __bf16 elem;
  static constexpr float kLoScale = 1.f;
  static __device__ inline f32x16 mma(vec a, vec b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};

template <>
struct Mma<__half> {
  typedef f16x8 vec;
  typedef _Float16 elem;
  static constexpr float kLoScale = 2048.f;  // 2^11
  static __device__ inline f32x16 mma(vec a, vec b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};

// hi/lo split of 8 fp32 values into two 16-bit operand vectors.
template <typename WT>
__device__ inline void split8(const float* x, typename Mma<WT>::vec& hi, typename Mma<WT>::vec& lo) {
  typedef typename Mma<WT>::elem E;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const E h = (E)x[e];
    hi[e] = h;
    lo[e] = (E)((x[e] - (float)h) * Mma<WT>::kLoScale);
  }
}

// ---------------------------------------------------------------------------
// absorb
// ---------------------------------------------------------------------------
constexpr int kAbsCols = 128;            // columns per block
constexpr int kAbsRowBytes = 256 + 32;   // 128 x 16-bit + pad: 4 tr rows hit 4 bank groups
// Threads per block: 8 waves share the loads (6-8 per wave instead of 14
// with 4 waves; a wave stalls its issue once about a dozen loads are in
// flight), 4 of them run the MFMAs. Config 3: 6.6 us per dispatch against
// 6.8 with 4 waves.
constexpr int kAbsThreads = 512;

// out_mode 0: q_abs (fp32, (T*nh, dc)). out_mode 1 / 2: q_prep rows (bf16 /
// fp16, (T*nh, dc + dR)) = [q_abs | q_rope] * scale for the MFMA attention
// kernel; blocks with cb == 0 also convert the q_rope part of their rows.
// All global loads (q_nope for every k-step, the W_UK tile) are issued before
// the first wait, spread over the block's 8 waves.
// NKS = dn / 16 when known at compile time (8 for dn = 128: no guards, every
// load unconditional), 0 for any dn <= 128 that is a multiple of 16.
template <typename WT, int NKS>
__global__ __launch_bounds__(kAbsThreads) void absorb_mfma_kernel(const float* __restrict__ q_nope, const WT* __restrict__ W,
                                                          void* __restrict__ out, int out_mode,
                                                          const float* __restrict__ q_rope, float scale, int dR,
                                                          int tokens, int nh, int dn, int dc, int qps,
                                                          float* __restrict__ zero_out, int64_t zero_n) {
  typedef Mma<WT> M;
  typedef typename M::vec vec;
  LA_RSTAMP_DECL;
  LA_RSTAMP(0);
  // both 64-B scalar-cache lines of the arguments in one round of loads (see
  // warm_kernarg_lines)
  asm volatile("" ::"s"(tokens), "s"(qps));
  __shared__ __attribute__((aligned(16))) char wt[128 * kAbsRowBytes];  // dn <= 128 rows
  // q operands (hi, lo) of the 8 k-steps, shared by the 4 waves: [ks][hi|lo][lane] 16 B
  __shared__ __attribute__((aligned(16))) char qs[8 * 2 * 64 * 16];
  // Block id -> (token block tb, head h, column block cb). A 128-B q_prep
  // line gathers the 16-B slots of 8 consecutive heads (same token and
  // k-step), and the ncb column blocks of a head read the same q_nope rows,
  // so all blocks of one (tb, 8-head group) run on one XCD (blocks go to XCDs
  // round-robin by id % 8): their slots meet in that XCD's L2 instead of
  // leaving it as partial lines, and q_nope is fetched once per head.
  const int ncb = dc / kAbsCols, nh8 = (nh + 7) / 8, gb = 8 * ncb;
  const int x = blockIdx.x & 7, k = blockIdx.x >> 3;
  const int grp = x + 8 * (k / gb), j = k % gb;  // (tb, 8-head group) group, block j in it
  const int tb = grp / nh8;
  const int h = 8 * (grp - tb * nh8) + (j & 7), cb = j >> 3, t0 = tb * 32;
  // zero_out: the decode output, which a latent-half merge adds into (every
  // block, before its early return, zeroes a grid-stride share)
  if (zero_out)
    for (int64_t i = (int64_t)blockIdx.x * kAbsThreads + threadIdx.x; i < zero_n; i += (int64_t)gridDim.x * kAbsThreads)
      zero_out[i] = 0.f;
  if (t0 >= tokens || h >= nh) return;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int nks = NKS > 0 ? NKS : dn / 16;  // <= 8
  if (NKS > 0) dn = 16 * NKS;

  // q_nope of token t0 + lane%32, elements 16ks + 8(lane/32) .. +8: wave w
  // loads k-step w, splits it into hi/lo 16-bit operands and stages them in
  // LDS for the MFMA waves (each wave issues 2 q loads, not 16)
  const int t = t0 + (lane & 31);
  const bool tvalid = t < tokens;
  const float* qrow = q_nope + ((int64_t)(tvalid ? t : 0) * nh + h) * dn + 8 * (lane >> 5);
  // (with NKS > 0 every wave's k-step exists: the loads go out
  // unconditionally, since a load under a branch gets its result copied at
  // the branch's end, which waits for it before the W_UK loads below issue)
  static_assert(kAbsThreads / 64 == 8, "one q k-step per wave");
  const int ks_w = wave;
  f32x4 qa, qb;
  if (NKS > 0 || ks_w < nks) {
    qa = *reinterpret_cast<const f32x4*>(qrow + 16 * ks_w);
    qb = *reinterpret_cast<const f32x4*>(qrow + 16 * ks_w + 4);
  }
  // W_UK[h*dn + i][cb*128 + 0..127] for i < dn, 16 B per thread-load
  constexpr int kWLoads = 128 * 16 / kAbsThreads;
  i16x8 wv[kWLoads];
#pragma unroll
  for (int k = 0; k < kWLoads; ++k) {
    const int q = tid + kAbsThreads * k;
    if (NKS > 0 || q < dn * 16)
      wv[k] = *reinterpret_cast<const i16x8*>(W + ((int64_t)h * dn + (q >> 4)) * dc + cb * kAbsCols + (q & 15) * 8);
  }
  // q_rope rows of the block's tokens for the q_prep rows' rope part, written
  // by the column block 0 of each head: 32 tokens x 64 = one 32-B piece per
  // MFMA-wave thread (dc + dR = 576 on this path, so dR = 64). Loaded here
  // with the operands, so the tail after the MFMAs is one store, not a load
  // round trip; by every block (the other column blocks of the head read the
  // same lines from the XCD's L2) and unconditionally (without q_rope,
  // out_mode 0, from q_nope instead, unused; waves 4..7 repeat waves 0..3's
  // pieces), since a load under a branch gets its result copied at the
  // branch's end, which would wait for every load before it.
  const int rt = tid & 255;
  const int rtr = min(t0 + (rt >> 3), tokens - 1);
  const float* rsrc = out_mode != 0 ? q_rope + ((int64_t)rtr * nh + h) * dR + 8 * (rt & 7) : q_nope;
  const f32x4 ra = *reinterpret_cast<const f32x4*>(rsrc);
  const f32x4 rb = *reinterpret_cast<const f32x4*>(rsrc + 4);
  LA_RSTAMP(1);
#pragma unroll
  for (int k = 0; k < kWLoads; ++k) {
    const int q = tid + kAbsThreads * k;
    if (NKS > 0 || q < dn * 16) *reinterpret_cast<i16x8*>(wt + (q >> 4) * kAbsRowBytes + (q & 15) * 16) = wv[k];
  }
  if (NKS > 0 || ks_w < nks) {
    float x[8];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      x[e] = tvalid ? qa[e] : 0.f;
      x[4 + e] = tvalid ? qb[e] : 0.f;
    }
    vec hi, lo;
    split8<WT>(x, hi, lo);
    *reinterpret_cast<vec*>(qs + (2 * ks_w) * 1024 + 16 * lane) = hi;
    *reinterpret_cast<vec*>(qs + (2 * ks_w + 1) * 1024 + 16 * lane) = lo;
  }
  LA_RSTAMP(2);
  __syncthreads();
  LA_RSTAMP(3);
  if (wave >= 4) return;  // the loading-only waves are done (no barrier follows)

  f32x16 acc_hi = {}, acc_lo = {};
  const int g = lane >> 4, s = lane & 15;
#pragma unroll
  for (int ks = 0; ks < 8; ++ks) {
    if (NKS > 0 ? ks >= NKS : ks >= nks) break;
    const vec ahi = *reinterpret_cast<const vec*>(qs + (2 * ks) * 1024 + 16 * lane);
    const vec alo = *reinterpret_cast<const vec*>(qs + (2 * ks + 1) * 1024 + 16 * lane);
    // B[k = i][n = c]: rows 16ks + 8(g>>1) + 4hf + (s>>2), columns 32w + 16(g&1) + 4(s&3)
    i16x8 bv;
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      const int row = 16 * ks + 8 * (g >> 1) + 4 * hf + (s >> 2);
      const int col = 32 * wave + 16 * (g & 1) + 4 * (s & 3);
      const i16x4 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (__attribute__((address_space(3))) i16x4*)(lds_void*)(wt + row * kAbsRowBytes + col * 2));
#pragma unroll
      for (int e = 0; e < 4; ++e) bv[4 * hf + e] = r[e];
    }
    const vec b = __builtin_bit_cast(vec, bv);
    // D^T = W^T . q^T: the W tile is the A operand (lane = column), q the B
    // operand (lane = token), so each lane ends up with runs of 4 columns
    acc_hi = M::mma(b, ahi, acc_hi);
    acc_lo = M::mma(b, alo, acc_lo);
  }
  LA_RSTAMP(4);
  // D^T[m = column][n = token]: register 4q + r holds column 32w + 8q + 4(lane/32) + r
  // of token t0 + lane%32, so one 16-byte (fp32) or 8-byte (16-bit) store per q.
  const int tt = t0 + (lane & 31);
  if (tt < tokens) {
    const int col0 = cb * kAbsCols + 32 * wave + 4 * (lane >> 5);
    // q_prep row of token tt: query tt % qps of sequence tt / qps, weight head h
    const int64_t qrow = out_mode != 0 ? (int64_t)(tt / qps) * qprep_rows_per_seq(qps * nh) + (tt % qps) * nh + h : 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      f32x4 v;
#pragma unroll
      for (int r = 0; r < 4; ++r) v[r] = acc_hi[4 * q + r] + acc_lo[4 * q + r] * (1.f / M::kLoScale);
      const int col = col0 + 8 * q;
      if (out_mode == 0) {
        *reinterpret_cast<f32x4*>(reinterpret_cast<float*>(out) + ((int64_t)tt * nh + h) * dc + col) = v;
      } else if (out_mode == 1) {
        bf16x4 o;
#pragma unroll
        for (int r = 0; r < 4; ++r) o[r] = (__bf16)(v[r] * scale);
        *reinterpret_cast<bf16x4*>(reinterpret_cast<__bf16*>(out) + qprep_index(qrow, col)) = o;
      } else {
        f16x4 o;
#pragma unroll
        for (int r = 0; r < 4; ++r) o[r] = (_Float16)(v[r] * scale);
        *reinterpret_cast<f16x4*>(reinterpret_cast<_Float16*>(out) + qprep_index(qrow, col)) = o;
      }
    }
  }
  if (out_mode != 0 && cb == 0) {
    // the q_rope part of the same rows (loaded with the operands above): one
    // 16-B slot of q_prep per thread
    const int tr = t0 + (tid >> 3), j = 8 * (tid & 7);
    if (tr < tokens) {
      const int64_t qr = (int64_t)(tr / qps) * qprep_rows_per_seq(qps * nh) + (int64_t)(tr % qps) * nh + h;
      const int64_t dst = qprep_index(qr, dc + j);
      if (out_mode == 1) {
        bf16x8 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          v[e] = (__bf16)(ra[e] * scale);
          v[4 + e] = (__bf16)(rb[e] * scale);
        }
        *reinterpret_cast<bf16x8*>(reinterpret_cast<__bf16*>(out) + dst) = v;
      } else {
        f16x8 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          v[e] = (_Float16)(ra[e] * scale);
          v[4 + e] = (_Float16)(rb[e] * scale);
        }
        *reinterpret_cast<f16x8*>(reinterpret_cast<_Float16*>(out) + dst) = v;
      }
    }
  }
  LA_RSTAMP_WRITE(0);
}

// ---------------------------------------------------------------------------
// combine + project
// ---------------------------------------------------------------------------
constexpr int kDcP = 512;
constexpr int kMPRows = 16;  // query rows per merge + projection workgroup

typedef float f32x4v __attribute__((ext_vector_type(4)));

template <typename WT>
struct Mma16;
template <>
struct Mma16<__hip_bfloat16> {
  typedef bf16x8 vec;
  static __device__ inline f32x4 mma(vec a, vec b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};
template <>
struct Mma16<__half> {
  typedef f16x8 vec;
  static __device__ inline f32x4 mma(vec a, vec b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};

// One slot's 8 columns of this lane, kept in the stored format until use
// (fp16 numerator rows: before their row scale, which the slot weight
// carries), so 8 slots in flight cost 32 VGPRs for fp16 rows.
template <bool F16>
struct SlotRow;
template <>
struct SlotRow<true> {
  f16x8 h;
  __device__ void load(const void* rowp) { h = *reinterpret_cast<const f16x8*>(rowp); }
  __device__ void fma(float w, f32x4& o0, f32x4& o1) const {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      o0[e] += w * (float)h[e];
      o1[e] += w * (float)h[4 + e];
    }
  }
};
template <>
struct SlotRow<false> {
  f32x4 a, b;
  __device__ void load(const void* rowp) {
    a = *reinterpret_cast<const f32x4*>(rowp);
    b = *reinterpret_cast<const f32x4*>(reinterpret_cast<const float*>(rowp) + 4);
  }
  __device__ void fma(float w, f32x4& o0, f32x4& o1) const {
    o0 += w * a;
    o1 += w * b;
  }
};

// One fp16 slot's 4 columns of this lane (half-row merge).
struct SlotRowHalf {
  f16x4 h;
  __device__ void load(const void* rowp) { h = *reinterpret_cast<const f16x4*>(rowp); }
  __device__ void fma(float w, f32x4& o0, f32x4&) const {
#pragma unroll
    for (int e = 0; e < 4; ++e) o0[e] += w * (float)h[e];
  }
};

// Log-sum-exp merge of split partial slots:
//   O = sum_s 2^(lse_s - M) (O/l)_s / sum_s 2^(lse_s - M),  M = max_s lse_s.
// F16 (MFMA attention kernel): slot rows hold the numerator N_s = sum 2^(s-m_s) V
// as fp16 N_s 2^-e per half row, so (O/l)_s 2^(lse_s - M) = N_s 2^(m_s - M) 2^e.
// F32 (VALU attention kernel): slot rows hold O/l in fp32.
//
// A merge task is (query row t, slot group g of G): it adds the slots
// s = g, g + G, g + 2G, ... of row t, each weighted and divided by the sum
// over ALL slots of the row, into this lane's 8 latent columns 8 lane ..
// 8 lane + 7 (one wave per task), so the G tasks of a row sum to its merged O.
// A half-row merge (fp16 slots) covers only the latent half c: 4 columns
// 256 c + 4 lane .. +3 per lane, weighted with that half's row scale.
// Rows past the batch and empty sequences give 0.
struct MergeTask {
  int n = 0;       // slots of the row
  int ns = 0;      // slots of this task (g, g + G, ...)
  int64_t row0 = 0;  // partial row of the row's first slot
};

__device__ inline MergeTask merge_task(const DecodeProblem& p, int t, int h, int g, int G) {
  MergeTask m;
  if (t < 0 || t >= p.num_seqs * p.qps) return m;
  const int s = t / p.qps;
  const int hq = (t % p.qps) * p.nh + h;
  const int64_t lo = seq_begin(p, s), hi = seq_end(p, s);
  if (hi <= lo) return m;
  const int64_t cf = lo / p.chunk_len;
  m.n = (int)((hi - 1) / p.chunk_len - cf + 1);  // slots cf+s .. cf+s+n-1
  m.ns = m.n > g ? (m.n - g + G - 1) / G : 0;
  m.row0 = (cf + s) * p.Hq + hq;
  return m;
}

// Merges up to two tasks (t[1] < 0: one) of the same slot group g of G.
// Every load of both tasks goes out before anything waits: the first NB slot
// rows of each task, each row's log-sum-exps (lane i: slot i, for the
// maximum and the denominator) and the weights' inputs of the task's own
// slots (lane i: slot g + G i), so a merge of up to NB own slots out of at
// most 64 takes one memory round trip. Longer merges loop over further
// groups of NB rows (and of 64 slots). Lane i's weights are broadcast with
// v_readlane.
// kHalf: half-row merge of latent half c (o[k][1] stays 0).
template <bool F16, bool kHalf, int NB>
__device__ inline void merge_tasks(const DecodeProblem& p, const int (&t)[2], int h, int g, int G, int lane,
                                   f32x4 (&o)[2][2], int c = 0) {
  static_assert(F16 || !kHalf, "half-row merges read fp16 slots");
  typedef typename std::conditional<F16, _Float16, float>::type PT;
  typedef typename std::conditional<kHalf, SlotRowHalf, SlotRow<F16>>::type SR;
  const int64_t sstride = (int64_t)p.Hq * kDcP;
  static_assert(NB >= 1 && NB <= 64, "slot rows per batch");
  MergeTask mt[2];
  const PT* src[2];
  SR d[2][NB];
  float ls_all[2], ls_own[2], m_own[2], sa_own[2], sb_own[2];
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    mt[k] = merge_task(p, t[k], h, g, G);
    src[k] = reinterpret_cast<const PT*>(p.part_o) + mt[k].row0 * kDcP + (kHalf ? 256 * c + 4 * lane : 8 * lane);
#pragma unroll
    for (int u = 0; u < NB; ++u)
      if (u < mt[k].ns) d[k][u].load(src[k] + (int64_t)(g + G * u) * sstride);
  }
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const float* lse = p.part_lse + mt[k].row0;
    ls_all[k] = lane < mt[k].n ? lse[(int64_t)lane * p.Hq] : -INFINITY;
    const bool own = lane < mt[k].ns;
    const int64_t pr = mt[k].row0 + (int64_t)(g + G * (own ? lane : 0)) * p.Hq;
    ls_own[k] = own ? p.part_lse[pr] : -INFINITY;
    if constexpr (F16) {
      m_own[k] = own ? p.part_m[pr] : -INFINITY;
      sa_own[k] = own ? p.part_scale[2 * pr + (kHalf ? c : 0)] : 0.f;
      sb_own[k] = own ? p.part_scale[2 * pr + (kHalf ? c : 1)] : 0.f;
    }
  }
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    o[k][0] = f32x4{0.f, 0.f, 0.f, 0.f};
    o[k][1] = o[k][0];
    const int n = mt[k].n, ns = mt[k].ns;
    if (n == 0) continue;  // wave-uniform
    const float* lse = p.part_lse + mt[k].row0;
    // M and the denominator over every slot of the row
    float mx = ls_all[k];
    for (int i = lane + 64; i < n; i += 64) mx = fmaxf(mx, lse[(int64_t)i * p.Hq]);
    mx = wave_max(mx);
    float den = lane < n ? exp2f(ls_all[k] - mx) : 0.f;
    for (int i = lane + 64; i < n; i += 64) den += exp2f(lse[(int64_t)i * p.Hq] - mx);
    const float inv = 1.f / wave_sum(den);
    for (int i0 = 0; i0 < ns; i0 += 64) {
      const int nb = min(64, ns - i0);
      // this lane's slot: g + G (i0 + lane)
      float ls = ls_own[k], mm = m_own[k], sa = sa_own[k], sb = sb_own[k];
      if (i0 > 0) {
        const bool ok = lane < nb;
        const int64_t pr = mt[k].row0 + (int64_t)(g + G * (i0 + (ok ? lane : 0))) * p.Hq;
        ls = ok ? p.part_lse[pr] : -INFINITY;
        if constexpr (F16) {
          mm = ok ? p.part_m[pr] : -INFINITY;
          sa = ok ? p.part_scale[2 * pr + (kHalf ? c : 0)] : 0.f;
          sb = ok ? p.part_scale[2 * pr + (kHalf ? c : 1)] : 0.f;
        }
      }
      float wlo, whi;
      if constexpr (F16) {
        const float a = exp2f(mm - mx) * inv;  // 0 for lanes past the task's slots
        wlo = a * sa;  // columns 0..255 (lanes 0..31); half c: all lanes
        whi = a * sb;  // columns 256..511 (lanes 32..63); half c: all lanes
      } else {
        wlo = whi = exp2f(ls - mx) * inv;
      }
      for (int j = 0; j < nb; j += NB) {
        if (i0 > 0 || j > 0) {
#pragma unroll
          for (int u = 0; u < NB; ++u)
            if (j + u < nb) d[k][u].load(src[k] + (int64_t)(g + G * (i0 + j + u)) * sstride);
        }
#pragma unroll
        for (int u = 0; u < NB; ++u) {
          if (j + u < nb) {
            const float w0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wlo), j + u));
            const float w1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, whi), j + u));
            d[k][u].fma(lane < 32 ? w0 : w1, o[k][0], o[k][1]);
          }
        }
      }
    }
  }
}

// Merge + W_UV projection, one workgroup of 8 waves per (weight head h,
// block of 16 query rows):
//   1. each wave issues the loads of its W_UV operands (output columns
//      16w .. 16w+15 of head h, all 512 latent columns: 16 x 16 B per lane),
//      which stay in flight through the merge;
//   2. the merge (merge_tasks): with 8 or more rows in the block, wave w
//      merges rows w and w + 8, every slot; with fewer rows, each row's slots
//      are split over G = 8 / rows waves (slot group w % G of row w / G) and
//      the groups' sums added in LDS. Each merged fp32 element is split once
//      into a 16-bit high part and a residual (split8), which go to LDS as
//      the projection's A operands;
//   3. out[row][16w + n] = sum_c O[row][c] W_UV[h dv + 16w + n][c] on
//      v_mfma_f32_16x16x32: two MFMAs per k-step (A = the high and the low
//      rows, ~16 bits of the fp32 O; B = the W_UV rows).
// Blocks of one head run on one XCD (the dispatcher assigns id % 8 to XCDs),
// so its 128 KB of W_UV is fetched once per head.
constexpr int kMPWaves = 8;
// slot rows each task loads up front (one memory round trip for up to this
// many; more loop over further batches, a round trip each). The half-row
// merge also comes with 32 (8 B per lane each), launched when a task has
// more than 8 slots (config 5: 32): more registers cost the short merges
// (measured: configs 2 and 3 +1.5 us per step with 16 / 32 everywhere).
constexpr int kMPSlots = 8;
constexpr int kMPPitch = kDcP + 4;  // floats per LDS row of a slot-group sum
// 16-bit elements per LDS row of the high / low operand rows: 1040 B, 16 B
// past a multiple of 256, so the 16 rows one A read touches (16 lanes, one
// 16-B column each) fall on distinct banks
constexpr int kMPOPitch = kDcP + 8;

template <typename WT, bool F16>
__global__ __launch_bounds__(kMPWaves * 64) void merge_project_kernel(DecodeProblem p) {
  LA_RSTAMP_DECL;
  LA_RSTAMP(0);
  warm_kernarg_lines(p);
  typedef Mma16<WT> M;
  typedef typename M::vec vec;
  constexpr float kLoScale = Mma<WT>::kLoScale;
  __shared__ __attribute__((aligned(16))) short oh[kMPRows * kMPOPitch];      // merged O rows, high parts
  __shared__ __attribute__((aligned(16))) short ol[kMPRows * kMPOPitch];      // and residuals
  __shared__ __attribute__((aligned(16))) float gp[kMPWaves * kMPPitch];      // slot-group sums
  const int R = p.num_seqs * p.qps;
  const int nrb = (R + kMPRows - 1) / kMPRows;
  const int x = blockIdx.x & 7, k = blockIdx.x >> 3;
  const int h = (k / nrb) * 8 + x, rb = k % nrb;
  if (h >= p.nh) return;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int rows = min(kMPRows, R - rb * kMPRows);

  // W_UV operands: B[k = 32 ks + 8 (lane / 16) + j][n = lane % 16]
  //              = W_UV[h dv + 16 wave + lane % 16][32 ks + 8 (lane / 16) + j]
  const WT* wrow = reinterpret_cast<const WT*>(p.W_UV) + ((int64_t)h * p.dv + 16 * wave + (lane & 15)) * kDcP +
                   8 * (lane >> 4);
  vec bw[16];
#pragma unroll
  for (int ks = 0; ks < 16; ++ks) bw[ks] = __builtin_bit_cast(vec, *reinterpret_cast<const i16x8*>(wrow + 32 * ks));
  LA_RSTAMP(1);

  // row r, columns c0 .. c0 + 7 of O -> high and low operand rows
  auto put8 = [&](int r, int c0, const float (&v)[8]) {
    vec hi, lo;
    split8<WT>(v, hi, lo);
    *reinterpret_cast<vec*>(&oh[r * kMPOPitch + c0]) = hi;
    *reinterpret_cast<vec*>(&ol[r * kMPOPitch + c0]) = lo;
  };
  f32x4 o[2][2];
  if (rows >= kMPWaves) {
    const int t[2] = {rb * kMPRows + wave, wave + kMPWaves < rows ? rb * kMPRows + wave + kMPWaves : -1};
    merge_tasks<F16, false, kMPSlots>(p, t, h, 0, 1, lane, o);
    LA_RSTAMP(2);
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const bool live = q == 0 || t[1] >= 0;
      float v[8];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v[e] = live ? o[q][0][e] : 0.f;
        v[4 + e] = live ? o[q][1][e] : 0.f;
      }
      put8(wave + kMPWaves * q, 8 * lane, v);
    }
    __syncthreads();
  } else {
    const int G = kMPWaves / rows;
    const int r = wave / G, g = wave % G;
    const int t[2] = {r < rows ? rb * kMPRows + r : -1, -1};
    merge_tasks<F16, false, kMPSlots>(p, t, h, g, G, lane, o);
    LA_RSTAMP(2);
    *reinterpret_cast<f32x4*>(&gp[wave * kMPPitch + 8 * lane]) = o[0][0];
    *reinterpret_cast<f32x4*>(&gp[wave * kMPPitch + 8 * lane + 4]) = o[0][1];
    __syncthreads();
    // O row r = sum of the G group rows of waves r G .. r G + G - 1; the
    // block's other rows are zero
    for (int i = tid; i < kMPRows * (kDcP / 8); i += kMPWaves * 64) {
      const int rr = i / (kDcP / 8), c8 = i % (kDcP / 8);
      f32x4 v0 = {0.f, 0.f, 0.f, 0.f}, v1 = v0;
      if (rr < rows)
        for (int q = 0; q < G; ++q) {
          v0 += *reinterpret_cast<const f32x4*>(&gp[(rr * G + q) * kMPPitch + 8 * c8]);
          v1 += *reinterpret_cast<const f32x4*>(&gp[(rr * G + q) * kMPPitch + 8 * c8 + 4]);
        }
      float v[8];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v[e] = v0[e];
        v[4 + e] = v1[e];
      }
      put8(rr, 8 * c8, v);
    }
    __syncthreads();
  }

  // A[m = lane % 16][k = 32 ks + 8 (lane / 16) + j] = O[m][k] (high, low)
  LA_RSTAMP(3);
  f32x4 acc_hi = {}, acc_lo = {};
  const int a0 = (lane & 15) * kMPOPitch + 8 * (lane >> 4);
#pragma unroll
  for (int ks = 0; ks < 16; ++ks) {
    const vec hi = *reinterpret_cast<const vec*>(&oh[a0 + 32 * ks]);
    const vec lo = *reinterpret_cast<const vec*>(&ol[a0 + 32 * ks]);
    acc_hi = M::mma(hi, bw[ks], acc_hi);
    acc_lo = M::mma(lo, bw[ks], acc_lo);
  }
  LA_RSTAMP(4);
  // D[m = 4 (lane / 16) + i][n = lane % 16]
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = 4 * (lane >> 4) + i;
    if (r < rows) {
      const int t = rb * kMPRows + r;
      const int64_t orow = (int64_t)(t / p.qps) * p.Hq + (t % p.qps) * p.nh + h;
      p.out[orow * p.dv + 16 * wave + (lane & 15)] = acc_hi[i] + acc_lo[i] * (1.f / kLoScale);
    }
  }
  LA_RSTAMP_WRITE(1);
}

// Merge + W_UV projection over one latent half, for launches with fewer
// (head, row block) workgroups than CUs (a few query rows): one workgroup of
// 8 waves per (head h, 16 query rows, latent half c) merges the half rows
// (fp16 slots, 512 B each) and multiplies them by W_UV's columns 256 c ..
// 256 c + 255 (64 KB per head), so twice as many workgroups move half the
// bytes each. Both halves add their products into out with float atomics;
// the kernel that writes the attention kernel's 16-bit queries
// (absorb_mfma_kernel, or prep_q_kernel for pre-absorbed queries) zeroes out
// earlier in the same call, and two addends onto zero give fl(a + b) in
// either order, so the result does not depend on which half lands first.
constexpr int kMPHPitch = 256 + 8;  // 16-bit elements per LDS operand row (528 B: 16 B past 2 x 256)
constexpr int kMPHSum = 256 + 4;    // floats per LDS row of a slot-group sum

template <typename WT, int NB>
__global__ __launch_bounds__(kMPWaves * 64) void merge_project_half_kernel(DecodeProblem p) {
  LA_RSTAMP_DECL;
  LA_RSTAMP(0);
  warm_kernarg_lines(p);
  typedef Mma16<WT> M;
  typedef typename M::vec vec;
  typedef typename Mma<WT>::elem E;
  typedef typename std::conditional<std::is_same<WT, __half>::value, f16x4, bf16x4>::type vec4;
  constexpr float kLoScale = Mma<WT>::kLoScale;
  __shared__ __attribute__((aligned(16))) short oh[kMPRows * kMPHPitch];  // merged O half rows, high parts
  __shared__ __attribute__((aligned(16))) short ol[kMPRows * kMPHPitch];  // and residuals
  __shared__ __attribute__((aligned(16))) float gp[kMPWaves * kMPHSum];   // slot-group sums
  const int R = p.num_seqs * p.qps;
  const int nrb = (R + kMPRows - 1) / kMPRows;
  // id = 8 (2 (head / 8 * nrb + row block) + c) + head % 8: both halves of a
  // (head, row block) run on one XCD
  const int x = blockIdx.x & 7, k = blockIdx.x >> 3;
  const int c = k & 1, k2 = k >> 1;
  const int h = (k2 / nrb) * 8 + x, rb = k2 % nrb;
  if (h >= p.nh) return;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int rows = min(kMPRows, R - rb * kMPRows);

  // W_UV operands: B[k = 32 ks + 8 (lane / 16) + j][n = lane % 16]
  //              = W_UV[h dv + 16 wave + lane % 16][256 c + 32 ks + 8 (lane / 16) + j]
  const WT* wrow = reinterpret_cast<const WT*>(p.W_UV) + ((int64_t)h * p.dv + 16 * wave + (lane & 15)) * kDcP +
                   256 * c + 8 * (lane >> 4);
  vec bw[8];
#pragma unroll
  for (int ks = 0; ks < 8; ++ks) bw[ks] = __builtin_bit_cast(vec, *reinterpret_cast<const i16x8*>(wrow + 32 * ks));
  LA_RSTAMP(1);

  // row r, columns c0 .. c0 + 3 of the half -> high and low operand rows
  auto put4 = [&](int r, int c0, const f32x4& v) {
    vec4 hi, lo;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const E hv = (E)v[e];
      hi[e] = hv;
      lo[e] = (E)((v[e] - (float)hv) * kLoScale);
    }
    *reinterpret_cast<vec4*>(&oh[r * kMPHPitch + c0]) = hi;
    *reinterpret_cast<vec4*>(&ol[r * kMPHPitch + c0]) = lo;
  };
  f32x4 o[2][2];
  if (rows >= kMPWaves) {
    const int t[2] = {rb * kMPRows + wave, wave + kMPWaves < rows ? rb * kMPRows + wave + kMPWaves : -1};
    merge_tasks<true, true, NB>(p, t, h, 0, 1, lane, o, c);
    LA_RSTAMP(2);
    put4(wave, 4 * lane, o[0][0]);
    put4(wave + kMPWaves, 4 * lane, t[1] >= 0 ? o[1][0] : f32x4{0.f, 0.f, 0.f, 0.f});
    __syncthreads();
  } else {
    const int G = kMPWaves / rows;
    const int r = wave / G, g = wave % G;
    const int t[2] = {r < rows ? rb * kMPRows + r : -1, -1};
    merge_tasks<true, true, NB>(p, t, h, g, G, lane, o, c);
    LA_RSTAMP(2);
    *reinterpret_cast<f32x4*>(&gp[wave * kMPHSum + 4 * lane]) = o[0][0];
    __syncthreads();
    // O half row r = sum of the G group rows of waves r G .. r G + G - 1; the
    // block's other rows are zero
    for (int i = tid; i < kMPRows * 64; i += kMPWaves * 64) {
      const int rr = i / 64, c4 = i % 64;
      f32x4 v = {0.f, 0.f, 0.f, 0.f};
      if (rr < rows)
        for (int q = 0; q < G; ++q) v += *reinterpret_cast<const f32x4*>(&gp[(rr * G + q) * kMPHSum + 4 * c4]);
      put4(rr, 4 * c4, v);
    }
    __syncthreads();
  }

  // A[m = lane % 16][k = 32 ks + 8 (lane / 16) + j] = O[m][256 c + k] (high, low)
  LA_RSTAMP(3);
  f32x4 acc_hi = {}, acc_lo = {};
  const int a0 = (lane & 15) * kMPHPitch + 8 * (lane >> 4);
#pragma unroll
  for (int ks = 0; ks < 8; ++ks) {
    const vec hi = *reinterpret_cast<const vec*>(&oh[a0 + 32 * ks]);
    const vec lo = *reinterpret_cast<const vec*>(&ol[a0 + 32 * ks]);
    acc_hi = M::mma(hi, bw[ks], acc_hi);
    acc_lo = M::mma(lo, bw[ks], acc_lo);
  }
  LA_RSTAMP(4);
  // D[m = 4 (lane / 16) + i][n = lane % 16], added into the zeroed output
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = 4 * (lane >> 4) + i;
    if (r < rows) {
      const int t = rb * kMPRows + r;
      const int64_t orow = (int64_t)(t / p.qps) * p.Hq + (t % p.qps) * p.nh + h;
      atomicAdd(&p.out[orow * p.dv + 16 * wave + (lane & 15)], acc_hi[i] + acc_lo[i] * (1.f / kLoScale));
    }
  }
  LA_RSTAMP_WRITE(1);
}

}  // namespace

bool absorb_mfma_supported(int w_dtype, int nh, int dn, int dc) {
  (void)nh;
  return (w_dtype == LA_DTYPE_BF16 || w_dtype == LA_DTYPE_F16) && dn % 16 == 0 && dn <= 128 && dc % kAbsCols == 0;
}

hipError_t launch_absorb_mfma(const float* q_nope, const void* W_UK, int w_dtype, void* out, int out_mode,
                              const float* q_rope, float scale, int dR, int tokens, int nh, int dn, int dc, int qps,
                              hipStream_t stream, float* zero_out, int64_t zero_n) {
  if (out_mode != 0 && (dc + dR != kQPrepRow || qps <= 0)) return hipErrorInvalidValue;
  // one block per (token block, head, column block), ordered for the XCDs:
  // groups of (token block, 8 heads) with 8 * (dc / 128) blocks each
  const int64_t groups = (int64_t)((tokens + 31) / 32) * ((nh + 7) / 8);
  dim3 grid((unsigned)(8 * 8 * (dc / kAbsCols) * ((groups + 7) / 8)));
  const bool d128 = dn == 128;
  if (w_dtype == LA_DTYPE_BF16) {
    auto k = d128 ? absorb_mfma_kernel<__hip_bfloat16, 8> : absorb_mfma_kernel<__hip_bfloat16, 0>;
    hipLaunchKernelGGL(k, grid, dim3(kAbsThreads), 0, stream, q_nope, reinterpret_cast<const __hip_bfloat16*>(W_UK), out,
                       out_mode, q_rope, scale, dR, tokens, nh, dn, dc, qps, zero_out, zero_n);
  } else {
    auto k = d128 ? absorb_mfma_kernel<__half, 8> : absorb_mfma_kernel<__half, 0>;
    hipLaunchKernelGGL(k, grid, dim3(kAbsThreads), 0, stream, q_nope, reinterpret_cast<const __half*>(W_UK), out, out_mode,
                       q_rope, scale, dR, tokens, nh, dn, dc, qps, zero_out, zero_n);
  }
  return hipGetLastError();
}

bool project_mfma_supported(const DecodeProblem& p) {
  return (p.wuv_dtype == LA_DTYPE_BF16 || p.wuv_dtype == LA_DTYPE_F16) && p.dc == kDcP && p.dv == 128 &&
         (reinterpret_cast<uintptr_t>(p.W_UV) & 15) == 0;
}

int merge_project_blocks(const DecodeProblem& p) {
  const int R = p.num_seqs * p.qps;
  return 8 * ((p.nh + 7) / 8) * ((R + kMPRows - 1) / kMPRows);
}

hipError_t launch_combine_project_mfma(const DecodeProblem& p, hipStream_t stream, bool halves) {
  const int R = p.num_seqs * p.qps;
  if (R == 0) return hipSuccess;
  const int nrb = (R + kMPRows - 1) / kMPRows;
  if (halves) {
    if (!p.part_f16) return hipErrorInvalidValue;
    // id = 8 (2 (head / 8 * nrb + row block) + half) + head % 8
    const dim3 grid((unsigned)(2 * merge_project_blocks(p)));
    // slots per task with equal sequences (seq_len / chunk_len when chunks
    // align with the sequences, else up to two more; rows of a block share
    // G = 8 / rows tasks); ragged or capacity caches keep the 8-slot batches
    const int rows = R < kMPRows ? R : kMPRows;
    const int G = rows >= kMPWaves ? 1 : kMPWaves / rows;
    const int64_t n = p.offsets || p.lens || p.chunk_len <= 0 ? 0
                      : p.seq_len % p.chunk_len == 0 ? p.seq_len / p.chunk_len
                                                     : p.seq_len / p.chunk_len + 2;
    const bool wide = (n + G - 1) / G > kMPSlots;
    auto k = p.wuv_dtype == LA_DTYPE_BF16 ? (wide ? merge_project_half_kernel<__hip_bfloat16, 32>
                                                  : merge_project_half_kernel<__hip_bfloat16, kMPSlots>)
                                          : (wide ? merge_project_half_kernel<__half, 32>
                                                  : merge_project_half_kernel<__half, kMPSlots>);
    hipLaunchKernelGGL(k, grid, dim3(kMPWaves * 64), 0, stream, p);
    return hipGetLastError();
  }
  // id = 8 (head / 8 * nrb + row block) + head % 8
  const dim3 grid((unsigned)(8 * ((p.nh + 7) / 8) * nrb));
  if (p.wuv_dtype == LA_DTYPE_BF16) {
    if (p.part_f16)
      hipLaunchKernelGGL((merge_project_kernel<__hip_bfloat16, true>), grid, dim3(kMPWaves * 64), 0, stream, p);
    else
      hipLaunchKernelGGL((merge_project_kernel<__hip_bfloat16, false>), grid, dim3(kMPWaves * 64), 0, stream, p);
  } else {
    if (p.part_f16)
      hipLaunchKernelGGL((merge_project_kernel<__half, true>), grid, dim3(kMPWaves * 64), 0, stream, p);
    else
      hipLaunchKernelGGL((merge_project_kernel<__half, false>), grid, dim3(kMPWaves * 64), 0, stream, p);
  }
  return hipGetLastError();
}

#ifdef LA_PHASE_STAMPS
// Phase-timing build: copies (clear == 0) the stamps of kernel kind (0
// absorb, 1 merge + projection) of blocks 0 .. blocks-1 (8 slots each) to
// host, or zeroes them.
extern "C" int la_phase_side_stamps(int kind, unsigned long long* host, int blocks, int clear) {
  if (kind < 0 || kind > 1) return (int)hipErrorInvalidValue;
  const size_t one = sizeof(unsigned long long) * 8 * kSideStampBlocks;
  if (clear) {
    static unsigned long long zeros[kSideStampBlocks * 8];
    return (int)hipMemcpyToSymbol(HIP_SYMBOL(g_side_stamps), zeros, one, one * kind, hipMemcpyHostToDevice);
  }
  const size_t n = sizeof(unsigned long long) * 8 * (size_t)(blocks < kSideStampBlocks ? blocks : kSideStampBlocks);
  return (int)hipMemcpyFromSymbol(host, HIP_SYMBOL(g_side_stamps), n, one * kind, hipMemcpyDeviceToHost);
}
#endif
}  // namespace la
