// MFMA kernels for the two small contractions around the attention kernel,
// for 16-bit weights (bf16 or fp16):
//
//   absorb:   q_abs[t,h,c] = sum_i q_nope[t,h,i] * W_UK[h*dn + i, c]
//             (reference tests/test_correctness.cu:29-46, tests/test_python.py:97-99)
//   project:  out[t,h,j]   = sum_c O[t,h,c] * W_UV[h*dv + j, c], where O is the
//             log-sum-exp merge of the split-KV partial slots
//             (reference src/fused_mla.cu:255-267: normalise, then W_UV)
//
// Both run v_mfma_f32_32x32x16 with 32 query tokens as M. The fp32 operand
// (q_nope, or the merged O) is split into a 16-bit high part and a 16-bit
// residual (hi = rn(x), lo = rn(x - hi)); two MFMAs accumulate W*hi + W*lo in
// fp32, so the result keeps ~16 bits of the fp32 operand instead of 8 (bf16)
// or 11 (fp16). For fp16 the residual is pre-multiplied by 2^11 (and its
// product by 2^-11) so it stays in the normal range.
//
// absorb:  grid (nh, dc/128, ceil(T/32)), 256 threads. W_UK[h][:, 128-col
//          block] (128 x 128) is staged in LDS; wave w owns 32 columns; the
//          B operand (8 consecutive rows i per lane) comes from
//          ds_read_b64_tr_b16.
// combine: merge_slots_kernel, one wave per (query row, weight head), writes
//          the log-sum-exp merge of the partial slots (fp32, workspace, in the
//          projection's A-operand order).
// project: one block per (head, 32-row block, 32 output columns); the 4
//          waves split the latent dimension and sum their tiles in LDS.
#include "la_internal.hpp"

#include <type_traits>

namespace la {
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

// out_mode 0: q_abs (fp32, (T*nh, dc)). out_mode 1 / 2: q_prep rows (bf16 /
// fp16, (T*nh, dc + dR)) = [q_abs | q_rope] * scale for the MFMA attention
// kernel; blocks with cb == 0 also convert the q_rope part of their rows.
// All global loads (q_nope for every k-step, the W_UK tile) are issued before
// the first wait.
// NKS = dn / 16 when known at compile time (8 for dn = 128: no guards, every
// load unconditional), 0 for any dn <= 128 that is a multiple of 16.
template <typename WT, int NKS>
__global__ __launch_bounds__(256) void absorb_mfma_kernel(const float* __restrict__ q_nope, const WT* __restrict__ W,
                                                          void* __restrict__ out, int out_mode,
                                                          const float* __restrict__ q_rope, float scale, int dR,
                                                          int tokens, int nh, int dn, int dc, int qps) {
  typedef Mma<WT> M;
  typedef typename M::vec vec;
  __shared__ __attribute__((aligned(16))) char wt[128 * kAbsRowBytes];  // dn <= 128 rows
  // q operands (hi, lo) of the 8 k-steps, shared by the 4 waves: [ks][hi|lo][lane] 16 B
  __shared__ __attribute__((aligned(16))) char qs[8 * 2 * 64 * 16];
  // Block id -> (token block tb, head h, column block cb). The q_prep line of
  // (token, 32-head group, k-step) gathers one 16-B slot from each head of the
  // group, so the blocks of one (tb, head group, cb) run on one XCD (blocks go
  // to XCDs round-robin by id % 8) and their slots meet in that XCD's L2
  // instead of leaving it as partial lines.
  const int ncb = dc / kAbsCols, nhg = (nh + 31) / 32;
  const int x = blockIdx.x & 7, k = blockIdx.x >> 3;
  const int grp = x + 8 * (k >> 5);  // (tb, head group, cb) group
  const int tb = grp / (nhg * ncb), rem = grp - tb * (nhg * ncb);
  const int h = 32 * (rem / ncb) + (k & 31), cb = rem % ncb, t0 = tb * 32;
  if (t0 >= tokens || h >= nh) return;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int nks = NKS > 0 ? NKS : dn / 16;  // <= 8
  if (NKS > 0) dn = 16 * NKS;

  // q_nope of token t0 + lane%32, elements 16ks + 8(lane/32) .. +8: wave w
  // loads k-steps 2w and 2w+1, splits them into hi/lo 16-bit operands and
  // stages them in LDS for all waves (each wave issues 4 q loads, not 16)
  const int t = t0 + (lane & 31);
  const bool tvalid = t < tokens;
  const float* qrow = q_nope + ((int64_t)(tvalid ? t : 0) * nh + h) * dn + 8 * (lane >> 5);
  f32x4 qa[2], qb[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int ks = 2 * wave + j;
    if (ks < nks) {
      qa[j] = *reinterpret_cast<const f32x4*>(qrow + 16 * ks);
      qb[j] = *reinterpret_cast<const f32x4*>(qrow + 16 * ks + 4);
    }
  }
  // W_UK[h*dn + i][cb*128 + 0..127] for i < dn, 16 B per thread-load
  i16x8 wv[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const int q = tid + 256 * k;
    if (NKS > 0 ? k < NKS : q < dn * 16)
      wv[k] = *reinterpret_cast<const i16x8*>(W + ((int64_t)h * dn + (q >> 4)) * dc + cb * kAbsCols + (q & 15) * 8);
  }
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const int q = tid + 256 * k;
    if (NKS > 0 ? k < NKS : q < dn * 16) *reinterpret_cast<i16x8*>(wt + (q >> 4) * kAbsRowBytes + (q & 15) * 16) = wv[k];
  }
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int ks = 2 * wave + j;
    if (ks < nks) {
      float x[8];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        x[e] = tvalid ? qa[j][e] : 0.f;
        x[4 + e] = tvalid ? qb[j][e] : 0.f;
      }
      vec hi, lo;
      split8<WT>(x, hi, lo);
      *reinterpret_cast<vec*>(qs + (2 * ks) * 1024 + 16 * lane) = hi;
      *reinterpret_cast<vec*>(qs + (2 * ks + 1) * 1024 + 16 * lane) = lo;
    }
  }
  __syncthreads();

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
  const int hq_pad = out_mode != 0 ? qprep_rows_per_seq(qps * nh) : 0;
  auto qrow_of = [&](int t) -> int64_t { return (int64_t)(t / qps) * hq_pad + (int64_t)(t % qps) * nh + h; };
  if (out_mode != 0 && cb == 0) {
    // q_rope part of the same rows: 8 elements (one 16-B slot of q_prep) per thread-step
    for (int q = tid; q < 32 * (dR / 8); q += 256) {
      const int tr = t0 + q / (dR / 8), j = 8 * (q % (dR / 8));
      if (tr >= tokens) continue;
      const int64_t row = (int64_t)tr * nh + h;
      const f32x4 a = *reinterpret_cast<const f32x4*>(q_rope + row * dR + j);
      const f32x4 b = *reinterpret_cast<const f32x4*>(q_rope + row * dR + j + 4);
      const int64_t dst = qprep_index(qrow_of(tr), dc + j);
      if (out_mode == 1) {
        bf16x8 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          v[e] = (__bf16)(a[e] * scale);
          v[4 + e] = (__bf16)(b[e] * scale);
        }
        *reinterpret_cast<bf16x8*>(reinterpret_cast<__bf16*>(out) + dst) = v;
      } else {
        f16x8 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          v[e] = (_Float16)(a[e] * scale);
          v[4 + e] = (_Float16)(b[e] * scale);
        }
        *reinterpret_cast<f16x8*>(reinterpret_cast<_Float16*>(out) + dst) = v;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// combine + project
// ---------------------------------------------------------------------------
constexpr int kDcP = 512;

// merge: one wave per (query row r, weight head h). o_merged[r][h][:] =
// sum_slots 2^(lse_s - m) * part_o_s / sum_slots 2^(lse_s - m), m = max lse
// (reference has no split; the merge is exact in real arithmetic). Lane l owns
// latent columns 8l .. 8l+7; the slot loads go out 8 at a time.
constexpr int kMergeWaves = 4;

// One slot's 8 columns of this lane, kept in the stored format until use
// (fp16 rows: before the row scale, which the caller folds into the slot
// weight), so 8 slots in flight cost 32 VGPRs for fp16 rows.
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

// F16: partial rows are fp16 numerators with a power-of-two scale per half row
// (part_scale) and the running max of their scores (part_m).
template <bool F16>
__global__ __launch_bounds__(kMergeWaves * 64) void merge_slots_kernel(DecodeProblem p, float* __restrict__ o_merged) {
  typedef typename std::conditional<F16, _Float16, float>::type PT;
  const int lane = threadIdx.x & 63;
  const int R = p.num_seqs * p.qps;
  const int Rp = (R + 31) & ~31;  // rows padded to the projection's 32-row blocks
  // wave -> (weight head h, query row r), r fastest: the waves of a block write
  // neighbouring rows, which share the 128-B lines of the operand-order output
  const int64_t pair = (int64_t)blockIdx.x * kMergeWaves + (threadIdx.x >> 6);
  if (pair >= (int64_t)Rp * p.nh) return;
  const int h = (int)(pair / Rp), r = (int)(pair % Rp);
  if (r >= R) return;
  const int s = r / p.qps;
  const int hq = (r % p.qps) * p.nh + h;
  f32x4 o0 = {0.f, 0.f, 0.f, 0.f}, o1 = {0.f, 0.f, 0.f, 0.f};
  const int64_t lo = seq_begin(p, s), hi = seq_end(p, s);
  if (hi > lo) {
    const int64_t cf = lo / p.chunk_len;
    const int n = (int)((hi - 1) / p.chunk_len - cf + 1);  // slots cf+s .. cf+s+n-1
    const int64_t row0 = (cf + s) * p.Hq + hq;
    const float* lse = p.part_lse + row0;
    const PT* src = reinterpret_cast<const PT*>(p.part_o) + row0 * kDcP + 8 * lane;
    const int64_t sstride = (int64_t)p.Hq * kDcP;
    // The first 8 slot rows go out before the log-sum-exps they are weighted
    // by, so a merge of up to 8 slots takes one memory round trip.
    SlotRow<F16> d[8];
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (u < n) d[u].load(src + (int64_t)u * sstride);
    // Lane i holds slot i of each 64-slot chunk (chunk 0 stays in registers).
    // Denominator weight 2^(lse - M); numerator weight 2^(lse - M) for fp32
    // O / l rows, 2^(m - M) * 2^e(half) for fp16 numerator rows (lanes 0..31
    // hold columns 0..255, half 0).
    const float ls0 = lane < n ? lse[(int64_t)lane * p.Hq] : -INFINITY;
    float mm0 = 0.f, sa0 = 1.f, sb0 = 1.f;
    if constexpr (F16) {
      if (lane < n) {
        const int64_t pr = row0 + (int64_t)lane * p.Hq;
        mm0 = p.part_m[pr];
        sa0 = p.part_scale[2 * pr];
        sb0 = p.part_scale[2 * pr + 1];
      }
    }
    float mx = ls0;
    for (int i = lane + 64; i < n; i += 64) mx = fmaxf(mx, lse[(int64_t)i * p.Hq]);
    mx = wave_max(mx);
    float wsum = 0.f;
    for (int i0 = 0; i0 < n; i0 += 64) {
      const int nb = min(64, n - i0);
      float ls = ls0, mm = mm0, sa = sa0, sb = sb0;
      if (i0 > 0) {
        const bool ok = lane < nb;
        const int64_t pr = row0 + (int64_t)(min(i0 + lane, n - 1)) * p.Hq;
        ls = ok ? lse[(int64_t)(i0 + lane) * p.Hq] : -INFINITY;
        if constexpr (F16) {
          mm = ok ? p.part_m[pr] : 0.f;
          sa = ok ? p.part_scale[2 * pr] : 1.f;
          sb = ok ? p.part_scale[2 * pr + 1] : 1.f;
        }
      }
      const float wden = lane < nb ? exp2f(ls - mx) : 0.f;
      wsum += wave_sum(wden);
      float wlo = wden, whi = wden;
      if constexpr (F16) {
        const float a = lane < nb ? exp2f(mm - mx) : 0.f;
        wlo = a * sa;
        whi = a * sb;
      }
      for (int j = 0; j < nb; j += 8) {
        if (i0 > 0 || j > 0) {
#pragma unroll
          for (int u = 0; u < 8; ++u)
            if (j + u < nb) d[u].load(src + (int64_t)(i0 + j + u) * sstride);
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          if (j + u < nb) {
            // slot weights broadcast from lane j + u (wave-uniform index: v_readlane, no LDS)
            const float w0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wlo), j + u));
            const float w1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, whi), j + u));
            d[u].fma(lane < 32 ? w0 : w1, o0, o1);
          }
        }
      }
    }
    const float inv = 1.f / wsum;
    o0 *= inv;
    o1 *= inv;
  }
  // o_merged in the projection's A-operand order: block (h, r / 32), k-step
  // ks = lane / 2 (16 columns), lane slot (r % 32) + 32 (lane % 2): 8 floats.
  float* dst = o_merged + (((int64_t)h * (Rp / 32) + r / 32) * (kDcP / 16) + (lane >> 1)) * 512 +
               ((r & 31) + 32 * (lane & 1)) * 8;
  *reinterpret_cast<f32x4*>(dst) = o0;
  *reinterpret_cast<f32x4*>(dst + 4) = o1;
}

// project: one block per (weight head h, 32-row block rb, 32 output columns
// dq), XCD-ordered so the 4 column blocks of (h, rb) share an L2. Wave w takes
// the latent columns 128w .. 128w+127 (8 k-steps): A = merged O rows (fp32 in
// the operand order the merge wrote, split into 16-bit hi/lo), B = 16
// contiguous bytes of a W_UV row; the 4 partial 32x32 tiles are summed in LDS.
// Every wave issues its 24 loads at once.
template <typename WT>
__global__ __launch_bounds__(256) void project_mfma_kernel(DecodeProblem p, const float* __restrict__ o_merged) {
  typedef Mma<WT> M;
  typedef typename M::vec vec;
  __shared__ __attribute__((aligned(16))) float red[3][16][64];  // partial tiles of waves 1..3
  const int R = p.num_seqs * p.qps;
  const int nrb = (R + 31) / 32;
  const int x = blockIdx.x & 7, k = blockIdx.x >> 3;
  const int grp = x + 8 * (k >> 2);  // (h, rb)
  const int dq = k & 3;
  if (grp >= p.nh * nrb) return;
  const int h = grp / nrb, rb = grp % nrb;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;

  const float* oa = o_merged + (((int64_t)h * nrb + rb) * (kDcP / 16) + 8 * wave) * 512 + 8 * lane;
  f32x4 olo[8], ohi[8];
#pragma unroll
  for (int ks = 0; ks < 8; ++ks) {
    olo[ks] = *reinterpret_cast<const f32x4*>(oa + 512 * ks);
    ohi[ks] = *reinterpret_cast<const f32x4*>(oa + 512 * ks + 4);
  }
  const WT* wrow = reinterpret_cast<const WT*>(p.W_UV) + ((int64_t)h * p.dv + 32 * dq + (lane & 31)) * kDcP +
                   128 * wave + 8 * (lane >> 5);
  vec bw[8];
#pragma unroll
  for (int ks = 0; ks < 8; ++ks) bw[ks] = __builtin_bit_cast(vec, *reinterpret_cast<const i16x8*>(wrow + 16 * ks));

  // out[row][32dq + n], partial over this wave's latent quarter
  f32x16 acc_hi = {}, acc_lo = {};
#pragma unroll
  for (int ks = 0; ks < 8; ++ks) {
    float o[8];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      o[e] = olo[ks][e];
      o[4 + e] = ohi[ks][e];
    }
    vec vh, vl;
    split8<WT>(o, vh, vl);
    acc_hi = M::mma(vh, bw[ks], acc_hi);
    acc_lo = M::mma(vl, bw[ks], acc_lo);
  }
  f32x16 part;
#pragma unroll
  for (int i = 0; i < 16; ++i) part[i] = acc_hi[i] + acc_lo[i] * (1.f / M::kLoScale);
  if (wave > 0) {
#pragma unroll
    for (int i = 0; i < 16; ++i) red[wave - 1][i][lane] = part[i];
  }
  __syncthreads();
  if (wave == 0) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const float v = part[i] + red[0][i][lane] + red[1][i][lane] + red[2][i][lane];
      const int r = 32 * rb + 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3);
      if (r < R) p.out[((int64_t)r * p.nh + h) * p.dv + 32 * dq + (lane & 31)] = v;
    }
  }
}

}  // namespace

bool absorb_mfma_supported(int w_dtype, int nh, int dn, int dc) {
  (void)nh;
  return (w_dtype == LA_DTYPE_BF16 || w_dtype == LA_DTYPE_F16) && dn % 16 == 0 && dn <= 128 && dc % kAbsCols == 0;
}

hipError_t launch_absorb_mfma(const float* q_nope, const void* W_UK, int w_dtype, void* out, int out_mode,
                              const float* q_rope, float scale, int dR, int tokens, int nh, int dn, int dc, int qps,
                              hipStream_t stream) {
  if (out_mode != 0 && (dc + dR != kQPrepRow || qps <= 0)) return hipErrorInvalidValue;
  // one block per (token block, head, column block), ordered for the XCDs
  const int64_t groups = (int64_t)((tokens + 31) / 32) * ((nh + 31) / 32) * (dc / kAbsCols);
  dim3 grid((unsigned)(8 * 32 * ((groups + 7) / 8)));
  const bool d128 = dn == 128;
  if (w_dtype == LA_DTYPE_BF16) {
    auto k = d128 ? absorb_mfma_kernel<__hip_bfloat16, 8> : absorb_mfma_kernel<__hip_bfloat16, 0>;
    hipLaunchKernelGGL(k, grid, dim3(256), 0, stream, q_nope, reinterpret_cast<const __hip_bfloat16*>(W_UK), out,
                       out_mode, q_rope, scale, dR, tokens, nh, dn, dc, qps);
  } else {
    auto k = d128 ? absorb_mfma_kernel<__half, 8> : absorb_mfma_kernel<__half, 0>;
    hipLaunchKernelGGL(k, grid, dim3(256), 0, stream, q_nope, reinterpret_cast<const __half*>(W_UK), out, out_mode,
                       q_rope, scale, dR, tokens, nh, dn, dc, qps);
  }
  return hipGetLastError();
}

bool project_mfma_supported(const DecodeProblem& p) {
  return (p.wuv_dtype == LA_DTYPE_BF16 || p.wuv_dtype == LA_DTYPE_F16) && p.dc == kDcP && p.dv % 128 == 0 &&
         p.dv == 128 && (reinterpret_cast<uintptr_t>(p.W_UV) & 15) == 0;
}

template <typename WT>
hipError_t launch_proj(const DecodeProblem& p, const float* o_merged, hipStream_t stream) {
  const int64_t groups = (int64_t)p.nh * ((p.num_seqs * p.qps + 31) / 32);  // (h, rb)
  dim3 grid((unsigned)(8 * 4 * ((groups + 7) / 8)));
  hipLaunchKernelGGL(project_mfma_kernel<WT>, grid, dim3(256), 0, stream, p, o_merged);
  return hipGetLastError();
}

size_t combine_project_mfma_workspace(const DecodeProblem& p) {
  const size_t rows = ((size_t)p.num_seqs * p.qps + 31) / 32 * 32;
  return rows * p.nh * kDcP * sizeof(float);
}

hipError_t launch_combine_project_mfma(const DecodeProblem& p, float* o_merged, hipStream_t stream) {
  const int64_t pairs = (int64_t)((p.num_seqs * p.qps + 31) / 32 * 32) * p.nh;  // rows padded to 32
  if (p.num_seqs * p.qps == 0) return hipSuccess;
  const dim3 grid((unsigned)((pairs + kMergeWaves - 1) / kMergeWaves));
  if (p.part_f16)
    hipLaunchKernelGGL((merge_slots_kernel<true>), grid, dim3(kMergeWaves * 64), 0, stream, p, o_merged);
  else
    hipLaunchKernelGGL((merge_slots_kernel<false>), grid, dim3(kMergeWaves * 64), 0, stream, p, o_merged);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  if (p.wuv_dtype == LA_DTYPE_BF16) return launch_proj<__hip_bfloat16>(p, o_merged, stream);
  return launch_proj<__half>(p, o_merged, stream);
}

}  // namespace la
