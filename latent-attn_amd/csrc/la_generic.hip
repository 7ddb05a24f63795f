// VALU kernels of liblatent_attn_hip.so: the dtype/dims-generic split-KV
// decode (used for float32 caches -- the 1e-4 parity mode -- and for shapes
// the MFMA kernel does not cover), the log-sum-exp combine fused with the W_UV
// projection, and the query absorption q_nope . W_UK.
//
// Math restated from the reference (paths relative to the reference repo):
//   score(pos) = scale * (q_abs . c_t[pos]) + scale * (q_rope . RoPE(k_rope[pos], pos))
//                                                      src/fused_mla.cu:234-235
//   RoPE rotate-half on k only, pairs (i, i + d_R/2)   src/fused_mla.cu:34-54
//   softmax over positions, latent accumulation, normalise, project with W_UV
//                                                      src/fused_mla.cu:218-267
// The reference runs that on one thread per head with a two-pass softmax; here
// each wave streams positions with an online (running max) softmax and the
// split-KV partials are merged by log-sum-exp.
#include "la_internal.hpp"

#include <cmath>

namespace la {

namespace {

constexpr int kGenericThreads = 256;  // 4 waves
constexpr int kGenericWaves = kGenericThreads / 64;

// Grid (num_chunks, Hq). Each block walks the segments of its chunk for one
// query head; wave w takes rows lo+w, lo+w+4, ...; lane owns latent columns
// lane + 64*j. Per segment the four waves' (max, sum, acc) are merged in LDS
// and written as one partial slot.
template <typename KT, int NC>
__global__ __launch_bounds__(kGenericThreads) void decode_generic_kernel(DecodeProblem p) {
  const int chunk = blockIdx.x;
  const int hq = blockIdx.y;
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int dc = p.dc, dR = p.dR, half = dR >> 1;

  extern __shared__ float smem[];
  float* q_s = smem;                 // dc
  float* qr_s = smem + dc;           // dR
  float* red = qr_s + dR;            // kGenericWaves * (dc + 2)

  const KT* kv = reinterpret_cast<const KT*>(p.kv);
  const int64_t end_all = seq_begin(p, p.num_seqs);
  int64_t lo = (int64_t)chunk * p.chunk_len;
  const int64_t hi = min(lo + (int64_t)p.chunk_len, end_all);
  lo = max(lo, seq_begin(p, 0));
  if (lo >= hi) return;
  int s = find_seq(p, lo);

  while (lo < hi) {
    const int64_t s_lo = seq_begin(p, s);
    lo = max(lo, s_lo);  // past the unfilled rows of the previous region
    if (lo >= hi) break;
    const int64_t s_hi = seq_end(p, s);
    if (s_hi <= lo) {  // empty sequence, already consumed, or lo in its unfilled rows
      if (++s >= p.num_seqs) break;
      continue;
    }
    const int64_t seg_hi = min(hi, s_hi);
    const int64_t qrow = (int64_t)s * p.Hq + hq;

    __syncthreads();  // previous segment finished with q_s / red
    for (int i = tid; i < dc; i += kGenericThreads) q_s[i] = p.q_abs[qrow * dc + i] * p.scale_log2;
    for (int i = tid; i < dR; i += kGenericThreads) qr_s[i] = p.q_rope[qrow * dR + i] * p.scale_log2;
    __syncthreads();

    float m = -INFINITY, l = 0.f;
    float acc[NC];
#pragma unroll
    for (int j = 0; j < NC; ++j) acc[j] = 0.f;

    for (int64_t r = lo + wave; r < seg_hi; r += kGenericWaves) {
      const int64_t pos = r - s_lo;
      const KT* row = kv + (p.block_table ? paged_row(p, s, pos) : r) * p.row_elems;
      float part = 0.f;
      float cv[NC];
#pragma unroll
      for (int j = 0; j < NC; ++j) {
        const int c = lane + 64 * j;
        cv[j] = c < dc ? to_f32(row[c]) : 0.f;
        part += c < dc ? q_s[c] * cv[j] : 0.f;
      }
      const float* cs = p.rope_cos + rope_row(p, pos) * half;
      const float* sn = p.rope_sin + rope_row(p, pos) * half;
      for (int i = lane; i < half; i += 64) {
        const float k0 = to_f32(row[dc + i]), k1 = to_f32(row[dc + i + half]);
        const float co = cs[i], si = sn[i];
        part += qr_s[i] * (k0 * co - k1 * si) + qr_s[i + half] * (k0 * si + k1 * co);
      }
      const float sc = wave_sum(part);
      const float m_new = fmaxf(m, sc);
      const float alpha = exp2f(m - m_new);
      const float pw = exp2f(sc - m_new);
      l = l * alpha + pw;
#pragma unroll
      for (int j = 0; j < NC; ++j) acc[j] = acc[j] * alpha + pw * cv[j];
      m = m_new;
    }

    float* my = red + wave * (dc + 2);
#pragma unroll
    for (int j = 0; j < NC; ++j) {
      const int c = lane + 64 * j;
      if (c < dc) my[c] = acc[j];
    }
    if (lane == 0) {
      my[dc] = m;
      my[dc + 1] = l;
    }
    __syncthreads();

    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kGenericWaves; ++w) M = fmaxf(M, red[w * (dc + 2) + dc]);
    float wts[kGenericWaves];
    float L = 0.f;
#pragma unroll
    for (int w = 0; w < kGenericWaves; ++w) {
      const float mw = red[w * (dc + 2) + dc];
      wts[w] = mw == -INFINITY ? 0.f : exp2f(mw - M);
      L += wts[w] * red[w * (dc + 2) + dc + 1];
    }
    const int64_t slot = (int64_t)chunk + s;
    const float invL = 1.f / L;
    float* dst = p.part_o + (slot * p.Hq + hq) * dc;
    for (int c = tid; c < dc; c += kGenericThreads) {
      float o = 0.f;
#pragma unroll
      for (int w = 0; w < kGenericWaves; ++w) o += wts[w] * red[w * (dc + 2) + c];
      dst[c] = o * invL;
    }
    if (tid == 0) p.part_lse[slot * p.Hq + hq] = M + log2f(L);

    lo = seg_hi;
    ++s;
  }
}

template <typename KT>
hipError_t launch_generic_t(const DecodeProblem& p, hipStream_t stream) {
  dim3 grid(p.num_chunks, p.Hq);
  const size_t smem = sizeof(float) * (p.dc + p.dR + kGenericWaves * (p.dc + 2));
  const int nc = (p.dc + 63) / 64;
  if (nc <= 1) hipLaunchKernelGGL((decode_generic_kernel<KT, 1>), grid, dim3(kGenericThreads), smem, stream, p);
  else if (nc <= 2) hipLaunchKernelGGL((decode_generic_kernel<KT, 2>), grid, dim3(kGenericThreads), smem, stream, p);
  else if (nc <= 4) hipLaunchKernelGGL((decode_generic_kernel<KT, 4>), grid, dim3(kGenericThreads), smem, stream, p);
  else if (nc <= 8) hipLaunchKernelGGL((decode_generic_kernel<KT, 8>), grid, dim3(kGenericThreads), smem, stream, p);
  else hipLaunchKernelGGL((decode_generic_kernel<KT, 16>), grid, dim3(kGenericThreads), smem, stream, p);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Combine + projection. Grid (nh, ceil(R / kRowsPerBlock)) with
// R = num_seqs * qps query tokens; block (h, rb) handles tokens
// [rb*kRowsPerBlock, ...) for weight head h, so W_UV[h] is read once per
// block. Token r lives in sequence s = r / qps with query head
// hq = (r % qps) * nh + h; its output row is r * nh + h.
// ---------------------------------------------------------------------------
constexpr int kRowsPerBlock = 8;
constexpr int kCombineThreads = 256;

__global__ __launch_bounds__(kCombineThreads) void combine_project_kernel(DecodeProblem p) {
  const int h = blockIdx.x;
  const int r0 = blockIdx.y * kRowsPerBlock;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int dc = p.dc, dv = p.dv;
  const int R = p.num_seqs * p.qps;
  extern __shared__ float Os[];  // kRowsPerBlock * dc

  for (int rr = wave; rr < kRowsPerBlock; rr += kCombineThreads / 64) {
    float* orow = Os + rr * dc;
    const int r = r0 + rr;
    int64_t lo = 0, hi = 0;
    int s = 0, hq = 0;
    if (r < R) {
      s = r / p.qps;
      hq = (r % p.qps) * p.nh + h;
      lo = seq_begin(p, s);
      hi = seq_end(p, s);
    }
    if (hi <= lo) {
      for (int c = lane; c < dc; c += 64) orow[c] = 0.f;
      continue;
    }
    const int64_t cf = lo / p.chunk_len, cl = (hi - 1) / p.chunk_len;
    float M = -INFINITY;
    for (int64_t c = cf; c <= cl; ++c) M = fmaxf(M, p.part_lse[(c + s) * p.Hq + hq]);
    float wsum = 0.f;
    for (int c = lane; c < dc; c += 64) orow[c] = 0.f;
    for (int64_t c = cf; c <= cl; ++c) {
      const int64_t slot = c + s;
      const float w = exp2f(p.part_lse[slot * p.Hq + hq] - M);
      wsum += w;
      const int64_t prow = slot * p.Hq + hq;
      for (int i = lane; i < dc; i += 64) orow[i] += w * load_part(p, prow, i);
    }
    const float inv = 1.f / wsum;
    for (int c = lane; c < dc; c += 64) orow[c] *= inv;
  }
  __syncthreads();

  // out[r*nh + h][j] = sum_c O[r][c] * W_UV[h*dv + j][c]
  for (int j = wave; j < dv; j += kCombineThreads / 64) {
    const int64_t wbase = ((int64_t)h * dv + j) * dc;
    float acc[kRowsPerBlock];
#pragma unroll
    for (int rr = 0; rr < kRowsPerBlock; ++rr) acc[rr] = 0.f;
    for (int c = lane; c < dc; c += 64) {
      const float w = load_any(p.W_UV, p.wuv_dtype, wbase + c);
#pragma unroll
      for (int rr = 0; rr < kRowsPerBlock; ++rr) acc[rr] += Os[rr * dc + c] * w;
    }
#pragma unroll
    for (int rr = 0; rr < kRowsPerBlock; ++rr) {
      const float v = wave_sum(acc[rr]);
      const int r = r0 + rr;
      if (lane == 0 && r < R) p.out[((int64_t)r * p.nh + h) * dv + j] = v;
    }
  }
}

// ---------------------------------------------------------------------------
// Absorption. Grid (nh, ceil(dc/256), ceil(tokens/kAbsTok)); thread = latent
// column c, so W_UK rows are read coalesced and once per token block.
// ---------------------------------------------------------------------------
constexpr int kAbsTok = 16;

__global__ __launch_bounds__(256) void absorb_kernel(const float* __restrict__ q_nope, const void* __restrict__ W,
                                                     int w_dtype, float* __restrict__ q_abs, int tokens, int nh,
                                                     int dn, int dc) {
  const int h = blockIdx.x;
  const int c = blockIdx.y * 256 + threadIdx.x;
  const int t0 = blockIdx.z * kAbsTok;
  extern __shared__ float qs[];  // kAbsTok * dn
  for (int i = threadIdx.x; i < kAbsTok * dn; i += 256) {
    const int tt = i / dn, d = i % dn;
    const int t = t0 + tt;
    qs[i] = t < tokens ? q_nope[((int64_t)t * nh + h) * dn + d] : 0.f;
  }
  __syncthreads();
  if (c >= dc) return;
  float acc[kAbsTok];
#pragma unroll
  for (int tt = 0; tt < kAbsTok; ++tt) acc[tt] = 0.f;
  for (int d = 0; d < dn; ++d) {
    const float w = load_any(W, w_dtype, ((int64_t)h * dn + d) * dc + c);
#pragma unroll
    for (int tt = 0; tt < kAbsTok; ++tt) acc[tt] += qs[tt * dn + d] * w;
  }
#pragma unroll
  for (int tt = 0; tt < kAbsTok; ++tt) {
    const int t = t0 + tt;
    if (t < tokens) q_abs[((int64_t)t * nh + h) * dc + c] = acc[tt];
  }
}

}  // namespace

bool generic_supported(const DecodeProblem& p) {
  return p.dc >= 1 && p.dc <= 1024 && p.dR >= 2 && p.dR <= 256 && (p.dR % 2) == 0 &&
         (p.kv_dtype == LA_DTYPE_F32 || p.kv_dtype == LA_DTYPE_F16 || p.kv_dtype == LA_DTYPE_BF16 ||
          p.kv_dtype == LA_DTYPE_FP8_E4M3);
}

hipError_t launch_decode_generic(const DecodeProblem& p, hipStream_t stream) {
  switch (p.kv_dtype) {
    case LA_DTYPE_F32: return launch_generic_t<float>(p, stream);
    case LA_DTYPE_F16: return launch_generic_t<__half>(p, stream);
    case LA_DTYPE_BF16: return launch_generic_t<__hip_bfloat16>(p, stream);
    case LA_DTYPE_FP8_E4M3: return launch_generic_t<fp8e4m3>(p, stream);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_combine_project(const DecodeProblem& p, hipStream_t stream) {
  const int R = p.num_seqs * p.qps;
  dim3 grid(p.nh, (R + kRowsPerBlock - 1) / kRowsPerBlock);
  const size_t smem = sizeof(float) * kRowsPerBlock * p.dc;
  hipLaunchKernelGGL(combine_project_kernel, grid, dim3(kCombineThreads), smem, stream, p);
  return hipGetLastError();
}

hipError_t launch_absorb(const float* q_nope, const void* W_UK, int w_dtype, float* q_abs, int tokens, int nh, int dn,
                         int dc, hipStream_t stream) {
  dim3 grid(nh, (dc + 255) / 256, (tokens + kAbsTok - 1) / kAbsTok);
  const size_t smem = sizeof(float) * kAbsTok * dn;
  hipLaunchKernelGGL(absorb_kernel, grid, dim3(256), smem, stream, q_nope, W_UK, w_dtype, q_abs, tokens, nh, dn, dc);
  return hipGetLastError();
}

}  // namespace la
