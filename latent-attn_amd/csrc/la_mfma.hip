// MFMA split-KV MLA decode kernel for gfx950 (MI355X): 16-bit latent cache
// (bf16 or fp16), kv_lora_rank 512, qk_rope_head_dim 64.
//
// Math (paths relative to the reference repo): for each query head h and
// cached position pos
//   s[h,pos] = scale*(q_abs[h] . c_t[pos]) + scale*(q_rope[h] . RoPE(k_rope[pos], pos))
//                                                      src/fused_mla.cu:234-235
//   RoPE rotate-half, pairs (i, i+32), cos/sin rows by position  src/fused_mla.cu:34-54
//   acc[h] = sum_pos softmax_pos(s[h,:]) * c_t[pos]    src/fused_mla.cu:240-256
// The reference computes this on one thread per head; here one workgroup
// streams a chunk of the cache for a group of up to 64 heads.
//
// Work decomposition. 1-D grid over (chunk, head group); the head groups of one
// chunk get block ids 8 apart, so they run on the same XCD at about the same
// time and the second read of every tile is an L2 hit. 512 threads = 8 waves.
// A block walks the segments of its chunk (pieces of the chunk inside one
// sequence) in tiles of 32 positions:
//   * Staging: each tile (32 rows x 1152 B, one contiguous HBM range) and its
//     cos/sin rows are copied HBM->LDS with global_load_lds_dwordx4 (no VGPR
//     staging), up to three tiles in flight. Inside a row the 16-B chunk j
//     lives at chunk j ^ (row & 7), so 16 lanes reading 16 rows at one column
//     hit distinct banks. k_rope is rotated in place in LDS once per position
//     (shared by all heads).
//   * Scores: wave w computes S[16 heads x 16 positions] for head block w&3
//     and position half w>>2 with v_mfma_f32_16x16x32 (A = Q in VGPRs as
//     16-bit, pre-scaled by scale*log2(e); B = 16-B reads of tile rows).
//   * Online softmax in base 2 (running max m shared by the two position
//     halves through LDS, per-half running sums l); P (16-bit) and the rescale
//     factor alpha go to LDS.
//   * PV: wave w owns latent columns [64w, 64w+64) of O for all 64 heads:
//     O += P[64 x 32] . Tile[32 x 64] with v_mfma_f32_32x32x16 (A = P rows,
//     B = tile columns via ds_read_b64_tr_b16).
//   * At a segment end O / l and the base-2 log-sum-exp m + log2(l) go to the
//     partial slot (chunk + sequence); a later kernel merges the slots.
#include "la_internal.hpp"

#include <cstring>
#include <mutex>

namespace la {
namespace {

constexpr int kDc = 512;
constexpr int kDr = 64;
constexpr int kRow = kDc + kDr;       // elements per cache row
constexpr int kRowBytes = kRow * 2;   // 1152
constexpr int kT = 32;                // positions per tile
constexpr int kWaves = 8;
constexpr int kThreads = kWaves * 64;
constexpr int kHG = 64;               // heads per group (block)
constexpr int kNHB = kHG / 32;        // 32-head blocks in PV
constexpr int kTileBytes = kT * kRowBytes;      // 36864
constexpr int kTabBytes = kT * (kDr / 2) * 4;   // 4096: 32 rows of 32 floats
constexpr int kBufBytes = kTileBytes + 2 * kTabBytes;
constexpr int kNBuf = 3;
constexpr int kPRowBytes = 80;                  // 32 x 16-bit P + 16 B pad
constexpr int kPOff = kNBuf * kBufBytes;
constexpr int kAlphaOff = kPOff + kHG * kPRowBytes;
constexpr int kTmaxOff = kAlphaOff + kHG * 4;   // [2][kHG] tile maxima per position half
constexpr int kLsumOff = kTmaxOff + 2 * kHG * 4;  // [2][kHG] running sums per half
constexpr int kInvLOff = kLsumOff + 2 * kHG * 4;
constexpr int kLdsBytes = kInvLOff + kHG * 4;
constexpr int kDmaPerTile = kTileBytes / 1024 + 2 * kTabBytes / 1024;  // 44
// Longest chunk the kernel accepts: keeps row byte offsets inside 32 bits.
constexpr int kMaxChunkRows = 1 << 20;

static_assert(kLdsBytes <= 160 * 1024, "LDS budget");

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef short i16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

typedef __attribute__((address_space(3))) void lds_void;

// Element-type traits: MFMA operand vector and instructions per 16-bit type.
template <typename KT>
struct Ops;

template <>
struct Ops<__hip_bfloat16> {
  typedef bf16x8 vec;
  typedef __bf16 elem;
  static __device__ inline f32x4 mma16(vec a, vec b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
  static __device__ inline f32x16 mma32(vec a, vec b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};

template <>
struct Ops<__half> {
  typedef f16x8 vec;
  typedef _Float16 elem;
  static __device__ inline f32x4 mma16(vec a, vec b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
  static __device__ inline f32x16 mma32(vec a, vec b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};

// Byte offset of logical 16-B chunk j of tile row `row` (XOR swizzle).
__device__ inline int swz(int row, int j) { return row * kRowBytes + ((j ^ (row & 7)) << 4); }

__device__ inline void wait_vm0() { __builtin_amdgcn_s_waitcnt(0x0F70); }  // vmcnt(0)

// LDS-visibility barrier that leaves outstanding HBM->LDS copies in flight:
// waits for this wave's LDS operations only, then s_barrier. The "memory"
// clobber keeps the compiler from moving LDS accesses across it.
__device__ inline void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

template <typename T>
__device__ inline T lds_load(const char* base, int off) {
  return *reinterpret_cast<const T*>(base + off);
}

struct SegCtx {
  const char* base;   // first byte of the segment's first row
  int64_t seg_lo;     // first row of the segment
  int64_t seg_hi;     // one past the last row
  int64_t pos0;       // in-sequence position of seg_lo
  int last;           // index of the segment's last row, relative to seg_lo
};

// Issue this wave's share of the HBM->LDS copies for tile k of the segment
// into buffer `buf`. Addresses are a wave-uniform base plus a 32-bit lane
// offset (segments are capped at kMaxChunkRows rows, tables at 2^24 rows).
// Rows past the segment end re-read its last row (their scores are masked);
// cos/sin rows are clamped the same way and to the table.
__device__ inline void issue_tile_dma(const DecodeProblem& p, const SegCtx& sg, int k, char* buf, int wave,
                                      int lane) {
  const int r0 = k * kT;
  for (int ii = wave; ii < kDmaPerTile; ii += kWaves) {
    const char* src;
    char* dst;
    if (ii < kTileBytes / 1024) {
      const int q = ii * 64 + lane;  // physical 16-B chunk index inside the tile
      const int row = q / 72, jp = q - row * 72;
      const int j = jp ^ (row & 7);
      const int r = min(r0 + row, sg.last);
      src = sg.base + (uint32_t)(r * kRowBytes + j * 16);
      dst = buf + ii * 1024;
    } else {
      const int t = ii - kTileBytes / 1024;  // 0..3 cos, 4..7 sin
      const int part = t & 3;
      const int r = min(r0 + part * 8 + (lane >> 3), sg.last);
      const int pos = (int)rope_row(p, sg.pos0 + r);
      const char* tab = reinterpret_cast<const char*>(t < 4 ? p.rope_cos : p.rope_sin);
      src = tab + (uint32_t)(pos * (kDr / 2 * 4) + (lane & 7) * 16);
      dst = buf + kTileBytes + (t < 4 ? 0 : kTabBytes) + part * 1024;
    }
    __builtin_amdgcn_global_load_lds(src, (lds_void*)dst, 16, 0, 0);
  }
}

// Rotate-half RoPE of the tile's k_rope in place (src/fused_mla.cu:43-51):
// r[i] = k[i]*c - k[i+32]*s, r[i+32] = k[i]*s + k[i+32]*c. Threads 0..255,
// each 4 consecutive i of one row.
template <typename KT>
__device__ inline void rotate_tile(char* buf, int tid) {
  typedef typename Ops<KT>::elem E;
  if (tid >= kT * 8) return;
  const int row = tid >> 3, u = tid & 7;
  const int i0 = u * 4;                        // 0..28
  const int ja = 64 + (i0 >> 3), jb = ja + 4;  // chunks holding k[i0], k[i0+32]
  const int sub = (i0 & 7) * 2;                // byte offset inside the chunk
  char* pa = buf + swz(row, ja) + sub;
  char* pb = buf + swz(row, jb) + sub;
  const i16x4 ka = *reinterpret_cast<i16x4*>(pa);
  const i16x4 kb = *reinterpret_cast<i16x4*>(pb);
  const f32x4 c = *reinterpret_cast<const f32x4*>(buf + kTileBytes + row * 128 + i0 * 4);
  const f32x4 s = *reinterpret_cast<const f32x4*>(buf + kTileBytes + kTabBytes + row * 128 + i0 * 4);
  i16x4 ra, rb;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float k0 = (float)__builtin_bit_cast(E, (short)ka[e]);
    const float k1 = (float)__builtin_bit_cast(E, (short)kb[e]);
    ra[e] = __builtin_bit_cast(short, (E)(k0 * c[e] - k1 * s[e]));
    rb[e] = __builtin_bit_cast(short, (E)(k0 * s[e] + k1 * c[e]));
  }
  *reinterpret_cast<i16x4*>(pa) = ra;
  *reinterpret_cast<i16x4*>(pb) = rb;
}

// Block id -> (chunk, head group). Head groups of one chunk sit 8 ids apart
// (same XCD under round-robin dispatch, consecutive dispatch rounds).
__device__ inline void block_coords(int groups, int* chunk, int* group) {
  const int id = blockIdx.x;
  const int x = id & 7, k = id >> 3;
  *group = k % groups;
  *chunk = (k / groups) * 8 + x;
}

template <typename KT>
__global__ __launch_bounds__(kThreads) void decode_mfma_kernel(DecodeProblem p, int groups) {
  typedef Ops<KT> O_;
  typedef typename O_::vec vec;
  typedef typename O_::elem E;

  extern __shared__ __attribute__((aligned(1024))) char lds[];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  int chunk, group;
  block_coords(groups, &chunk, &group);
  if (chunk >= p.num_chunks) return;
  const int hg_heads = min(kHG, p.Hq - group * kHG);
  const int hb = wave & 3;                  // QK head block (16 heads)
  const int nbq = wave >> 2;                // QK position half (16 positions)
  const bool qk_wave = hb * 16 < hg_heads;

  char* pbuf = lds + kPOff;
  float* alpha_s = reinterpret_cast<float*>(lds + kAlphaOff);
  float* tmax_s = reinterpret_cast<float*>(lds + kTmaxOff);
  float* lsum_s = reinterpret_cast<float*>(lds + kLsumOff);
  float* invl_s = reinterpret_cast<float*>(lds + kInvLOff);
  // Heads without a query keep P = 0, alpha = 1, 1/l = 0 for the whole block.
  for (int i = tid; i < kHG * kPRowBytes / 4; i += kThreads) reinterpret_cast<float*>(pbuf)[i] = 0.f;
  for (int i = tid; i < kHG; i += kThreads) {
    alpha_s[i] = 1.f;
    invl_s[i] = 0.f;
  }

  const int64_t end_all = seq_begin(p, p.num_seqs);
  int64_t lo = (int64_t)chunk * p.chunk_len;
  const int64_t hi = min(lo + (int64_t)p.chunk_len, end_all);
  lo = max(lo, seq_begin(p, 0));
  if (lo >= hi) return;
  int s = find_seq(p, lo);

  const int l16 = lane & 15, g16 = lane >> 4;

  while (lo < hi) {
    const int64_t s_lo = seq_begin(p, s), s_hi = seq_begin(p, s + 1);
    if (s_hi <= lo) {
      ++s;
      continue;
    }
    SegCtx sg;
    sg.base = reinterpret_cast<const char*>(p.kv) + lo * kRowBytes;
    sg.seg_lo = lo;
    sg.seg_hi = min(hi, s_hi);
    sg.pos0 = lo - s_lo;
    sg.last = (int)(sg.seg_hi - sg.seg_lo - 1);
    const int ntiles = (int)((sg.seg_hi - sg.seg_lo + kT - 1) / kT);

    lds_barrier();  // previous segment (or the init above) is done with LDS

    // ---- prologue: tiles 0 and 1 in flight, Q into registers ----
    issue_tile_dma(p, sg, 0, lds + 0 * kBufBytes, wave, lane);
    if (ntiles > 1) issue_tile_dma(p, sg, 1, lds + 1 * kBufBytes, wave, lane);

    vec qa[18];
    if (qk_wave) {
      const int64_t qhead = (int64_t)s * p.Hq + group * kHG + hb * 16 + l16;
      const float* qsrc = p.q_abs + qhead * kDc + 8 * g16;
      const float* rsrc = p.q_rope + qhead * kDr + 8 * g16;
#pragma unroll
      for (int kk = 0; kk < 18; ++kk) {
        const float* src = kk < 16 ? qsrc + 32 * kk : rsrc + 32 * (kk - 16);
        const f32x4 a = *reinterpret_cast<const f32x4*>(src);
        const f32x4 b = *reinterpret_cast<const f32x4*>(src + 4);
        vec v;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          v[e] = (E)(a[e] * p.scale_log2);
          v[4 + e] = (E)(b[e] * p.scale_log2);
        }
        qa[kk] = v;
      }
    }

    float m_run[4], l_run[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      m_run[i] = -INFINITY;
      l_run[i] = 0.f;
    }
    f32x16 acc[kNHB][2];
#pragma unroll
    for (int mb = 0; mb < kNHB; ++mb)
#pragma unroll
      for (int nb = 0; nb < 2; ++nb)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[mb][nb][e] = 0.f;

    wait_vm0();
    lds_barrier();
    rotate_tile<KT>(lds + 0 * kBufBytes, tid);
    if (ntiles > 1) rotate_tile<KT>(lds + 1 * kBufBytes, tid);
    lds_barrier();

    for (int t = 0; t < ntiles; ++t) {
      char* cur = lds + (t % kNBuf) * kBufBytes;
      const int64_t trow0 = sg.seg_lo + (int64_t)t * kT;
      const int hrow = hb * 16 + 4 * g16;  // first of this lane's 4 heads (QK layout)

      // ---- scores: 16 heads x 16 positions per wave ----
      // Row brow, logical chunk 4kk + g16 sits at physical chunk
      // 8(kk>>1) + ((4(kk&1) + g16) ^ (brow&7)): two lane bases (kk even/odd)
      // plus compile-time offsets 128(kk>>1).
      f32x4 sc = {0.f, 0.f, 0.f, 0.f};
      if (qk_wave) {
        f32x4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
        const int brow = 16 * nbq + l16;
        const char* be = cur + brow * kRowBytes + ((g16 ^ (brow & 7)) << 4);
        const char* bo = cur + brow * kRowBytes + (((4 + g16) ^ (brow & 7)) << 4);
#pragma unroll
        for (int kk = 0; kk < 18; kk += 2) {
          const vec b0 = lds_load<vec>(be, 128 * (kk >> 1));
          const vec b1 = lds_load<vec>(bo, 128 * (kk >> 1));
          s0 = O_::mma16(qa[kk], b0, s0);
          s1 = O_::mma16(qa[kk + 1], b1, s1);
        }
        sc = s0 + s1;
        const bool valid = trow0 + brow < sg.seg_hi;
        float mx[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          sc[i] = valid ? sc[i] : -INFINITY;
          float v = sc[i];
          v = fmaxf(v, __shfl_xor(v, 1, 64));
          v = fmaxf(v, __shfl_xor(v, 2, 64));
          v = fmaxf(v, __shfl_xor(v, 4, 64));
          v = fmaxf(v, __shfl_xor(v, 8, 64));
          mx[i] = v;
        }
        if (l16 == 0) *reinterpret_cast<f32x4*>(tmax_s + nbq * kHG + hrow) = f32x4{mx[0], mx[1], mx[2], mx[3]};
      }
      lds_barrier();  // both position halves' tile maxima visible

      if (qk_wave) {
        const f32x4 mo = *reinterpret_cast<const f32x4*>(tmax_s + (1 - nbq) * kHG + hrow);
        const f32x4 mm = *reinterpret_cast<const f32x4*>(tmax_s + nbq * kHG + hrow);
        float alpha[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float m_new = fmaxf(m_run[i], fmaxf(mm[i], mo[i]));
          alpha[i] = m_run[i] == -INFINITY ? 0.f : exp2f(m_run[i] - m_new);
          const E pe = (E)exp2f(sc[i] - m_new);
          *reinterpret_cast<E*>(pbuf + (hrow + i) * kPRowBytes + (16 * nbq + l16) * 2) = pe;
          float ts = (float)pe;
          ts += __shfl_xor(ts, 1, 64);
          ts += __shfl_xor(ts, 2, 64);
          ts += __shfl_xor(ts, 4, 64);
          ts += __shfl_xor(ts, 8, 64);
          l_run[i] = l_run[i] * alpha[i] + ts;
          m_run[i] = m_new;
        }
        if (nbq == 0 && l16 == 0)
          *reinterpret_cast<f32x4*>(alpha_s + hrow) = f32x4{alpha[0], alpha[1], alpha[2], alpha[3]};
      }

      wait_vm0();     // this wave's copies of tile t+1 have landed
      lds_barrier();  // P/alpha of tile t visible; tile t+1 complete; PV(t-1) done

      if (t + 2 < ntiles) issue_tile_dma(p, sg, t + 2, lds + ((t + 2) % kNBuf) * kBufBytes, wave, lane);
      if (t >= 1 && t + 1 < ntiles) rotate_tile<KT>(lds + ((t + 1) % kNBuf) * kBufBytes, tid);

      // ---- O[:, 64w : 64w+64] = alpha * O + P . tile ----
#pragma unroll
      for (int mb = 0; mb < kNHB; ++mb) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const f32x4 a4 = *reinterpret_cast<const f32x4*>(alpha_s + 32 * mb + 8 * q + 4 * (lane >> 5));
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            acc[mb][0][4 * q + r] *= a4[r];
            acc[mb][1][4 * q + r] *= a4[r];
          }
        }
      }
      // B operand rows 16ks + 8(g16>>1) + 4hf + (l16>>2), logical chunk
      // 8w + 4nb + 2(g16&1) + ((l16&3)>>1); row&7 = 4hf + (l16>>2), so the
      // physical chunk is 8w + ((4nb + 2(g16&1) + ((l16&3)>>1)) ^ (4hf + (l16>>2))).
      const char* trb[2][2];
#pragma unroll
      for (int nb = 0; nb < 2; ++nb)
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) {
          const int row = 8 * (g16 >> 1) + 4 * hf + (l16 >> 2);
          const int pj = 8 * wave + ((4 * nb + 2 * (g16 & 1) + ((l16 & 3) >> 1)) ^ (4 * hf + (l16 >> 2)));
          trb[nb][hf] = cur + row * kRowBytes + pj * 16 + 8 * (l16 & 1);
        }
      const char* pa = pbuf + (lane & 31) * kPRowBytes + 16 * (lane >> 5);
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        vec bv[2];
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) {
          i16x8 v;
#pragma unroll
          for (int hf = 0; hf < 2; ++hf) {
            const i16x4 x = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (__attribute__((address_space(3))) i16x4*)(lds_void*)(trb[nb][hf] + 16 * ks * kRowBytes));
#pragma unroll
            for (int e = 0; e < 4; ++e) v[4 * hf + e] = x[e];
          }
          bv[nb] = __builtin_bit_cast(vec, v);
        }
#pragma unroll
        for (int mb = 0; mb < kNHB; ++mb) {
          const vec av = lds_load<vec>(pa, 32 * mb * kPRowBytes + 32 * ks);
#pragma unroll
          for (int nb = 0; nb < 2; ++nb) acc[mb][nb] = O_::mma32(av, bv[nb], acc[mb][nb]);
        }
      }
      lds_barrier();  // PV(t) done with P; rotation of tile t+1 visible
    }

    // ---- segment end: l = l(half 0) + l(half 1); normalise; write the slot ----
    const int64_t slot = (int64_t)chunk + s;
    const int hrow = hb * 16 + 4 * g16;
    if (qk_wave && l16 == 0)
      *reinterpret_cast<f32x4*>(lsum_s + nbq * kHG + hrow) = f32x4{l_run[0], l_run[1], l_run[2], l_run[3]};
    lds_barrier();
    if (qk_wave && nbq == 0 && l16 == 0) {
      const f32x4 l0 = *reinterpret_cast<const f32x4*>(lsum_s + hrow);
      const f32x4 l1 = *reinterpret_cast<const f32x4*>(lsum_s + kHG + hrow);
      f32x4 il;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float lt = l0[i] + l1[i];
        il[i] = 1.f / lt;
        p.part_lse[slot * p.Hq + group * kHG + hrow + i] = m_run[i] + log2f(lt);
      }
      *reinterpret_cast<f32x4*>(invl_s + hrow) = il;
    }
    lds_barrier();
    // head h = 32mb + 8q + 4(lane>>5) + r lies in 16-head block 2mb + (q>>1);
    // hg_heads is a multiple of 16, so validity is uniform per (mb, q).
    float* dst0 = p.part_o + (slot * p.Hq + group * kHG + 4 * (lane >> 5)) * kDc + 64 * wave + (lane & 31);
#pragma unroll
    for (int mb = 0; mb < kNHB; ++mb) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        if ((2 * mb + (q >> 1)) * 16 >= hg_heads) continue;
        const int hbase = 32 * mb + 8 * q;
        const f32x4 il = *reinterpret_cast<const f32x4*>(invl_s + hbase + 4 * (lane >> 5));
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          float* dst = dst0 + (int64_t)(hbase + r) * kDc;
          dst[0] = acc[mb][0][4 * q + r] * il[r];
          dst[32] = acc[mb][1][4 * q + r] * il[r];
        }
      }
    }
    lo = sg.seg_hi;
    ++s;
  }
}

template <typename KT>
hipError_t launch_t(const DecodeProblem& p, hipStream_t stream) {
  static bool attr_set = false;  // per instance; setting it twice is harmless
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&decode_mfma_kernel<KT>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, kLdsBytes);
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  const int groups = (p.Hq + kHG - 1) / kHG;
  const int64_t blocks = (int64_t)((p.num_chunks + 7) / 8) * 8 * groups;
  hipLaunchKernelGGL((decode_mfma_kernel<KT>), dim3((unsigned)blocks), dim3(kThreads), kLdsBytes, stream, p, groups);
  return hipGetLastError();
}

// The kernel uses gfx950-only instructions; cache the answer per device.
bool device_is_gfx950() {
  static std::mutex mu;
  static int cache[64] = {0};  // 0 unknown, 1 yes, 2 no
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return false;
  std::lock_guard<std::mutex> lock(mu);
  if (cache[dev] == 0) {
    hipDeviceProp_t prop;
    bool ok = hipGetDeviceProperties(&prop, dev) == hipSuccess && std::strncmp(prop.gcnArchName, "gfx950", 6) == 0;
    cache[dev] = ok ? 1 : 2;
  }
  return cache[dev] == 1;
}

}  // namespace

int mfma_heads_per_group() { return kHG; }
int mfma_max_chunk_rows() { return kMaxChunkRows; }

bool mfma_supported(const DecodeProblem& p) {
  if (p.kv_dtype != LA_DTYPE_BF16 && p.kv_dtype != LA_DTYPE_F16) return false;
  if (p.dc != kDc || p.dR != kDr || p.Hq % 16 != 0 || p.Hq <= 0) return false;
  if (p.rope_rows > (1 << 24) || (p.rope_rows == 0 && p.total_rows > (1 << 24))) return false;
  // 16-byte aligned cache rows, table rows and query rows
  if ((reinterpret_cast<uintptr_t>(p.kv) & 15) || (reinterpret_cast<uintptr_t>(p.rope_cos) & 15) ||
      (reinterpret_cast<uintptr_t>(p.rope_sin) & 15) || (reinterpret_cast<uintptr_t>(p.q_rope) & 15) ||
      (reinterpret_cast<uintptr_t>(p.q_abs) & 15))
    return false;
  return device_is_gfx950();
}

hipError_t launch_decode_mfma(const DecodeProblem& p, hipStream_t stream) {
  if (p.kv_dtype == LA_DTYPE_BF16) return launch_t<__hip_bfloat16>(p, stream);
  return launch_t<__half>(p, stream);
}

}  // namespace la
