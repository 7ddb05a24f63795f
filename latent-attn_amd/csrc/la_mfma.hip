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
// streams a chunk of the cache once for a group of up to 128 heads.
//
// Work decomposition. 1-D grid over (chunk, head group); when there are
// several head groups, the groups of one chunk get block ids 8 apart (same
// XCD under round-robin dispatch, so re-reads of a tile hit L2). 256 threads
// = 4 waves, one per SIMD; wave w owns heads [32w, 32w+32) of the group. A
// block walks the segments of its chunk (pieces of the chunk inside one
// sequence) in tiles of 32 positions:
//   * Staging: per tile, wave w copies rows 8w..8w+7 HBM->LDS with
//     global_load_lds_dwordx4 (c_t rows, k_rope rows, cos and sin rows: 11
//     copies per wave, no VGPR staging) into a 3-deep ring, two tiles ahead.
//     Inside a row the 16-B chunk j lives at chunk j ^ f(row),
//     f(row) = 2(row&3) | ((row>>2)&1): 8 consecutive rows at one column and
//     4 consecutive rows at two adjacent columns both land in distinct banks.
//     Each wave rotates (RoPE) the k_rope rows it copied itself, so only its
//     own vmcnt has to drain; one s_barrier per tile publishes the tile.
//   * Scores: S^T[32 pos x 32 heads] = sum over 36 k-steps of
//     v_mfma_f32_32x32x16(A = 16 B of a tile row, B = Q^T). Q (pre-scaled by
//     scale*log2(e), 16-bit) stays in 144 VGPRs.
//   * Softmax in base 2, lazily rescaled: P = 2^(s - m) with a running max m
//     that is only raised when a score exceeds it by more than 8 (then O and
//     the running sum are rescaled). P <= 2^8 is exact enough in 16 bits and
//     the 256 O accumulators are almost never touched outside the MFMAs.
//   * PV: O[32 heads x 512] += P[32 x 32] . Tile[32 x 512]: the S^T
//     accumulator layout already is the A-operand layout of P (lane = head,
//     8 positions per k-step), so P never goes through LDS; B = tile columns
//     via ds_read_b64_tr_b16.
//   * At a segment end O / l and the base-2 log-sum-exp m + log2(l) go to
//     partial slot (chunk + sequence); la_proj.hip merges the slots.
#include "la_internal.hpp"

#include <cstring>
#include <mutex>

namespace la {
namespace {

constexpr int kDc = 512;
constexpr int kDr = 64;
constexpr int kT = 32;                 // positions per tile
constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;
constexpr int kHG = 128;               // heads per group (block)
constexpr int kCtBytes = kT * kDc * 2;       // 32768: c_t rows, 1024 B each
constexpr int kRopeOff = kCtBytes;           // k_rope rows, 128 B each
constexpr int kCosOff = kRopeOff + kT * 128; // cos rows (32 floats)
constexpr int kSinOff = kCosOff + kT * 128;  // sin rows
constexpr int kBufBytes = kSinOff + kT * 128;  // 45056
constexpr int kNBuf = 3;
constexpr int kScratchOff = kNBuf * kBufBytes;  // per-wave 32 floats
constexpr int kQropeOff = kScratchOff + kWaves * 32 * 4;  // q_rope of the group: 128 rows x 128 B
constexpr int kLdsBytes = kQropeOff + kHG * kDr * 2;
constexpr int kDmaPerWave = 11;        // 8 c_t rows + k_rope + cos + sin
constexpr int kRescaleSlack = 8;       // log2 units before the running max moves
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

template <typename KT>
struct Ops;

// The attention kernel issues its MFMAs as inline asm so that the register
// classes are fixed: the score tile S accumulates in VGPRs (mma_v0 / mma_v)
// and the 256 O accumulators stay in AGPRs (mma_a) across the tile loop --
// left to itself the compiler puts both in AGPRs and spills. The compiler
// does not see inside the asm, so wait states are explicit: a VALU read of an
// MFMA result goes after settle()/settle_acc() (32 wait states), an MFMA that
// reads VALU-written operands after operands_ready() (8 wait states). Chained
// MFMAs on the same accumulator need none (the hardware interlocks srcC ==
// vdst of the same opcode).
template <>
struct Ops<__hip_bfloat16> {
  typedef bf16x8 vec;
  typedef __bf16 elem;
  static __device__ inline f32x16 mma(vec a, vec b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
  static __device__ inline void mma_v0(f32x16& d, vec a, vec b) {
    asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, 0" : "=&v"(d) : "v"(a), "v"(b));
  }
  static __device__ inline void mma_v(f32x16& d, vec a, vec b) {
    asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(d) : "v"(a), "v"(b));
  }
  static __device__ inline void mma_a(f32x16& d, vec a, vec b) {
    asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(d) : "v"(a), "v"(b));
  }
};

template <>
struct Ops<__half> {
  typedef f16x8 vec;
  typedef _Float16 elem;
  static __device__ inline f32x16 mma(vec a, vec b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
  static __device__ inline void mma_v0(f32x16& d, vec a, vec b) {
    asm volatile("v_mfma_f32_32x32x16_f16 %0, %1, %2, 0" : "=&v"(d) : "v"(a), "v"(b));
  }
  static __device__ inline void mma_v(f32x16& d, vec a, vec b) {
    asm volatile("v_mfma_f32_32x32x16_f16 %0, %1, %2, %0" : "+v"(d) : "v"(a), "v"(b));
  }
  static __device__ inline void mma_a(f32x16& d, vec a, vec b) {
    asm volatile("v_mfma_f32_32x32x16_f16 %0, %1, %2, %0" : "+a"(d) : "v"(a), "v"(b));
  }
};

// 32 wait states after the last inline-asm MFMA writing d0/d1 and before any
// other instruction reads them (covers the MFMA-result -> VALU read hazard
// for up to 16-pass MFMAs). Taking d0/d1 as in-out operands orders every
// later use after it.
__device__ inline void settle(f32x16& d0, f32x16& d1) {
  asm volatile("s_nop 15\n\ts_nop 15" : "+v"(d0), "+v"(d1));
}

__device__ inline void settle1(f32x16& d0) { asm volatile("s_nop 15\n\ts_nop 15" : "+v"(d0)); }

// 32 wait states before the O accumulators (AGPRs written by MFMAs) are read
// or rewritten by VALU code; every later access is ordered after it.
__device__ inline void settle_acc(f32x16 (&acc)[16]) {
  asm volatile("s_nop 15\n\ts_nop 15" : "+a"(acc[0]), "+a"(acc[1]), "+a"(acc[2]), "+a"(acc[3]), "+a"(acc[4]),
               "+a"(acc[5]), "+a"(acc[6]), "+a"(acc[7]), "+a"(acc[8]), "+a"(acc[9]), "+a"(acc[10]), "+a"(acc[11]),
               "+a"(acc[12]), "+a"(acc[13]), "+a"(acc[14]), "+a"(acc[15]));
}

// Forces one accumulator block back into AGPRs at this point (no code).
__device__ inline void pin_agpr(f32x16& d) { asm volatile("" : "+a"(d)); }

// 8 wait states between VALU/v_accvgpr_write producers and MFMA consumers.
template <typename V>
__device__ inline void operands_ready(V& a, V& b) {
  asm volatile("s_nop 7" : "+v"(a), "+v"(b));
}
__device__ inline void acc_ready(f32x16 (&acc)[16]) {
  asm volatile("s_nop 7" : "+a"(acc[0]), "+a"(acc[1]), "+a"(acc[2]), "+a"(acc[3]), "+a"(acc[4]), "+a"(acc[5]),
               "+a"(acc[6]), "+a"(acc[7]), "+a"(acc[8]), "+a"(acc[9]), "+a"(acc[10]), "+a"(acc[11]), "+a"(acc[12]),
               "+a"(acc[13]), "+a"(acc[14]), "+a"(acc[15]));
}

__device__ inline int swzf(int row) { return ((row & 3) << 1) | ((row >> 2) & 1); }

// vmcnt(n) with the other counters left alone (gfx9 encoding, n < 16).
template <int N>
__device__ inline void wait_vm() {
  static_assert(N >= 0 && N < 16, "vmcnt range");
  __builtin_amdgcn_s_waitcnt(0x0F70 | N);
}

// LDS-visibility barrier that leaves outstanding HBM->LDS copies in flight.
// The "memory" clobber keeps the compiler from moving LDS accesses across it.
__device__ inline void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Returns x through an empty asm: values computed from the result cannot be
// hoisted out of the enclosing loop. Used on the lane index at the top of each
// tile so per-lane addresses are recomputed (a few VALU ops) instead of being
// kept live across the loop in dozens of VGPRs.
__device__ inline int opaque(int x) {
  asm volatile("" : "+v"(x));
  return x;
}

// LDS is addressed with 32-bit byte offsets from the start of the dynamic LDS
// block (address-space-3 pointers), never with 64-bit generic pointers.
typedef __attribute__((address_space(3))) char lchar;

template <typename T>
__device__ inline T lds_ld(const lchar* L, uint32_t off) {
  return *reinterpret_cast<const __attribute__((address_space(3))) T*>(L + off);
}
template <typename T>
__device__ inline void lds_st(lchar* L, uint32_t off, T v) {
  *reinterpret_cast<__attribute__((address_space(3))) T*>(L + off) = v;
}
// ds_read_b64_tr_b16 as inline asm: the builtin makes the compiler assume the
// read may alias the in-flight HBM->LDS copies and drain vmcnt before it. The
// asm result must not be used before b_wait() (lgkmcnt).
__device__ inline i16x4 lds_tr(const lchar* L, uint32_t off) {
  i16x4 r;
  const uint32_t addr = (uint32_t)(uintptr_t)(L + off);
  asm volatile("ds_read_b64_tr_b16 %0, %1" : "=v"(r) : "v"(addr));
  return r;
}

struct TrPair {
  i16x4 x0, x1;
};

struct SegCtx {
  const char* base;  // first byte of the segment's first row
  int64_t pos0;      // in-sequence position of the segment's first row
  int last;          // index of the segment's last row, relative to its first
};

// Wave w's 11 HBM->LDS copies for tile k into the buffer at LDS offset buf:
// c_t of rows 8w..8w+7 (one copy per row), then their k_rope, cos and sin rows
// (one copy each). Global addresses are a wave-uniform base plus a 32-bit lane
// offset (segments are capped at kMaxChunkRows rows, tables at 2^24 rows).
// Rows past the segment end re-read its last row; their scores are masked.
__device__ inline void issue_tile_dma(const DecodeProblem& p, const SegCtx& sg, int k, lchar* L, uint32_t buf,
                                      int wave, int lane) {
  const int r_first = 8 * wave;
#pragma unroll
  for (int rr = 0; rr < 8; ++rr) {
    const int row = r_first + rr;
    const int r = min(k * kT + row, sg.last);
    const int j = lane ^ swzf(rr);  // row & 7 == rr
    __builtin_amdgcn_global_load_lds(sg.base + (uint32_t)(r * (kDc + kDr) * 2 + j * 16),
                                     (lds_void*)(L + buf + row * 1024), 16, 0, 0);
  }
  const int row = r_first + (lane >> 3);
  const int r = min(k * kT + row, sg.last);
  const int jr = (lane & 7) ^ swzf(lane >> 3);  // row & 7 == lane >> 3
  __builtin_amdgcn_global_load_lds(sg.base + (uint32_t)(r * (kDc + kDr) * 2 + kDc * 2 + jr * 16),
                                   (lds_void*)(L + buf + kRopeOff + r_first * 128), 16, 0, 0);
  const uint32_t toff = (uint32_t)(rope_row(p, sg.pos0 + r) * (kDr / 2) * 4 + (lane & 7) * 16);
  __builtin_amdgcn_global_load_lds(reinterpret_cast<const char*>(p.rope_cos) + toff,
                                   (lds_void*)(L + buf + kCosOff + r_first * 128), 16, 0, 0);
  __builtin_amdgcn_global_load_lds(reinterpret_cast<const char*>(p.rope_sin) + toff,
                                   (lds_void*)(L + buf + kSinOff + r_first * 128), 16, 0, 0);
}

// Rotate-half RoPE of rows 8w..8w+7 of the tile at LDS offset buf, in place
// (src/fused_mla.cu:43-51): r[i] = k[i]*c - k[i+32]*s, r[i+32] = k[i]*s +
// k[i+32]*c. Lane: row 8w + lane/8, pairs i = 4(lane%8) .. +3.
template <typename KT>
__device__ inline void rotate_rows(lchar* L, uint32_t buf, int wave, int lane) {
  typedef typename Ops<KT>::elem E;
  const int rl = lane >> 3, u = lane & 7;
  const int row = 8 * wave + rl;
  const int f = swzf(rl);
  const uint32_t pa = buf + kRopeOff + row * 128 + (((u >> 1) ^ f) << 4) + 8 * (u & 1);
  const uint32_t pb = buf + kRopeOff + row * 128 + (((4 + (u >> 1)) ^ f) << 4) + 8 * (u & 1);
  const i16x4 ka = lds_ld<i16x4>(L, pa);
  const i16x4 kb = lds_ld<i16x4>(L, pb);
  const f32x4 c = lds_ld<f32x4>(L, buf + kCosOff + row * 128 + 16 * u);
  const f32x4 s = lds_ld<f32x4>(L, buf + kSinOff + row * 128 + 16 * u);
  i16x4 ra, rb;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float k0 = (float)__builtin_bit_cast(E, (short)ka[e]);
    const float k1 = (float)__builtin_bit_cast(E, (short)kb[e]);
    ra[e] = __builtin_bit_cast(short, (E)(k0 * c[e] - k1 * s[e]));
    rb[e] = __builtin_bit_cast(short, (E)(k0 * s[e] + k1 * c[e]));
  }
  lds_st(L, pa, ra);
  lds_st(L, pb, rb);
}

// Block id -> (chunk, head group).
__device__ inline void block_coords(int groups, int* chunk, int* group) {
  const int id = blockIdx.x;
  if (groups == 1) {
    *chunk = id;
    *group = 0;
    return;
  }
  const int x = id & 7, k = id >> 3;
  *group = k % groups;
  *chunk = (k / groups) * 8 + x;
}

template <typename KT>
__global__ __launch_bounds__(kThreads) void decode_mfma_kernel(DecodeProblem p, int groups) {
  typedef Ops<KT> O_;
  typedef typename O_::vec vec;
  typedef typename O_::elem E;

  extern __shared__ __attribute__((aligned(1024))) char lds_raw[];
  lchar* L = (lchar*)lds_raw;
  const int tid = threadIdx.x, lane0 = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: keep in SGPRs
  int chunk, group;
  block_coords(groups, &chunk, &group);
  if (chunk >= p.num_chunks) return;
  const int hg_heads = min(kHG, p.Hq - group * kHG);
  const uint32_t scratch = kScratchOff + 128 * wave;  // per-wave 32 floats

  const int64_t end_all = seq_begin(p, p.num_seqs);
  int64_t lo = (int64_t)chunk * p.chunk_len;
  const int64_t hi = min(lo + (int64_t)p.chunk_len, end_all);
  lo = max(lo, seq_begin(p, 0));
  if (lo >= hi) return;
  int s = find_seq(p, lo);

  while (lo < hi) {
    const int64_t s_lo = seq_begin(p, s), s_hi = seq_begin(p, s + 1);
    if (s_hi <= lo) {
      ++s;
      continue;
    }
    const int64_t seg_hi = min(hi, s_hi);
    SegCtx sg;
    sg.base = reinterpret_cast<const char*>(p.kv) + lo * (kDc + kDr) * 2;
    sg.pos0 = lo - s_lo;
    sg.last = (int)(seg_hi - lo - 1);
    const int seg_len = sg.last + 1;
    const int ntiles = (seg_len + kT - 1) / kT;

    lds_barrier();  // all waves are done with the previous segment's buffers

    issue_tile_dma(p, sg, 0, L, 0, wave, lane0);
    if (ntiles > 1) issue_tile_dma(p, sg, 1, L, kBufBytes, wave, lane0);

    // Q^T as the B operand: lane holds Q[head][16kk + 8*g2 .. +8], pre-scaled.
    // The 32 latent k-steps stay in VGPRs; the 4 rope k-steps go to this
    // wave's rows of an LDS table (row = head, 16-B chunk j at j ^ (head & 7))
    // to save 16 VGPRs.
    vec qb[32];
    {
      const int g2 = lane0 >> 5;
      const int head = 32 * wave + (lane0 & 31);
      const bool head_ok = head < hg_heads;
      const int64_t qrow = (int64_t)s * p.Hq + group * kHG + (head_ok ? head : 0);
      const float* qsrc = p.q_abs + qrow * kDc + 8 * g2;
      const float* rsrc = p.q_rope + qrow * kDr + 8 * g2;
      const float sc = head_ok ? p.scale_log2 : 0.f;
#pragma unroll
      for (int kk = 0; kk < 36; ++kk) {
        const float* src = kk < 32 ? qsrc + 16 * kk : rsrc + 16 * (kk - 32);
        const f32x4 a = *reinterpret_cast<const f32x4*>(src);
        const f32x4 b = *reinterpret_cast<const f32x4*>(src + 4);
        vec v;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          v[e] = (E)(a[e] * sc);
          v[4 + e] = (E)(b[e] * sc);
        }
        if (kk < 32) {
          qb[kk] = v;
        } else {
          const int j = 2 * (kk - 32) + g2;
          lds_st(L, kQropeOff + head * 128 + ((j ^ (head & 7)) << 4), v);
        }
        __builtin_amdgcn_sched_barrier(0);  // bound the loads in flight (register pressure)
      }
    }

    float m_run = -INFINITY, l_run = 0.f;
    f32x16 acc[16];
#pragma unroll
    for (int nb = 0; nb < 16; ++nb)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[nb][e] = 0.f;
    acc_ready(acc);

    wait_vm<0>();
    rotate_rows<KT>(L, 0, wave, lane0);
    if (ntiles > 1) rotate_rows<KT>(L, kBufBytes, wave, lane0);

    for (int t = 0; t < ntiles; ++t) {
      lds_barrier();  // tile t staged and rotated by every wave; tile t-1 fully consumed
      const int lane = opaque(tid & 63);
      const int g2 = lane >> 5;
      const int q16 = lane >> 4, s16 = lane & 15;
      const int head = 32 * wave + (lane & 31);
      if (t + 2 < ntiles) issue_tile_dma(p, sg, t + 2, L, ((t + 2) % kNBuf) * kBufBytes, wave, lane);
      const uint32_t cur = (t % kNBuf) * kBufBytes;

      // ---- S^T[pos][head] over 36 k-steps (32 latent + 4 rope) ----
      // A operand of k-step kk: row arow, logical chunk 2kk + g2, stored at
      // 2(kk ^ (af>>1)) + (g2 ^ (af&1)). For kk = 4m + r that is byte offset
      // 128m + 32(r ^ (af>>1)) + 16(g2 ^ (af&1)). A operands are prefetched two
      // k-steps ahead.
      const int arow = lane & 31;
      const int af = swzf(arow & 7);
      const uint32_t ct_row = cur + arow * 1024 + 16 * (g2 ^ (af & 1));
      const uint32_t rp_row = cur + kRopeOff + arow * 128 + 16 * (g2 ^ (af & 1));
      auto a_off = [&](int kk) -> uint32_t {
        const uint32_t o = 32 * ((kk & 3) ^ (af >> 1)) + 128 * (kk >> 2);
        return kk < 32 ? ct_row + o : rp_row + o - 128 * 8;
      };
      const uint32_t qr_row = kQropeOff + head * 128;
      // two independent accumulation chains (even / odd k-steps)
      f32x16 s0, s1;
      vec an0 = lds_ld<vec>(L, a_off(0)), an1 = lds_ld<vec>(L, a_off(1));
#pragma unroll
      for (int kk = 0; kk < 36; kk += 2) {
        const vec a0 = an0, a1 = an1;
        if (kk + 2 < 36) {
          an0 = lds_ld<vec>(L, a_off(kk + 2));
          an1 = lds_ld<vec>(L, a_off(kk + 3));
        }
        if (kk == 0) {
          O_::mma_v0(s0, a0, qb[0]);
          O_::mma_v0(s1, a1, qb[1]);
        } else if (kk < 32) {
          O_::mma_v(s0, a0, qb[kk]);
          O_::mma_v(s1, a1, qb[kk + 1]);
        } else {
          const vec b0 = lds_ld<vec>(L, qr_row + (((2 * (kk - 32) + g2) ^ (head & 7)) << 4));
          const vec b1 = lds_ld<vec>(L, qr_row + (((2 * (kk - 31) + g2) ^ (head & 7)) << 4));
          O_::mma_v(s0, a0, b0);
          O_::mma_v(s1, a1, b1);
        }
      }
      settle(s0, s1);
      f32x16 sc = s0 + s1;

      // ---- lazy online softmax; lane = head, 16 positions 8(i/4)+4*g2+(i%4) ----
      const int valid = min(kT, seg_len - t * kT);
      float lmax = -INFINITY;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int pos = 8 * (i >> 2) + 4 * g2 + (i & 3);
        sc[i] = pos < valid ? sc[i] : -INFINITY;
        lmax = fmaxf(lmax, sc[i]);
      }
      const bool need = lmax > m_run + (float)kRescaleSlack;
      if (__builtin_amdgcn_ballot_w64(need) != 0) {
        const float tmax = fmaxf(lmax, __shfl_xor(lmax, 32, 64));
        const float m_new = fmaxf(m_run, tmax);
        const bool first = m_run == -INFINITY;
        const float alpha = first ? 0.f : exp2f(m_run - m_new);
        m_run = m_new;
        l_run *= alpha;
        // O rows are heads 8(i/4) + 4*g2 + (i%4); alpha of head h sits in lane h.
        if (__builtin_amdgcn_ballot_w64(!first && alpha != 1.f) != 0) {
          if (lane < 32) lds_st(L, scratch + 4 * lane, alpha);
          __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): own LDS write before own read
          settle_acc(acc);
          f32x16 a16;
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const f32x4 a4 = lds_ld<f32x4>(L, scratch + 4 * (8 * q + 4 * g2));
#pragma unroll
            for (int r = 0; r < 4; ++r) a16[4 * q + r] = a4[r];
          }
          // one 16-register block at a time, pinned back to AGPRs after each,
          // so the rescale needs 16 temporaries instead of 256
#pragma unroll
          for (int nb = 0; nb < 16; ++nb) {
            acc[nb] *= a16;
            pin_agpr(acc[nb]);
            __builtin_amdgcn_sched_barrier(0);
          }
          acc_ready(acc);
        }
      }
      vec pv[2];
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const E pe = (E)exp2f(sc[8 * ks + j] - m_run);
          pv[ks][j] = pe;
          l_run += (float)pe;
        }
      }
      operands_ready(pv[0], pv[1]);

      // ---- O[head][c] += P[head][pos] . tile[pos][c], 16 column blocks ----
      // B operand for (ks, nb): rows 16ks + 8hf + 4(q16>>1) + (s16>>2) (row&7
      // does not depend on ks, hf), logical chunk 4nb + jlo with
      // jlo = 2(q16&1) + ((s16&3)>>1). With F = swzf(row), the physical chunk is
      // 4(nb ^ (F>>2)) + (jlo ^ (F&3)): byte offset 64nb +- 64(F>>2) (sign by the
      // parity of nb) + 16(jlo ^ (F&3)) -- two lane bases plus immediates.
      const int trow = 4 * (q16 >> 1) + (s16 >> 2);
      const int tf = swzf(trow);
      const uint32_t tb = cur + trow * 1024 + 16 * ((2 * (q16 & 1) + ((s16 & 3) >> 1)) ^ (tf & 3)) + 8 * (s16 & 1);
      const uint32_t tb_even = tb + 64 * (tf >> 2);
      const uint32_t tb_odd = tb - 64 * (tf >> 2);
      // The two transposed reads of step s+1 are issued before the MFMA of
      // step s; lgkmcnt(2) then guarantees everything older than them (the
      // reads of step s) has landed (LDS operations complete in order). The
      // wait takes the raw read registers as operands so nothing copies them
      // earlier.
      auto b_issue = [&](int step) -> TrPair {
        const int ks = step >> 4, nb = step & 15;
        const uint32_t base = ((nb & 1) ? tb_odd : tb_even) + 64 * nb;
        TrPair r;
        r.x0 = lds_tr(L, base + (16 * ks) * 1024);
        r.x1 = lds_tr(L, base + (16 * ks + 8) * 1024);
        return r;
      };
      TrPair bn = b_issue(0);
#pragma unroll
      for (int step = 0; step < 32; ++step) {
        TrPair bc = bn;
        if (step + 1 < 32) {
          bn = b_issue(step + 1);
          asm volatile("s_waitcnt lgkmcnt(2)" : "+v"(bc.x0), "+v"(bc.x1));
        } else {
          asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(bc.x0), "+v"(bc.x1));
        }
        i16x8 bv;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          bv[e] = bc.x0[e];
          bv[4 + e] = bc.x1[e];
        }
        O_::mma_a(acc[step & 15], pv[step >> 4], __builtin_bit_cast(vec, bv));
      }

      if (t + 1 < ntiles && t >= 1) {
        if (t + 2 < ntiles) wait_vm<kDmaPerWave>();
        else wait_vm<0>();
        rotate_rows<KT>(L, ((t + 1) % kNBuf) * kBufBytes, wave, lane);
      }
    }

    // ---- segment end: l over both lane halves; normalise; write the slot ----
    settle_acc(acc);
    const int g2 = lane0 >> 5;
    const float l_tot = l_run + __shfl_xor(l_run, 32, 64);
    const int64_t slot = (int64_t)chunk + s;
    const int64_t hq0 = slot * p.Hq + group * kHG + 32 * wave;
    if (lane0 < 32) {
      lds_st(L, scratch + 4 * lane0, 1.f / l_tot);
      if (32 * wave + lane0 < hg_heads) p.part_lse[hq0 + lane0] = m_run + log2f(l_tot);
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);
    f32x16 il16;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const f32x4 il = lds_ld<f32x4>(L, scratch + 4 * (8 * q + 4 * g2));
#pragma unroll
      for (int r = 0; r < 4; ++r) il16[4 * q + r] = il[r];
    }
    // register i of block nb: head 8(i/4) + 4*g2 + (i%4), column 32nb + lane%32.
    // Heads come in 16-aligned groups, so validity is uniform per i.
    float* dst0 = p.part_o + hq0 * kDc + (lane0 & 31);
#pragma unroll
    for (int nb = 0; nb < 16; ++nb) {
      const f32x16 v = acc[nb] * il16;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int hh = 8 * (i >> 2) + 4 * g2 + (i & 3);
        if (32 * wave + hh < hg_heads) dst0[(int64_t)hh * kDc + 32 * nb] = v[i];
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    lo = seg_hi;
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
  const int64_t blocks = groups == 1 ? p.num_chunks : (int64_t)((p.num_chunks + 7) / 8) * 8 * groups;
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
