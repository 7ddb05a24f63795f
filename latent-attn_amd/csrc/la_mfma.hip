// MFMA split-KV MLA decode kernel for gfx950 (MI355X): 16-bit latent cache
// (bf16 or fp16) or FP8 E4M3 cache (copied as fp8, expanded to bf16 tiles in
// LDS), kv_lora_rank 512, qk_rope_head_dim 64.
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
// Work decomposition. 1-D grid over (chunk, head group), mapped XCD-aware
// (block_coords): each XCD gets a contiguous range of chunks, so the chunks
// of one sequence (and the head groups of one chunk) share an L2. 256 threads
// = 4 waves, one per SIMD; wave w owns heads [32w, 32w+32) of the group. A
// block walks the segments of its chunk (pieces of the chunk inside one
// sequence) in tiles of 32 positions:
//   * Staging: per tile, wave w copies rows 8w..8w+7 HBM->LDS with
//     global_load_lds_dwordx4 (c_t rows, k_rope rows, cos and sin rows: 11
//     copies per wave, no VGPR staging) into a 3-deep ring, two tiles ahead.
//     c_t row r sits at ct_row_off(r) = 1088r + 16((r/4)%4), unswizzled (one
//     lane offset serves every row copy); inside a k_rope row the
//     16-B chunk j lives at j ^ fr(row), fr(row) = (row>>1)&7. With 64 banks
//     of 4 B both the score reads (16 rows at one column per 16 lanes) and the
//     transposed value reads (4 rows x 4 columns per 16 lanes) are
//     conflict-free, and c_t reads need no per-read address arithmetic.
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
//   * At a segment end O / l (fp16, with a power-of-two scale per row) and
//     the base-2 log-sum-exp m + log2(l) go to partial slot (chunk +
//     sequence); la_proj.hip merges the slots.
#include "la_internal.hpp"

#include <hip/hip_ext.h>

#include <cstring>
#include <mutex>
#include <type_traits>

namespace la {

// Phase-timing build only (-DLA_PHASE_STAMPS: build.py --phase-stamps, read
// by phase_profile.py; the shipped library has none of it). Every wave of
// the attention kernel records the shader clock (s_memtime) at the phase
// boundaries of its last segment and writes the 11 values at exit:
//   0 entry (after the first round of argument loads)  1 segment set up
//   2 past the segment's opening barrier  3 Q loads issued
//   4 tile 0 landed  5 tile 0 rotated  6 loop at t = 0 (after iteration -1)
//   7 loop done  8 past the staging barrier  9 partial stores issued
//   10 stores complete
// and, summed over the iterations t >= 0 of the segment, the cycles of each
// iteration's parts: 11 the barrier (from the iteration's start), 12 QK(t+1)
// with the copies of tile t+2, 13 PV(t) with softmax(t+1), the RoPE of tile
// t+2 and the P publication, 14 the wait for the iteration's copies; 15 the
// number of those iterations.
// A stamp waits for the scalar data path (lgkmcnt), which drains the wave's
// LDS queue: the instrumented kernel runs a few per cent slower.
#ifdef LA_PHASE_STAMPS
constexpr int kStampSlots = 16;
constexpr int kStampBlocks = 4096;
__device__ unsigned long long g_attn_stamps[kStampBlocks * 4 * kStampSlots];
#define LA_STAMP(i)                                                                                  \
  do {                                                                                               \
    unsigned long long t_;                                                                           \
    asm volatile("s_memtime %0\n\ts_waitcnt lgkmcnt(0)" : "=s"(t_)::"memory");                       \
    stamps_[i] = t_;                                                                                 \
  } while (0)
#define LA_TSTAMP(v) asm volatile("s_memtime %0\n\ts_waitcnt lgkmcnt(0)" : "=s"(v)::"memory")
#else
#define LA_STAMP(i) ((void)0)
#endif

namespace {

constexpr int kDc = 512;
constexpr int kDr = 64;
constexpr int kT = 32;                 // positions per tile
constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;
constexpr int kHG = 128;               // heads per group (block)
// c_t row r of a tile starts at LDS byte ct_row_off(r) of its buffer: pitch
// 1088 B (64 B past a multiple of 256) plus 16 ((r/4) % 4) B, i.e. in 16-B
// bank slots row r starts at slot 4(r%4) + (r/4)%4 (mod 16), a rotation that
// spreads the rows without overlapping them. Every read of a tile (score A
// operands: 16 rows at one chunk per 16 lanes; value reads: 4 consecutive
// rows x 32 B per 16 lanes, x 64 B per 32) then hits distinct banks, and
// every address is a lane base plus an instruction immediate.
constexpr int kRowPitch = 1088;
__host__ __device__ constexpr int ct_row_off(int r) { return r * kRowPitch + 16 * ((r >> 2) & 3); }
constexpr int kCtBytes = ct_row_off(kT - 1) + kDc * 2;  // 34800
// k_rope rows, 128 B each; 128-aligned (as is every buffer) because their
// swizzled addresses are built with OR / XOR on the low 7 bits
constexpr int kRopeOff = (kCtBytes + 127) / 128 * 128;  // 34816
constexpr int kBufBytes = kRopeOff + kT * 128;          // 38912: one tile
static_assert(kRopeOff % 128 == 0 && kBufBytes % 128 == 0, "k_rope rows must be 128-aligned");
constexpr int kNBuf = 3;
// cos / sin rows (32 floats each) of the tile being staged. They are read
// only by that tile's RoPE, in the iteration that copies them, so one buffer
// serves every tile.
constexpr int kCosOff = kNBuf * kBufBytes;
constexpr int kSinOff = kCosOff + kT * 128;
constexpr int kPtabOff = kSinOff + kT * 128;          // P operands: [parity][wave][ks][lane] 16 B
constexpr int kPtabPar = kWaves * 2 * 1024;
constexpr int kAtabWave = 160;                        // per wave: 32 alphas, rescale flag at +128
constexpr int kAtabOff = kPtabOff + 2 * kPtabPar;     // [parity][wave]
constexpr int kAtabPar = kWaves * kAtabWave;
constexpr int kLdsBytes = kAtabOff + 2 * kAtabPar;
// epilogue staging: per wave 64 fp16 half rows (512 B) at a 528-B pitch
constexpr int kStagePitch = 528;
constexpr int kStageBytes = 64 * kStagePitch;
static_assert(kWaves * kStageBytes <= kLdsBytes, "epilogue staging fits the LDS block");
constexpr int kDmaPerWave = 11;        // 8 c_t rows + k_rope + cos + sin
constexpr int kRescaleSlack = 8;       // log2 units before the running max moves
constexpr int kQkDepth = 6;            // score A operands read this many k-steps ahead
constexpr int kPvSteps = 16;           // PV operand steps: (ks, column block), 2 MFMAs each
constexpr int kPvDepth = 4;            // value-read pairs in flight (2 reads per step, lgkmcnt <= 15)
constexpr int kRotStep = 9;            // PV step after which the RoPE reads of tile t+2 are issued
constexpr int kRotSlot0 = 24;          // PV slots kRotSlot0 .. +6 rotate and store them
// PV steps from kPostStep0 on keep their odd slot after their second MFMA
// (the compiler would hoist it above the MFMA, next to the even slot)
constexpr int kPostStep0 = 12, kPostStep1 = 14;
// LDS operations a 16-bit cache's wave issues after its RoPE reads (step
// kRotStep, after its value reads) and before PV slot kRotSlot0 (an even slot:
// before that step's value reads): the value-read pairs of the steps between
constexpr int rot_later() {
  int n = 0;
  for (int s = kRotStep + 1; s < kRotSlot0 / 2; ++s)
    if (s + kPvDepth < kPvSteps) n += 2;
  return n;
}
static_assert(kRotSlot0 % 2 == 0 && kRotSlot0 / 2 > kRotStep && rot_later() < 16, "RoPE wait count");
// FP8 cache: the expansion of tile t+2's staged rows to bf16 runs inside PV(t):
// rows 0..3 of the wave are read at step kRotStep (after the RoPE reads),
// everything is waited for at step kExpWaitStep, rows 0..3 are converted and
// stored in slots kExpSlot0 .. +3, rows 4..7 read after that and converted
// and stored in slots kExpSlot0 + 4 .. +7.
constexpr int kExpWaitStep = 12;
constexpr int kExpSlot0 = 2 * kExpWaitStep;
// Copy J of a tile goes out at QK step copy_step(i) for i with J =
// dma_order(i): k_rope, cos and sin first, so the RoPE of the tile only waits
// for those.
constexpr int kCopyFirst = 2, kCopyStride = 3;
constexpr int copy_step(int i) { return kCopyFirst + kCopyStride * i; }
constexpr int dma_order(int i) { return (i + 8) % 11; }
constexpr int kQrAt = 32 - kQkDepth;   // QK step before which the partner-P reads are issued
constexpr int kTrAt = 36 - kPvDepth;   // QK steps kTrAt.. issue the first kPvDepth PV value-read pairs
constexpr int kSmSettle = 1;           // softmax slot (two per PV step) that starts softmax(t+1)
constexpr int kSmPipe0 = 4;            // PV steps kSmPipe0 .. +8 run the exp2 pipeline (one score pair each)
constexpr int kSmDone = 26;            // softmax slot that takes the summed l
// the softmax's slots in order: settle / mask, 4 max-tree slots, the running
// max (kSmSettle + 5), the exp2 pipeline (its own lead / mid pieces of PV
// steps kSmPipe0 .. +8, after the running max), then l: overlapping ranges
// would drop a piece (each slot runs one branch of sm_piece)
static_assert(2 * kSmPipe0 > kSmSettle + 5 && kSmDone > 2 * (kSmPipe0 + 8) && kSmDone < 2 * kPvSteps,
              "softmax slots in order, inside PV");

// LDS issue order of one iteration (all reads counted by lgkmcnt):
//   QK:  [partner flag] A(0..D-1); per step kk: [kk == kQrAt: 2 partner-P
//        reads] wait A(kk), MFMA, A(kk+D), [kk >= kTrAt:
//        value-read pair kk-kTrAt];
//   PV:  per step s: wait pair s, 2 MFMAs, pair s+kPvDepth, [s == kRotStep:
//        4 RoPE reads].
// qk_later(kk) / pv_later(s) = LDS reads issued after the awaited one and
// before its wait; lgkmcnt(that) then guarantees it has completed.
constexpr int qk_later(int kk) {
  const int D = kQkDepth;
  int seq = 0, seq_a = -1;
  for (int j = 0; j < D; ++j) {
    if (j == kk) seq_a = seq;
    ++seq;
  }
  for (int k = 0; k <= kk; ++k) {
    if (k == kQrAt) seq += 2;
    if (k == kk) return seq - seq_a - 1;
    if (k + D < 36) {
      if (k + D == kk) seq_a = seq;
      ++seq;
    }
    if (k >= kTrAt && k - kTrAt < kPvDepth) seq += 2;
  }
  return -1;
}
constexpr int pv_later(int s) {
  // pairs 0..kPvDepth-1 were issued at the end of QK, back to back
  int seq = 2 * kPvDepth, seq_s = s < kPvDepth ? 2 * s : -1;
  for (int k = 0; k <= s; ++k) {
    if (k == s) return seq - seq_s - 2;
    if (k + kPvDepth < kPvSteps) {
      if (k + kPvDepth == s) seq_s = seq;
      seq += 2;
    }
    if (k == kRotStep) seq += 4;
  }
  return -1;
}
// The lgkmcnt of PV step s's value-read wait. FP8 cache: the 4 expansion
// reads of rows 0..3 go out with the RoPE reads at kRotStep (4 more later
// operations for steps up to kExpWaitStep - 1); step kExpWaitStep waits for
// everything issued so far (lgkmcnt 0), so the later steps' pairs are complete
// and their waits only order the registers (15: never binding, at most 8 LDS
// operations are outstanding then).
constexpr int pv_wait_n(int s, bool fp8) {
  if (!fp8 || s <= kRotStep) return pv_later(s);
  if (s < kExpWaitStep) return pv_later(s) + 4 < 15 ? pv_later(s) + 4 : 15;
  return s == kExpWaitStep ? 0 : 15;
}
static_assert(pv_wait_n(kExpWaitStep - 1, true) == pv_later(kExpWaitStep - 1) + 4, "fp8 expansion reads counted exactly");
static_assert(kExpWaitStep > kRotStep && kExpWaitStep + 3 < kPvSteps && kExpSlot0 + 7 < 2 * kPvSteps,
              "fp8 expansion slots inside PV");
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
  // mma_v with the A operand's LDS wait (lgkmcnt(N)) in the same asm
  // statement: as separate statements the compiler pads a wait state between
  // them. mma_v_lvw / mma_v0_lvw: also the wait for the Q loads of operands b
  // and q1 .. q5 (vmcnt(M)), which the statement marks as produced.
  template <int N>
  static __device__ inline void mma_v_lw(f32x16& d, vec a, vec b) {
    asm volatile("s_waitcnt lgkmcnt(%3)\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(d) : "v"(a), "v"(b), "n"(N));
  }
  template <int N, int M>
  static __device__ inline void mma_v_lvw(f32x16& d, vec a, vec b, vec& q1, vec& q2, vec& q3, vec& q4, vec& q5) {
    asm volatile("s_waitcnt vmcnt(%9) lgkmcnt(%8)\n\tv_mfma_f32_32x32x16_bf16 %0, %6, %7, %0"
                 : "+v"(d), "+v"(q1), "+v"(q2), "+v"(q3), "+v"(q4), "+v"(q5) : "v"(a), "v"(b), "n"(N), "n"(M));
  }
  template <int N, int M>
  static __device__ inline void mma_v0_lvw(f32x16& d, vec a, vec b, vec& q1, vec& q2, vec& q3, vec& q4, vec& q5) {
    asm volatile("s_waitcnt vmcnt(%9) lgkmcnt(%8)\n\tv_mfma_f32_32x32x16_bf16 %0, %6, %7, 0"
                 : "=&v"(d), "+v"(q1), "+v"(q2), "+v"(q3), "+v"(q4), "+v"(q5) : "v"(a), "v"(b), "n"(N), "n"(M));
  }
  static __device__ inline void mma_a(f32x16& d, vec a, vec b) {
    asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(d) : "v"(a), "v"(b));
  }
  static __device__ inline void mma_a0(f32x16& d, vec a, vec b) {
    asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, 0" : "=a"(d) : "v"(a), "v"(b));
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
  // mma_v with the A operand's LDS wait (lgkmcnt(N)) in the same asm
  // statement: as separate statements the compiler pads a wait state between
  // them. mma_v_lvw / mma_v0_lvw: also the wait for the Q loads of operands b
  // and q1 .. q5 (vmcnt(M)), which the statement marks as produced.
  template <int N>
  static __device__ inline void mma_v_lw(f32x16& d, vec a, vec b) {
    asm volatile("s_waitcnt lgkmcnt(%3)\n\tv_mfma_f32_32x32x16_f16 %0, %1, %2, %0" : "+v"(d) : "v"(a), "v"(b), "n"(N));
  }
  template <int N, int M>
  static __device__ inline void mma_v_lvw(f32x16& d, vec a, vec b, vec& q1, vec& q2, vec& q3, vec& q4, vec& q5) {
    asm volatile("s_waitcnt vmcnt(%9) lgkmcnt(%8)\n\tv_mfma_f32_32x32x16_f16 %0, %6, %7, %0"
                 : "+v"(d), "+v"(q1), "+v"(q2), "+v"(q3), "+v"(q4), "+v"(q5) : "v"(a), "v"(b), "n"(N), "n"(M));
  }
  template <int N, int M>
  static __device__ inline void mma_v0_lvw(f32x16& d, vec a, vec b, vec& q1, vec& q2, vec& q3, vec& q4, vec& q5) {
    asm volatile("s_waitcnt vmcnt(%9) lgkmcnt(%8)\n\tv_mfma_f32_32x32x16_f16 %0, %6, %7, 0"
                 : "=&v"(d), "+v"(q1), "+v"(q2), "+v"(q3), "+v"(q4), "+v"(q5) : "v"(a), "v"(b), "n"(N), "n"(M));
  }
  static __device__ inline void mma_a(f32x16& d, vec a, vec b) {
    asm volatile("v_mfma_f32_32x32x16_f16 %0, %1, %2, %0" : "+a"(d) : "v"(a), "v"(b));
  }
  static __device__ inline void mma_a0(f32x16& d, vec a, vec b) {
    asm volatile("v_mfma_f32_32x32x16_f16 %0, %1, %2, 0" : "=a"(d) : "v"(a), "v"(b));
  }
};

// 32 wait states after the last inline-asm MFMA writing d0/d1 and before any
// other instruction reads them (covers the MFMA-result -> VALU read hazard
// for up to 16-pass MFMAs). Taking d0/d1 as in-out operands orders every
// later use after it.
__device__ inline void settle(f32x16& d0, f32x16& d1) {
  asm volatile("s_nop 15\n\ts_nop 15" : "+v"(d0), "+v"(d1));
}

// The QK accumulator before softmax(t+1) reads it (PV slot kSmSettle = 1):
// 16 wait states, and the code between the last QK MFMA and that slot issues
// at least 7 more instructions (step 35's two value reads, PV step 0's wait,
// its two MFMAs and step 4's two value reads), 23 in all.
__device__ inline void settle1(f32x16& d0) { asm volatile("s_nop 15" : "+v"(d0)); }

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

// Chunk swizzle of 128-B rows (k_rope): logical chunk j is stored at chunk
// j ^ fr(row).
__device__ inline int fr(int row) { return (row >> 1) & 7; }

// vmcnt(n) with the other counters left alone (gfx9 encoding, n < 16).
template <int N>
__device__ inline void wait_vm() {
  static_assert(N >= 0 && N < 16, "vmcnt range");
  __builtin_amdgcn_s_waitcnt(0x0F70 | N);
}

// vmcnt(N) for N < 64 (gfx9 encoding: low 4 bits at [3:0], high 2 at
// [15:14]), the other counters left alone.
template <int N>
__device__ inline void wait_vm_ext() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0F70);
}

// QK step kk (a multiple of 6) of the first QK phase of a segment needs Q
// k-steps kk .. kk+5, loaded by the prologue's 36 untracked loads after tile
// 0's copies. Issued after Q k-step kk+5 by then: the 30 - kk later Q loads,
// the tile copies of QK steps before kk (copy m at step copy_step(m), m <
// copies) and, paged, the table entry load before the phase. In every later
// QK phase only those copies and that entry are outstanding, so the same
// wait never binds there. The wait goes into the MFMA's asm statement
// (mma_v_lvw), which also marks q[KK+1 .. KK+5] as produced there.
template <int KK, int Copies, bool Paged>
constexpr int qb_vm_n() {
  static_assert(KK % 6 == 0 && KK + 5 < 36, "six k-steps per wait");
  int c = 0;
  for (int m = 0; m < Copies; ++m)
    if (copy_step(m) < KK) ++c;
  return (30 - KK) + c + (Paged ? 1 : 0);
}

// LDS-visibility barrier that leaves outstanding HBM->LDS copies in flight.
// The "memory" clobber keeps the compiler from moving LDS accesses across it.
__device__ inline void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// The lane index, computed by a volatile asm (v_mbcnt) at each use: nothing
// derived from it can be hoisted out of the enclosing loop, so per-lane
// addresses are recomputed per tile (a few VALU ops) instead of being kept
// live across the loop (or spilled) in VGPRs.
__device__ inline int lane_id() {
  int l;
  asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
  return l;
}

// Cross-lane combines without a lane index (no ds_bpermute: no LDS counter
// traffic and no lane-id register to keep live). permlane32_swap(x, x)
// returns (x[l % 32], x[l % 32 + 32]) in every lane l, permlane16_swap(x, x)
// the same for 16-lane halves of each 32-lane half; DPP 0xB1 / 0x4E / 0x141
// / 0x140 read lane l^1 / l^2 / the mirror inside 8 / inside 16 lanes.
__device__ inline float f_of(unsigned u) { return __builtin_bit_cast(float, u); }
__device__ inline unsigned u_of(float f) { return __builtin_bit_cast(unsigned, f); }
// x[l] + x[l ^ 32]
__device__ inline float sum_halves(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(u_of(x), u_of(x), false, false);
  return f_of(r[0]) + f_of(r[1]);
}
// max of x over lanes l^32
__device__ inline float max_halves(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(u_of(x), u_of(x), false, false);
  return fmaxf(f_of(r[0]), f_of(r[1]));
}
template <int CTRL>
__device__ inline float dpp_f(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), CTRL, 0xF, 0xF, false));
}
// max of x over the 32 lanes of this lane's half of the wave
__device__ inline float max32(float x) {
  x = fmaxf(x, dpp_f<0xB1>(x));
  x = fmaxf(x, dpp_f<0x4E>(x));
  x = fmaxf(x, dpp_f<0x141>(x));
  x = fmaxf(x, dpp_f<0x140>(x));
  const auto r = __builtin_amdgcn_permlane16_swap(u_of(x), u_of(x), false, false);
  return fmaxf(f_of(r[0]), f_of(r[1]));
}

// LDS is addressed with 32-bit byte offsets from the start of the dynamic LDS
// block (address-space-3 pointers), never with 64-bit generic pointers. The
// decode kernel declares no static LDS, so its dynamic block starts at LDS
// address 0 and the inline-asm accessors below use the offset itself as the
// address (the launcher checks the kernel's static LDS size is 0).
typedef __attribute__((address_space(3))) char lchar;

template <typename T>
__device__ inline T lds_ld(const lchar* L, uint32_t off) {
  return *reinterpret_cast<const __attribute__((address_space(3))) T*>(L + off);
}
template <typename T>
__device__ inline void lds_st(lchar* L, uint32_t off, T v) {
  *reinterpret_cast<__attribute__((address_space(3))) T*>(L + off) = v;
}
// Partial-slot stores go out at device scope: the cache-policy operand's sc1
// bit on a buffer store writes through this XCD's L2 to the device's
// coherence point, so the release at the end of the grid finds no dirty
// partial lines left in the L2s to write back (attention -2 us at config 3),
// and the merge kernel, on any XCD, still reads them from the infinity cache
// (its time is unchanged). kBufferRsrcWord3 is word 3 of a raw buffer
// resource (32-bit data format, as the gfx9 family expects).
constexpr int kCpolSc1 = 16;
constexpr int kBufferRsrcWord3 = 0x00020000;
// ds_read_b64_tr_b16 as inline asm: the builtin makes the compiler assume the
// read may alias the in-flight HBM->LDS copies and drain vmcnt before it. OFF
// is the instruction's immediate byte offset. The result must not be used
// before an lgkmcnt wait that covers it.
template <int OFF>
__device__ inline i16x4 lds_tr(const lchar* L, uint32_t off) {
  static_assert(OFF >= 0 && OFF < 65536, "ds offset field");
  i16x4 r;
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(r) : "v"(off), "n"(OFF));
  return r;
}

// ds_read_b128 as inline asm, for the same reason; same contract as lds_tr.
template <typename V, int OFF = 0>
__device__ inline V lds_rd128(const lchar* L, uint32_t off) {
  static_assert(OFF >= 0 && OFF < 65536, "ds offset field");
  V r;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(off), "n"(OFF));
  return r;
}

__device__ inline i16x4 lds_rd64(const lchar* L, uint32_t off) {
  i16x4 r;
  asm volatile("ds_read_b64 %0, %1" : "=v"(r) : "v"(off));
  return r;
}

// lgkmcnt(N) as inline asm whose operands are the registers it protects, so
// no copy of them is scheduled before the wait.
template <int N>
__device__ inline void wait_lgkm(i16x4& a, i16x4& b) {
  static_assert(N >= 0 && N < 16, "lgkmcnt range");
  asm volatile("s_waitcnt lgkmcnt(%2)" : "+v"(a), "+v"(b) : "n"(N));
}
template <int N, typename V>
__device__ inline void wait_lgkm(V& a) {
  static_assert(N >= 0 && N < 16, "lgkmcnt range");
  asm volatile("s_waitcnt lgkmcnt(%1)" : "+v"(a) : "n"(N));
}

template <int N, typename V>
__device__ inline void wait_lgkm(i16x4& a, i16x4& b, V& c, V& d) {
  static_assert(N >= 0 && N < 16, "lgkmcnt range");
  asm volatile("s_waitcnt lgkmcnt(%4)" : "+v"(a), "+v"(b), "+v"(c), "+v"(d) : "n"(N));
}
// max(|a|, |b|, c)
__device__ inline float max3abs(float a, float b, float c) {
  float r;
  asm("v_max3_f32 %0, |%1|, |%2|, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}
__device__ inline float max3f(float a, float b, float c) {
  float r;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}
// The partner's rescale flag and the first six score operands of a QK phase,
// in one asm statement that waits for the flag (issued first) before it
// ends. A value read by one asm and waited for by a later one can be copied by
// the compiler in between, before it has landed; the flag lives across the
// whole phase, so it is complete where it is defined. The operands are waited
// for by the phase's counted waits (the flag is not among their later reads).
template <typename V>
__device__ inline void qk_open(float& flag, V (&a)[6], uint32_t flag_at, uint32_t ct) {
  asm volatile(
      "ds_read_b32 %0, %7\n\t"
      "ds_read_b128 %1, %8\n\t"
      "ds_read_b128 %2, %8 offset:32\n\t"
      "ds_read_b128 %3, %8 offset:64\n\t"
      "ds_read_b128 %4, %8 offset:96\n\t"
      "ds_read_b128 %5, %8 offset:128\n\t"
      "ds_read_b128 %6, %8 offset:160\n\t"
      "s_waitcnt lgkmcnt(6)"
      : "=&v"(flag), "=&v"(a[0]), "=&v"(a[1]), "=&v"(a[2]), "=&v"(a[3]), "=&v"(a[4]), "=&v"(a[5])
      : "v"(flag_at), "v"(ct));
}
// The same flag alone, read and waited for in one asm statement.
__device__ inline float lds_rd32_now(uint32_t off) {
  float r;
  asm volatile("ds_read_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(r) : "v"(off));
  return r;
}

// Marks v as produced here (no code): for a value read by inline asm whose
// completion an earlier, later-issued wait already guarantees.
template <typename V>
__device__ inline void tie(V& v) {
  asm volatile("" : "+v"(v));
}
__device__ inline float lds_rd32(const lchar* L, uint32_t off) {
  float r;
  asm volatile("ds_read_b32 %0, %1" : "=v"(r) : "v"(off));
  return r;
}

// Calls f(std::integral_constant<int, i>) for i = 0 .. N-1.
template <int I, int N, typename F>
__device__ inline void static_for_impl(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>());
    static_for_impl<I + 1, N>(f);
  }
}
template <int N, typename F>
__device__ inline void static_for(F&& f) {
  static_for_impl<0, N>(f);
}

struct TrPair {
  i16x4 x0, x1;
};

constexpr int kRowBytes = (kDc + kDr) * 2;  // 1152: one packed cache row
// Bytes of one cache row in HBM: a 16-bit row, or an FP8 E4M3 row (576).
template <bool kFp8>
constexpr int cache_row_bytes() { return kFp8 ? kDc + kDr : kRowBytes; }
// FP8 E4M3 cache: wave w's 8 rows of a tile (576 B each, contiguous in HBM)
// are copied packed to fp8_stage_off(w) .. + 4608 of the tile's buffer, in
// kFp8RowCopies copies of 1 KB (lanes 0..31 of the last one). That range lies
// inside the bytes of the wave's own bf16 rows 8w..8w+7 and below the k_rope
// rows, so once the wave has read its staged rows (RoPE reads the k_rope
// parts, expand_rows the c_t parts) it expands them in place to the bf16 tile
// layout without touching another wave's staging. Every E4M3 value is a bf16
// value, so the expanded tile is exactly what a bf16 cache holding the same
// values gives.
__host__ __device__ constexpr int fp8_stage_off(int w) { return 8704 * w + 4096; }
constexpr int kFp8RowCopies = 5;  // 8 x 576 B = 4.5 KB
constexpr int dma_per_wave(bool fp8) { return fp8 ? kFp8RowCopies + 2 : kDmaPerWave; }
static_assert(fp8_stage_off(0) >= 0 && fp8_stage_off(3) + 8 * (kDc + kDr) <= kRopeOff, "staging below k_rope");
// Wave w's expanded rows 8w..8w+7 stay clear of the other waves' staging.
constexpr bool fp8_staging_disjoint() {
  for (int w = 0; w < kWaves; ++w) {
    if (w > 0 && ct_row_off(8 * w) < fp8_stage_off(w - 1) + 8 * (kDc + kDr)) return false;
    if (w + 1 < kWaves && ct_row_off(8 * w + 7) + 2 * kDc > fp8_stage_off(w + 1)) return false;
  }
  return true;
}
static_assert(fp8_staging_disjoint(), "fp8 staging of one wave overlaps another wave's rows");
// Cache policy of the cache-row copies: non-temporal (the nt bit of the gfx9.4+
// cache-policy field). Every row is read exactly once per call; streaming the
// ~300 MB past the caches keeps the weights, queries and partial slots of the
// surrounding kernels resident in L2 / the infinity cache.
constexpr int kStreamPolicy = 2;

struct SegCtx {
  const char* base;  // contiguous cache: first byte of the segment's first row
  int64_t pos0;      // in-sequence position of the segment's first row
  int last;          // index of the segment's last row, relative to its first
  int seq;           // sequence
  const int32_t* tab;  // paged cache: the sequence's block-table row
  uint32_t tile0;      // paged cache: in-sequence tile index of the segment's first tile
  // RoPE table row of position pos0 + r, r >= 0: min(pc + r, rlim), where
  // rlim = rope_rows - 1 (INT32_MAX when unchecked) and pc = min(pos0, rlim):
  // the clamp of rope_row in 32 bits (the MFMA kernels' positions and table
  // rows stay below 2^24 + 2^20, mfma_supported)
  int pc, rlim;
};

// Tile k covers segment rows [32k, 32k + 32). The pipeline also copies up to
// two tiles past the segment's last one; those copies re-read rows of the
// last tile, so every copy of tile k reads rows of tile tile_eff(k) only.
__device__ inline int tile_eff(const SegCtx& sg, int k) { return min(k, sg.last / kT); }

// Paged cache: tile k is in-sequence tile q = tile0 + tile_eff(k), in block
// q / tile_per_block at tile q % tile_per_block. A tile never straddles two
// blocks: block_size and the segment's first position are multiples of 32
// (the launcher rounds chunk_len and requires block_size % 32 == 0). q <
// 2^26, so the launcher's multiplier divides exactly, in 32 bits.
__device__ inline uint32_t tile_seq_index(const SegCtx& sg, int k) { return sg.tile0 + (uint32_t)tile_eff(sg, k); }
__device__ inline uint32_t tile_block_index(const DecodeProblem& p, uint32_t q) {
  return (__umulhi(q, p.tpb_magic) + q) >> p.tpb_shift;
}
__device__ inline int tile_block_entry(const DecodeProblem& p, const SegCtx& sg, int k) {
  return sg.tab[tile_block_index(p, tile_seq_index(sg, k))];
}
// Starts loading tile k's entry into v (inline asm: the compiler neither
// waits for it nor copies v while it is in flight). The caller's next
// vmcnt(0) completes it; tie(v) after that wait marks v as produced there.
__device__ inline void tile_block_entry_async(const DecodeProblem& p, const SegCtx& sg, int k, int& v) {
  const int32_t* a = sg.tab + tile_block_index(p, tile_seq_index(sg, k));
  asm volatile("global_load_dword %0, %1, off" : "=v"(v) : "v"(a));
}
// First byte of tile k's first row: contiguous cache (entry unused) or the
// pool block given by its table entry (clamped into the pool; pool rows fit
// in 32 bits, which the launcher checks).
template <bool kPaged, bool kFp8>
__device__ inline const char* tile_base(const DecodeProblem& p, const SegCtx& sg, int k, int entry) {
  constexpr int kRowB = cache_row_bytes<kFp8>();
  if constexpr (kPaged) {
    const uint32_t q = tile_seq_index(sg, k);
    const uint32_t in_block = q - tile_block_index(p, q) * p.tile_per_block;
    const int b = min(max(__builtin_amdgcn_readfirstlane(entry), 0), p.pool_last);
    const uint32_t row = (uint32_t)b * (uint32_t)p.block_size + in_block * kT;
    return reinterpret_cast<const char*>(p.kv) + (uint64_t)row * kRowB;
  } else {
    return sg.base + (int64_t)(tile_eff(sg, k) * kT) * kRowB;
  }
}

// Wave w's copies of tile k, rows tb = 32k + 8w ..: the tile's base address,
// the per-lane byte offset of row tb's chunk lane from it, how far the
// segment's last row is past tb (rows past it re-read the last row: their
// scores are masked), and the k_rope copy's offset (row min(tb + lane/8,
// last), the logical chunk (lane%8) ^ fr(row) that lands in chunk lane%8).
// Offsets are relative to the tile base (rows of tile_eff(k) only; for the
// copies past the segment tb - 32 tile_eff(k) is large, but every row they
// read is clamped to the last one, and the 32-bit sum wraps back to it).
struct TileDma {
  const char* base;
  uint32_t ct, rope;
  int dlast;  // last - tb, wave-uniform
};
// The k_rope copy's offset alone (rope of tile_dma): row delta below 64, so
// a 24-bit multiply.
template <bool kFp8>
__device__ inline uint32_t tile_dma_rope(const SegCtx& sg, int k, int wave, int lane) {
  if constexpr (kFp8) return 0u;
  const int tb = k * kT + 8 * wave, t0 = tile_eff(sg, k) * kT, rr = lane >> 3;
  return __umul24((uint32_t)(min(tb + rr, sg.last) - t0), (uint32_t)cache_row_bytes<kFp8>()) + kDc * 2 +
         16 * ((lane & 7) ^ fr(8 * wave + rr));
}
template <bool kFp8, bool kRope = true>
__device__ inline TileDma tile_dma(const SegCtx& sg, int k, const char* base, int wave, int lane) {
  constexpr int kRowB = cache_row_bytes<kFp8>();
  const int tb = k * kT + 8 * wave;
  const int t0 = tile_eff(sg, k) * kT;
  const int rr = lane >> 3;
  TileDma d;
  d.base = base;
  d.ct = (uint32_t)(tb - t0) * kRowB + 16 * lane;
  d.dlast = sg.last - tb;
  (void)rr;
  d.rope = kRope ? tile_dma_rope<kFp8>(sg, k, wave, lane) : 0u;
  return d;
}

// Wave w's HBM->LDS copy J (0..10) of tile k into the buffer at LDS offset
// buf: J < 8 is the c_t row 8w+J, J = 8 the k_rope rows 8w..8w+7, J = 9 / 10
// their cos / sin rows. Lane i writes LDS chunk i (M0 + 16i): c_t rows land
// unswizzled at ct_row_off, so the lane offset is the same for every row. The
// instruction's immediate offset would move the LDS destination too, so row
// steps go into the VGPR offset.
template <int J>
__device__ inline void issue_copy(const DecodeProblem& p, const SegCtx& sg, int k, lchar* L, uint32_t buf, int wave,
                                  int lane, const TileDma& d) {
  const int r_first = 8 * wave;
  if constexpr (J < 8) {
    const int j = min(J, d.dlast);
    __builtin_amdgcn_global_load_lds(d.base + (d.ct + (uint32_t)(j * kRowBytes)),
                                     (lds_void*)(L + buf + ct_row_off(r_first + J)), 16, 0, kStreamPolicy);
  } else if constexpr (J == 8) {
    __builtin_amdgcn_global_load_lds(d.base + d.rope, (lds_void*)(L + buf + kRopeOff + r_first * 128), 16, 0,
                                     kStreamPolicy);
  } else {
    const int row = r_first + (lane >> 3);
    const int r = min(k * kT + row, sg.last);
    const uint32_t toff = (uint32_t)min(sg.pc + r, sg.rlim) * ((kDr / 2) * 4) + (lane & 7) * 16;
    const float* tab = J == 9 ? p.rope_cos : p.rope_sin;
    __builtin_amdgcn_global_load_lds(reinterpret_cast<const char*>(tab) + toff,
                                     (lds_void*)(L + (J == 9 ? kCosOff : kSinOff) + r_first * 128), 16, 0, 0);
  }
}

// FP8 cache: wave w's copy J of tile k. J < kFp8RowCopies: 1 KB of the
// wave's 8 packed rows (chunk q = 64J + lane of 288 16-B chunks, i.e. row
// q / 36, bytes 16 (q % 36) of it) to its staging bytes; past the segment's
// last row each lane re-reads that chunk of the last row instead (rows past it
// are masked, and unfilled capacity is never read). J = kFp8RowCopies /
// + 1: the cos / sin rows, as for a 16-bit cache.
template <int J>
__device__ inline void issue_copy_fp8(const DecodeProblem& p, const SegCtx& sg, int k, lchar* L, uint32_t buf,
                                      int wave, int lane, const TileDma& d) {
  if constexpr (J < kFp8RowCopies) {
    uint32_t off;
    if (d.dlast >= 7) {  // wave-uniform: all 8 rows inside the segment
      off = d.ct + 1024 * J;
    } else {
      const int q = 64 * J + lane;
      const int r = (q * 1821) >> 16;  // q / 36, exact for q < 320
      off = d.ct - 16 * lane + (uint32_t)(min(r, d.dlast) * (kDc + kDr) + 16 * (q - 36 * r));
    }
    lds_void* dst = (lds_void*)(L + buf + fp8_stage_off(wave) + 1024 * J);
    if constexpr (J == kFp8RowCopies - 1) {
      if (lane < 32) __builtin_amdgcn_global_load_lds(d.base + off, dst, 16, 0, kStreamPolicy);
    } else {
      __builtin_amdgcn_global_load_lds(d.base + off, dst, 16, 0, kStreamPolicy);
    }
  } else {
    issue_copy<J - kFp8RowCopies + 9>(p, sg, k, L, buf, wave, lane, d);
  }
}

template <bool kFp8, int J>
__device__ inline void issue_copy_any(const DecodeProblem& p, const SegCtx& sg, int k, lchar* L, uint32_t buf,
                                      int wave, int lane, const TileDma& d) {
  if constexpr (kFp8) issue_copy_fp8<J>(p, sg, k, L, buf, wave, lane, d);
  else issue_copy<J>(p, sg, k, L, buf, wave, lane, d);
}

// All copies of tile k (base: tile_base of tile k).
template <bool kFp8>
__device__ inline void issue_tile_dma(const DecodeProblem& p, const SegCtx& sg, int k, const char* base, lchar* L,
                                      uint32_t buf, int wave, int lane) {
  const TileDma d = tile_dma<kFp8>(sg, k, base, wave, lane);
  static_for<dma_per_wave(kFp8)>([&](auto j) { issue_copy_any<kFp8, decltype(j)::value>(p, sg, k, L, buf, wave, lane, d); });
}

// Rotate-half RoPE of rows 8w..8w+7 of the tile at LDS offset buf, in place
// (src/fused_mla.cu:43-51): r[i] = k[i]*c - k[i+32]*s, r[i+32] = k[i]*s +
// k[i+32]*c. Lane: row 8w + lane/8, pairs i = 4(lane%8) .. +3. Split in two:
// rot_issue starts the four LDS reads (inline asm; the caller waits for them
// with lgkmcnt), rot_finish rotates and stores.
struct RotIn {
  i16x4 ka, kb;      // 16-bit cache: k[i .. i+3], k[i+32 .. i+35]
  uint32_t k8a, k8b;  // FP8 cache: the same elements as 4 + 4 codes
  f32x4 c, s;
  uint32_t pa, pb;
};

// FP8 cache: ka / kb are the 4 + 4 fp8 codes of the staged row (in their low
// 32 bits); the rotated values go to the bf16 k_rope rows as for a 16-bit
// cache.
template <bool kFp8 = false>
__device__ inline RotIn rot_issue(const lchar* L, uint32_t buf, int wave, int lane) {
  const int rl = lane >> 3, u = lane & 7;
  const int row = 8 * wave + rl;
  const int f = fr(row);
  RotIn r;
  r.pa = buf + kRopeOff + row * 128 + (((u >> 1) ^ f) << 4) + 8 * (u & 1);
  r.pb = buf + kRopeOff + row * 128 + (((4 + (u >> 1)) ^ f) << 4) + 8 * (u & 1);
  if constexpr (kFp8) {
    const uint32_t src = buf + fp8_stage_off(wave) + rl * (kDc + kDr) + kDc + 4 * u;
    r.k8a = __builtin_bit_cast(uint32_t, lds_rd32(L, src));
    r.k8b = __builtin_bit_cast(uint32_t, lds_rd32(L, src + kDr / 2));
  } else {
    r.ka = lds_rd64(L, r.pa);
    r.kb = lds_rd64(L, r.pb);
  }
  r.c = lds_rd128<f32x4>(L, kCosOff + row * 128 + 16 * u);
  r.s = lds_rd128<f32x4>(L, kSinOff + row * 128 + 16 * u);
  return r;
}

// rot_issue for a 16-bit cache from precomputed addresses: pa = buf +
// kRopeOff + the lane part (row 8w + lane/8, chunk (lane%8)/2 ^ fr(row),
// half lane%2); the chunk of elements i + 32 is that of i XOR 4, so pb = pa ^
// 64 (rows are 128-aligned); cs = kCosOff + 1024w + 16 lane, the sin row at
// the same offset from kSinOff.
__device__ inline RotIn rot_issue_at(const lchar* L, uint32_t pa, uint32_t cs) {
  RotIn r;
  r.pa = pa;
  r.pb = pa ^ 64;
  r.ka = lds_rd64(L, r.pa);
  r.kb = lds_rd64(L, r.pb);
  r.c = lds_rd128<f32x4>(L, cs);
  r.s = lds_rd128<f32x4, kSinOff - kCosOff>(L, cs);
  return r;
}

// Element e (0..3) of ka / kb as f32.
template <typename KT, bool kFp8>
__device__ inline float rot_k(const RotIn& in, bool second, int e) {
  typedef typename Ops<KT>::elem E;
  if constexpr (kFp8) {
    const uint32_t w = second ? in.k8b : in.k8a;
    const auto v = (e & 2) ? __builtin_amdgcn_cvt_pk_f32_fp8(w, true) : __builtin_amdgcn_cvt_pk_f32_fp8(w, false);
    return v[e & 1];
  } else {
    return (float)__builtin_bit_cast(E, (short)(second ? in.kb[e] : in.ka[e]));
  }
}

template <typename KT, bool kFp8, int N = 0>
__device__ inline void rot_wait(RotIn& in) {
  if constexpr (kFp8) asm volatile("s_waitcnt lgkmcnt(%4)" : "+v"(in.k8a), "+v"(in.k8b), "+v"(in.c), "+v"(in.s) : "n"(N));
  else asm volatile("s_waitcnt lgkmcnt(%4)" : "+v"(in.ka), "+v"(in.kb), "+v"(in.c), "+v"(in.s) : "n"(N));
}

template <typename KT, bool kFp8>
__device__ inline void rot_finish(lchar* L, RotIn& in) {
  typedef typename Ops<KT>::elem E;
  rot_wait<KT, kFp8>(in);
  i16x4 ra, rb;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float k0 = rot_k<KT, kFp8>(in, false, e);
    const float k1 = rot_k<KT, kFp8>(in, true, e);
    ra[e] = __builtin_bit_cast(short, (E)(k0 * in.c[e] - k1 * in.s[e]));
    rb[e] = __builtin_bit_cast(short, (E)(k0 * in.s[e] + k1 * in.c[e]));
  }
  lds_st(L, in.pa, ra);
  lds_st(L, in.pb, rb);
}

template <typename KT>
__device__ inline void rot_store(lchar* L, const RotIn& in, const float (&ra)[4], const float (&rb)[4]) {
  typedef typename Ops<KT>::elem E;
  i16x4 a, b;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    a[e] = __builtin_bit_cast(short, (E)ra[e]);
    b[e] = __builtin_bit_cast(short, (E)rb[e]);
  }
  lds_st(L, in.pa, a);
  lds_st(L, in.pb, b);
}

template <typename KT, bool kFp8>
__device__ inline void rotate_rows(lchar* L, uint32_t buf, int wave, int lane) {
  RotIn r = rot_issue<kFp8>(L, buf, wave, lane);
  rot_finish<KT, kFp8>(L, r);
}

// FP8 cache: expands this wave's 8 staged rows of the tile at buf to the
// bf16 c_t rows 8w..8w+7 (lane: latent columns 8 lane .. 8 lane + 7). All
// eight reads complete before the first write, and the rows' k_rope parts
// must have been read already (RoPE). Row j of the wave starts at
// ct_row_off(8w) + 1088 j + 16 (j >= 4): (8w + j) / 4 % 4 steps by one at
// j = 4 for every w.
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
// ds_read_b64 with immediate offset OFF (inline asm; the caller waits).
template <int OFF>
__device__ inline u32x2 lds_rd64_at(uint32_t off) {
  static_assert(OFF >= 0 && OFF < 65536, "ds offset field");
  u32x2 r;
  asm volatile("ds_read_b64 %0, %1 offset:%2" : "=v"(r) : "v"(off), "n"(OFF));
  return r;
}
__device__ inline void expand_rows(lchar* L, uint32_t buf, int wave, int lane) {
  const uint32_t src = buf + fp8_stage_off(wave) + 8 * lane;
  const uint32_t dst = buf + ct_row_off(8 * wave) + 16 * lane;
  u32x2 x[8];
  static_for<8>([&](auto j_c) {
    constexpr int j = decltype(j_c)::value;
    x[j] = lds_rd64_at<j * (kDc + kDr)>(src);
  });
  asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(x[0]), "+v"(x[1]), "+v"(x[2]), "+v"(x[3]), "+v"(x[4]), "+v"(x[5]),
               "+v"(x[6]), "+v"(x[7]));
  static_for<8>([&](auto j_c) {
    constexpr int j = decltype(j_c)::value;
    u32x4 y;
    y[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(x[j][0], 1.f, false));
    y[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(x[j][0], 1.f, true));
    y[2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(x[j][1], 1.f, false));
    y[3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(x[j][1], 1.f, true));
    lds_st(L, dst + 1088 * j + (j >= 4 ? 16 : 0), y);
  });
}

// FP8 cache, the expansion spread over PV: the reads of staged rows
// 4H .. 4H+3 of this wave (lane's 8 codes each) ...
template <int H>
__device__ inline void fp8_exp_issue(uint32_t src, u32x2 (&x)[4]) {
  static_for<4>([&](auto i_c) {
    constexpr int i = decltype(i_c)::value;
    x[i] = lds_rd64_at<(4 * H + i) * (kDc + kDr)>(src);
  });
}
// ... and row J's conversion and 16-B store (x read and waited for).
template <int J>
__device__ inline void fp8_exp_row(lchar* L, uint32_t dst, u32x2 x) {
  u32x4 y;
  y[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(x[0], 1.f, false));
  y[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(x[0], 1.f, true));
  y[2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(x[1], 1.f, false));
  y[3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(x[1], 1.f, true));
  lds_st(L, dst + 1088 * J + (J >= 4 ? 16 : 0), y);
}
// Rows 0..3's stores never reach staged rows 4..7 (every wave; rows 4..7's
// stores reach staged rows 0..7, so all their reads complete first).
constexpr bool fp8_half_order_ok() {
  for (int w = 0; w < kWaves; ++w)
    for (int j = 0; j < 4; ++j)
      for (int i = 4; i < 8; ++i) {
        const int a0 = ct_row_off(8 * w + j), s0 = fp8_stage_off(w) + i * (kDc + kDr);
        if (a0 < s0 + kDc + kDr && s0 < a0 + 2 * kDc) return false;
      }
  return true;
}
static_assert(fp8_half_order_ok(), "fp8 expansion halves overlap");

// Block id -> (chunk, head group), XCD-aware. Workgroups are dispatched
// round-robin over the 8 XCDs (id % 8), each with its own L2. The work items
// (chunk, group), chunk-major, are cut into 8 contiguous ranges, one per XCD
// (XCD x: items [x*per, (x+1)*per), id = 8 k + x is item x*per + k). With
// one head group per chunk the chunks of one sequence share an L2, so the
// sequence's Q rows are fetched from HBM once per XCD rather than once per
// chunk, and every XCD streams one contiguous piece of the cache; with many
// head groups (several queries over one cache) the groups of a chunk share an
// L2 and its rows, and every XCD has work even when there are fewer chunks
// than XCDs. Ids past the last item return at once (chunk >= num_chunks).
__host__ __device__ inline int64_t mfma_grid_blocks(int num_chunks, int groups) {
  return 8 * (((int64_t)num_chunks * groups + 7) / 8);
}
// 32-bit arithmetic: the grid (8 per blocks) is below 2^31, so every item
// is (a 64-bit division here is ~130 dependent scalar instructions at the
// kernel's start).
__device__ inline void block_coords(int num_chunks, int groups, int* chunk, int* group) {
  const uint32_t id = blockIdx.x;
  const uint32_t per = ((uint32_t)num_chunks * (uint32_t)groups + 7) / 8;
  const uint32_t item = (id & 7) * per + (id >> 3);
  if (groups == 1) {
    *group = 0;
    *chunk = (int)item;
  } else {
    const uint32_t c = item / (uint32_t)groups;
    *group = (int)(item - c * (uint32_t)groups);
    *chunk = (int)c;
  }
}

// find_seq for the MFMA kernels: with uniform sequences the row space is
// below 2^31 rows (mfma_supported), so the division is a 32-bit one.
__device__ inline int find_seq_mfma(const DecodeProblem& p, int64_t r) {
  if (p.offsets) return find_seq(p, r);
  return (int)((uint32_t)r / (uint32_t)p.seq_len);
}

// kFp8: FP8 E4M3 cache rows (KT = bf16: the tiles are expanded to bf16 in
// LDS and the MFMAs run on bf16).
template <typename KT, bool kPaged, bool kFp8>
__global__ __launch_bounds__(kThreads) void decode_mfma_kernel(DecodeProblem p, int groups) {
  static_assert(!kFp8 || std::is_same<KT, __hip_bfloat16>::value, "fp8 tiles expand to bf16");
  constexpr int kDma = dma_per_wave(kFp8);
  typedef Ops<KT> O_;
  typedef typename O_::vec vec;
  typedef typename O_::elem E;

#ifdef LA_PHASE_STAMPS
  unsigned long long stamps_[kStampSlots] = {};
#endif
  LA_STAMP(0);
  warm_kernarg_lines(p);
  extern __shared__ __attribute__((aligned(1024))) char lds_raw[];
  lchar* L = (lchar*)lds_raw;
  const int tid = threadIdx.x, lane0 = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: keep in SGPRs
  int chunk, group;
  block_coords(p.num_chunks, groups, &chunk, &group);
  if (chunk >= p.num_chunks) return;
  const int hg_heads = min(kHG, p.Hq - group * kHG);

  const int64_t end_all = seq_begin(p, p.num_seqs);
  int64_t lo = (int64_t)chunk * p.chunk_len;
  const int64_t hi = min(lo + (int64_t)p.chunk_len, end_all);
  lo = max(lo, seq_begin(p, 0));
  if (lo >= hi) return;
  int s = find_seq_mfma(p, lo);

  while (lo < hi) {
    const int64_t s_lo = seq_begin(p, s);
    lo = max(lo, s_lo);  // past the unfilled rows of the previous region
    if (lo >= hi) break;
    const int64_t s_hi = seq_end(p, s);
    if (s_hi <= lo) {  // empty sequence, or lo in its unfilled rows
      if (++s >= p.num_seqs) break;
      continue;
    }
    const int64_t seg_hi = min(hi, s_hi);
    SegCtx sg;
    sg.base = reinterpret_cast<const char*>(p.kv) + (kPaged ? 0 : lo * cache_row_bytes<kFp8>());
    sg.pos0 = lo - s_lo;
    sg.last = (int)(seg_hi - lo - 1);
    sg.seq = s;
    sg.tab = kPaged ? p.block_table + (int64_t)s * p.blocks_per_seq : nullptr;
    sg.tile0 = (uint32_t)(sg.pos0 / kT);
    sg.rlim = p.rope_rows > 0 ? (int)(p.rope_rows - 1) : INT32_MAX;
    sg.pc = (int)min(sg.pos0, (int64_t)sg.rlim);
    const int seg_len = sg.last + 1;
    const int ntiles = (seg_len + kT - 1) / kT;

    LA_STAMP(1);
#ifdef LA_PHASE_STAMPS
    for (int i = 11; i < 16; ++i) stamps_[i] = 0;
#endif
    lds_barrier();  // all waves are done with the previous segment's buffers
    LA_STAMP(2);

    // paged cache: the table entries of tiles 0 and 1 (tile 1 is copied in
    // iteration -1); iteration t loads the entry of tile t+3 into blk_cur once
    // its own copies have their base, for the next iteration
    int blk_cur = 0;
    const char* base0 = tile_base<kPaged, kFp8>(p, sg, 0, 0);
    if constexpr (kPaged) {
      const int e0 = tile_block_entry(p, sg, 0);
      blk_cur = tile_block_entry(p, sg, 1);
      base0 = tile_base<kPaged, kFp8>(p, sg, 0, e0);
      // both entries have landed before the copies and the Q loads go out
      // (the compiler's wait for blk_cur would otherwise count the untracked
      // Q loads short and wait for most of them in the first QK phase)
      asm volatile("" : "+v"(blk_cur));
    }

    // tile 1 rides along iteration -1; a fresh lane index keeps the per-lane
    // addresses out of the registers (and spill slots) that live across the
    // prologue: a spill reload here would wait on vmcnt and so serialise the copies
    issue_tile_dma<kFp8>(p, sg, 0, base0, L, 0, wave, lane_id());

    // Q^T as the B operand: lane holds Q[head][16kk + 8*g2 .. +8], pre-scaled.
    // q_prep is stored in operand order (qprep_index): the wave's 32 rows form
    // one block and k-step kk is the coalesced 1 KB at element 512kk. All 36
    // k-steps (32 latent, 4 rope) stay in VGPRs for the segment. A wave
    // without valid heads reads the group's last block (in bounds); a lane of
    // an invalid head reads the block's last valid row (finite values; its
    // results are never stored, and it crosses the rescale threshold exactly
    // when that row's head does).
    // The 36 loads are inline asm, after tile 0's copies: the compiler does
    // not track them, and the first QK phase waits for them k-step group by
    // k-step group (qb_vm_n), so it overlaps the loads' tail.
    vec qb[36];
    {
      const int q_lane = lane_id();
      const int wblk = min(32 * wave, (hg_heads - 1) & ~31);
      const int r = min(q_lane & 31, hg_heads - 1 - wblk);
      const int64_t qrow0 = (int64_t)s * qprep_rows_per_seq(p.Hq) + group * kHG + wblk;
      const E* qbase = reinterpret_cast<const E*>(p.q_prep) + qprep_index(qrow0, 0);
      const vec* qsrc = reinterpret_cast<const vec*>(qbase) + (r + (q_lane & 32));
#pragma unroll
      for (int kk = 0; kk < 36; ++kk) asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(qb[kk]) : "v"(qsrc + 64 * kk));
    }
    LA_STAMP(3);

    float m_run = -INFINITY, l_run = 0.f;
    // O = 0, written by MFMAs of zero operands straight into the AGPRs (a
    // zero vector built by the compiler would be kept in a spill slot)
    f32x16 acc[16];
    {
      vec z = {}, z2 = {};
      operands_ready(z, z2);  // VALU-written operands: wait states before the (inline asm) MFMAs
#pragma unroll
      for (int nb = 0; nb < 16; ++nb) O_::mma_a0(acc[nb], z, z2);
    }

    wait_vm_ext<36>();  // tile 0's copies have landed (the 36 Q loads went out after them)
    LA_STAMP(4);
    rotate_rows<KT, kFp8>(L, 0, wave, lane_id());  // fresh lane index: no spilled addresses
    if constexpr (kFp8) expand_rows(L, 0, wave, lane_id());
    LA_STAMP(5);

    // Software pipeline over tiles; iteration t (from -1):
    //   [apply the rescale of own-head O rows decided by softmax(t)]
    //   QK(t+1) -> s_next, with the HBM->LDS copies of tile t+2 riding along;
    //   [apply the partner's rescale to its O rows held here]
    //   PV(t): O += P(t) . V(t), with softmax(t+1) (s_next -> P(t+1)) spread
    //   between its MFMAs; then RoPE of tile t+2 (own rows), P(t+1) and the
    //   rescale of softmax(t+1) published in LDS, and a barrier.
    // Work split: wave w owns heads 32w.. for QK and the softmax. For PV the
    // waves pair up (w, w^1): each holds O for the pair's 64 heads over one
    // half of the latent columns (256 * (w & 1) ..), so it reads half of the
    // value tile and takes the partner's P(t) from LDS. acc[cb] holds own
    // heads, acc[8 + cb] the partner's, column block cb of the half, transposed
    // (lane = head).
    // Buffers: tile k lives in buffer k % 3. In iteration t, V(t) and K(t+1)
    // are read and tile t+2 is written; t+2 = t-1 (mod 3) was last read in
    // iteration t-1, before the barrier that opens iteration t. P and rescale
    // tables alternate by parity, so a table is rewritten only after the
    // barrier that follows its last read.
    // Every LDS read that a static lgkmcnt count includes is always issued;
    // where its data is not needed it reads a valid buffer and is dropped.
    const int ch = wave & 1;   // column half of the PV split
    const int pw = wave ^ 1;   // partner wave (same heads for PV, other half)
    vec p_cur[2] = {};         // P(t); zero for t = -1
    float alpha_pend = 1.f;    // O rescale owed before PV(t) (per head = lane % 32)
    bool resc_pend = false;    // wave-uniform
    {
      // P(-1) = 0 for the partner read of iteration -1; no rescale pending
      const int lz = lane_id();
      const vec zero = {};
#pragma unroll
      for (int par = 0; par < 2; ++par) {
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) lds_st(L, kPtabOff + par * kPtabPar + wave * 2048 + ks * 1024 + 16 * lz, zero);
        if (lz < 40) lds_st(L, kAtabOff + par * kAtabPar + wave * kAtabWave + 4 * lz, 0.f);
      }
    }
    // lane parts of the loop's LDS addresses (the buffer offsets are
    // per-iteration scalars added to them)
    int lct, lrp, ltb0, ltb1, lrot, lr1152, lrope;
    {
      const int ln = lane_id();
      const int ar = ln & 31, gg = ln >> 5, q16 = ln >> 4, s16 = ln & 15;
      lct = ct_row_off(ar) + 16 * gg;
      lrp = ar * 128 + 16 * (gg ^ fr(ar));
      const int rrow = 8 * wave + (ln >> 3), ru = ln & 7;
      lrot = rrow * 128 + (((ru >> 1) ^ fr(rrow)) << 4) + 8 * (ru & 1);
      // the k_rope copy's lane parts (tile_dma_rope): row 8w + lane/8 times
      // the row bytes, and the swizzled chunk past the latent part
      lr1152 = rrow * cache_row_bytes<kFp8>();
      lrope = kDc * 2 + 16 * (ru ^ fr(rrow));
      const int tc = 32 * (q16 & 1) + 8 * (s16 & 3) + 512 * ch;
      ltb0 = tc + ct_row_off(4 * (q16 >> 1) + (s16 >> 2));
      ltb1 = tc + ct_row_off(8 + 4 * (q16 >> 1) + (s16 >> 2));
    }
    // buffers of tiles t, t+1, t+2 (iteration -1: tile 0 in both of the
    // first two), carried from iteration to iteration
    uint32_t cur_b = 0, nxt_b = 0, dbuf_b = kBufBytes;
    for (int t = -1; t < ntiles; ++t) {
#ifdef LA_PHASE_STAMPS
      if (t == 0) LA_STAMP(6);
#endif
#ifdef LA_PHASE_STAMPS
      unsigned long long tt0, tt1, tt2, tt3, tt4;
      LA_TSTAMP(tt0);
#endif
      // this wave's copies of tile t+1 were waited for at the end of
      // iteration t-1 (t = -1: tile 0 in the prologue; the Q loads are still
      // in flight and QK(0) waits for them group by group)
      lds_barrier();  // tile t+1 staged and rotated by every wave; iteration t-1 done
#ifdef LA_PHASE_STAMPS
      LA_TSTAMP(tt1);
#endif
      const int lane = lane_id();
      const int g2 = lane >> 5;
      const int q16 = lane >> 4, s16 = lane & 15;
      const int head = 32 * wave + (lane & 31);
      const bool sm = t + 1 < ntiles;  // softmax(t+1) runs in this iteration
      const uint32_t cur = cur_b, nxt = nxt_b, dbuf = dbuf_b;
      const int par = t & 1;  // tables of P(t) and of softmax(t)'s rescale
      const uint32_t atab = kAtabOff + par * kAtabPar;

      // ---- own-head O rows *= alpha where softmax(t) moved the running max ----
      // O is held transposed (lane = head), so the factor is this lane's own
      // alpha from softmax(t).
      if (resc_pend) {
        settle_acc(acc);
        // one 16-register block at a time, pinned back to AGPRs after each
#pragma unroll
        for (int nb = 0; nb < 8; ++nb) {
          acc[nb] *= alpha_pend;
          pin_agpr(acc[nb]);
          __builtin_amdgcn_sched_barrier(0);
        }
        acc_ready(acc);
        resc_pend = false;
      }
      // the partner's flag for the same rescale (applied to its rows before PV)
      // (read together with the first score operands of QK, qk_open)
      const uint32_t pflag_at = atab + pw * kAtabWave + 128;
      float pflag;

      // ---- QK(t+1): S^T[pos][head] over 36 k-steps (32 latent + 4 rope) ----
      // A operand of k-step kk: tile row arow = lane%32, logical chunk
      // 2kk + g2. For c_t (kk < 32) that is byte ct_row_off(arow) + 16 g2 +
      // 32kk: a lane base plus the immediate 32kk. For the 128-B k_rope rows
      // the byte offset is 16((2(kk-32) + g2) ^ fr(arow)) = 32(kk-32) ^
      // 16(g2 ^ fr(arow)): a lane constant XOR an immediate. A operands are
      // read kQkDepth k-steps ahead of their MFMA. The last iteration skips
      // the phase (no tile t+1).
      const int arow = lane & 31;
      const uint32_t ct_x = nxt + lct;
      uint32_t rp_x, pp_x;
      // paged: this iteration's copies use tile t+2's entry (loaded in the
      // previous iteration or the prologue); tile t+3's goes out now and is
      // waited for by the next iteration's vmcnt(0)
      const int ent2 = kPaged ? __builtin_amdgcn_readfirstlane(blk_cur) : 0;
      if constexpr (kPaged) tile_block_entry_async(p, sg, t + 3, blk_cur);
      TileDma dm;
      auto a_rd = [&](auto kk_c) -> vec {
        constexpr int kk = decltype(kk_c)::value;
        if constexpr (kk < 32) return lds_rd128<vec, 32 * kk>(L, ct_x);
        else return lds_rd128<vec>(L, rp_x ^ (32 * (kk - 32)));
      };

      // PV(t) value reads: lane (q16, s16), read x of step (ks, nb) supplies
      // the address of tile[rho][32nb + 16(q16&1) + 4(s16&3)], rho = 16ks + 8x
      // + 4(q16>>1) + (s16>>2) (P's k-slot j of lane half g2 is position
      // 16ks + 8(j>>2) + 4g2 + (j&3), the S^T accumulator layout).
      // ct_row_off(rho) = 16ks kRowPitch + ct_row_off(rho - 16ks), so read x
      // is lane base tb_x plus the immediate 16ks kRowPitch + 64nb; this
      // wave's column blocks are nb = 8ch + cb.
      uint32_t tb0, tb1;
      TrPair tr[kPvDepth];
      auto b_issue = [&](TrPair& r, auto step_c) {
        constexpr int step = decltype(step_c)::value;
        constexpr int ks = step >> 3, cb = step & 7;
        r.x0 = lds_tr<16 * kRowPitch * ks + 64 * cb>(L, tb0);
        r.x1 = lds_tr<16 * kRowPitch * ks + 64 * cb>(L, tb1);
      };

      // Addresses the QK phase needs only later are made inside it, in the
      // issue slack between its MFMAs (the empty asm statements keep each
      // computation at its step), not between the barrier and the first
      // MFMA: the copies' addresses of tile t+2 after step 0, the partner-P
      // address after step 20, the k_rope operand address after step 22, the
      // value-read bases after step 28.
      auto qk_setup = [&](auto kk_c) {
        constexpr int kk = decltype(kk_c)::value;
        if constexpr (kk == 0) {
          int t2 = t + 2;
          asm volatile("" : "+s"(t2));
          dm = tile_dma<kFp8, false>(sg, t2, tile_base<kPaged, kFp8>(p, sg, t2, ent2), wave, lane);
        } else if constexpr (kk == 1 && !kFp8) {
          // tile_dma_rope from the lane parts: (min(tb + lane/8, last) - t0)
          // row bytes = min(lo + lr1152, hi), tb = 32 t2 + 8w, t0 its tile's
          // first row (tile_eff)
          int t2 = t + 2;
          asm volatile("" : "+s"(t2));
          const int t0 = tile_eff(sg, t2) * kT;
          const int lo = (t2 * kT - t0) * kRowBytes, hi = (sg.last - t0) * kRowBytes;
          dm.rope = (uint32_t)(min(lo + lr1152, hi) + lrope);
        } else if constexpr (kk == 20) {
          uint32_t pb = kPtabOff + par * kPtabPar + pw * 2048;
          asm volatile("" : "+s"(pb));
          pp_x = pb + 16 * lane;
        } else if constexpr (kk == 22) {
          uint32_t nb = nxt;
          asm volatile("" : "+s"(nb));
          rp_x = nb + kRopeOff + lrp;  // nxt + kRopeOff is a multiple of 128
        } else if constexpr (kk == 28) {
          uint32_t cb = cur;
          asm volatile("" : "+s"(cb));
          tb0 = cb + ltb0;
          tb1 = cb + ltb1;
        }
      };
      static_assert(kQrAt > 20 && 32 - kQkDepth > 22 && kTrAt > 28 && kCopyFirst > 1, "setup before first use");

      f32x16 s_next;
      vec pp[2];  // partner's P(t), read at step kQrAt
      if (t + 1 < ntiles) {
      vec ar[kQkDepth];
      static_assert(kQkDepth == 6, "qk_open reads six operands");
      qk_open(pflag, ar, pflag_at, ct_x);
      static_for<36>([&](auto kk_c) {
        constexpr int kk = decltype(kk_c)::value;
        constexpr int D = kQkDepth;
        if constexpr (kk == kQrAt) {
          pp[0] = lds_rd128<vec>(L, pp_x);
          pp[1] = lds_rd128<vec>(L, pp_x + 1024);
        }
        vec& a = ar[kk % D];
        // the operand's wait (and every sixth step the wait for Q k-steps kk
        // .. kk+5, qb_vm_n) in the MFMA's asm statement
        if constexpr (kk % 6 == 0) {
          constexpr int M = qb_vm_n<kk, kDma, kPaged>();
          static_assert(M >= 0 && M < 64, "vmcnt range");
          if constexpr (kk == 0)
            O_::template mma_v0_lvw<qk_later(kk), M>(s_next, a, qb[kk], qb[kk + 1], qb[kk + 2], qb[kk + 3], qb[kk + 4], qb[kk + 5]);
          else
            O_::template mma_v_lvw<qk_later(kk), M>(s_next, a, qb[kk], qb[kk + 1], qb[kk + 2], qb[kk + 3], qb[kk + 4], qb[kk + 5]);
        } else {
          O_::template mma_v_lw<qk_later(kk)>(s_next, a, qb[kk]);
        }
        if constexpr (kk + D < 36) a = a_rd(std::integral_constant<int, kk + D>());
        constexpr int cm = (kk - kCopyFirst) / kCopyStride;  // the copy of this step, if any
        if constexpr (kk >= kCopyFirst && (kk - kCopyFirst) % kCopyStride == 0 && cm < kDma) {
          if constexpr (kFp8) issue_copy_fp8<cm>(p, sg, t + 2, L, dbuf, wave, lane, dm);
          else issue_copy<dma_order(cm)>(p, sg, t + 2, L, dbuf, wave, lane, dm);
        }
        if constexpr (kk >= kTrAt && kk - kTrAt < kPvDepth) b_issue(tr[kk - kTrAt], std::integral_constant<int, kk - kTrAt>());
        qk_setup(kk_c);
        __builtin_amdgcn_sched_barrier(0);
      });
      } else {
        // The last iteration has no tile t+1 to score: only the LDS reads
        // that PV(t) waits for go out, in QK's order (partner P, then the
        // first kPvDepth value-read pairs), so PV's static counts still hold.
        pflag = lds_rd32_now(pflag_at);
        pp_x = kPtabOff + par * kPtabPar + pw * 2048 + 16 * lane;
        tb0 = cur + ltb0;
        tb1 = cur + ltb1;
        pp[0] = lds_rd128<vec>(L, pp_x);
        pp[1] = lds_rd128<vec>(L, pp_x + 1024);
        static_for<kPvDepth>([&](auto i) { b_issue(tr[decltype(i)::value], i); });
        s_next = f32x16{};
      }

#ifdef LA_PHASE_STAMPS
      LA_TSTAMP(tt2);
#endif
      // ---- softmax(t+1) pieces, spread over the PV(t) steps ----
      // s_next lane = head, 16 positions 8(i/4) + 4*g2 + (i%4); lazy base-2
      // online softmax: P = 2^(s - m) with m raised only when a score exceeds
      // it by more than kRescaleSlack; O's matching rescale is applied at the
      // top of the next iteration, after PV(t) has added P(t) . V(t) at the
      // old scale.
      const int valid = min(kT, seg_len - (t + 1) * kT);
      float mx[5];
      float lmax = -INFINITY;
      uint32_t pw_next[8];  // P(t+1) as bf16/fp16 pairs: word j = positions 2j, 2j+1 of the lane's 16
      float lacc;  // l_run plus the P(t+1) values summed so far
      float sd[16], sx[16];  // s - m and 2^(s - m) of the lane's 16 scores
      auto sm_piece = [&](auto step_c) {
        constexpr int step = decltype(step_c)::value;
        if constexpr (step == kSmSettle) {
          settle1(s_next);
          if (sm && valid < kT) {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
              const int pos = 8 * (i >> 2) + 4 * g2 + (i & 3);
              s_next[i] = pos < valid ? s_next[i] : -INFINITY;
            }
          }
        } else if constexpr (step >= kSmSettle + 1 && step <= kSmSettle + 4) {
          // max over the lane's 16 scores: a tree of v_max3 (inline asm: the
          // compiler would canonicalise every operand of fmaxf first), two
          // independent ops per slot
          constexpr int q = step - kSmSettle - 1;
          if constexpr (q == 0) {
            mx[0] = max3f(s_next[0], s_next[1], s_next[2]);
            mx[1] = max3f(s_next[3], s_next[4], s_next[5]);
          } else if constexpr (q == 1) {
            mx[2] = max3f(s_next[6], s_next[7], s_next[8]);
            mx[3] = max3f(s_next[9], s_next[10], s_next[11]);
          } else if constexpr (q == 2) {
            mx[4] = max3f(s_next[12], s_next[13], s_next[14]);
            mx[0] = max3f(mx[0], mx[1], s_next[15]);
          } else {
            mx[1] = max3f(mx[2], mx[3], mx[4]);
          }
          asm volatile("" : "+v"(mx[0]), "+v"(mx[1]), "+v"(mx[2]), "+v"(mx[3]), "+v"(mx[4]));
        } else if constexpr (step == kSmSettle + 5) {
          lmax = max3f(mx[0], mx[1], mx[1]);
          const bool need = sm && lmax > m_run + (float)kRescaleSlack;
          if (__builtin_amdgcn_ballot_w64(need) != 0) {
            const float tmax = max_halves(lmax);
            const float m_new = fmaxf(m_run, tmax);
            const bool first = m_run == -INFINITY;
            const float alpha = first ? 0.f : __builtin_amdgcn_exp2f(m_run - m_new);
            m_run = m_new;
            l_run *= alpha;
            alpha_pend = alpha;
            resc_pend = __builtin_amdgcn_ballot_w64(!first && alpha != 1.f) != 0;
          }
        } else if constexpr (step == kSmDone) {
          if (sm) l_run = lacc;
        }
      };
      // The exp2 pipeline, one pair of the lane's 16 scores per PV step k =
      // step - kSmPipe0: P = 2^(s - m) <= 2^kRescaleSlack (masked and
      // far-below-max scores give 0); l sums P in fp32 with v_add (a v_dot2
      // over the packed pair would wait for the MFMA in flight, like every
      // dot instruction). The lead piece runs after the step's value-read
      // wait, before its first MFMA (while the previous step's second MFMA
      // runs): s - m of pair k, the packing of pair k-1 and the sum of its
      // first value. The mid piece runs between the step's two MFMAs: the sum
      // of pair k-1's second value and 2^(s - m) of pair k. The empty asm
      // statements hold each result in its piece: without them the compiler
      // sinks the chain past the PV loop (its only uses are after it), where
      // no MFMA hides it.
      typedef E E2 __attribute__((ext_vector_type(2)));
      auto sm_lead = [&](auto step_c) {
        constexpr int k = decltype(step_c)::value - kSmPipe0;
        if constexpr (k >= 0 && k <= 7) {
          sd[2 * k] = s_next[2 * k] - m_run;
          sd[2 * k + 1] = s_next[2 * k + 1] - m_run;
          asm volatile("" : "+v"(sd[2 * k]), "+v"(sd[2 * k + 1]));
        }
        if constexpr (k >= 1 && k <= 8) {
          const E2 pr = {(E)sx[2 * k - 2], (E)sx[2 * k - 1]};
          pw_next[k - 1] = __builtin_bit_cast(uint32_t, pr);
          lacc = (k == 1 ? l_run : lacc) + sx[2 * k - 2];
          asm volatile("" : "+v"(pw_next[k - 1]), "+v"(lacc));
        }
      };
      auto sm_mid = [&](auto step_c) {
        constexpr int k = decltype(step_c)::value - kSmPipe0;
        if constexpr (k >= 1 && k <= 8) {
          lacc += sx[2 * k - 1];
          asm volatile("" : "+v"(lacc));
        }
        if constexpr (k >= 0 && k <= 7) {
          sx[2 * k] = __builtin_amdgcn_exp2f(sd[2 * k]);
          sx[2 * k + 1] = __builtin_amdgcn_exp2f(sd[2 * k + 1]);
          asm volatile("" : "+v"(sx[2 * k]), "+v"(sx[2 * k + 1]));
        }
      };


      // ---- partner-head O rows *= alpha where the partner's softmax(t) moved its max ----
      if (__builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, pflag)) != 0) {
        const float a1 = lds_ld<float>(L, atab + pw * kAtabWave + 4 * (lane & 31));  // partner head lane%32
        settle_acc(acc);
#pragma unroll
        for (int nb = 8; nb < 16; ++nb) {
          acc[nb] *= a1;
          pin_agpr(acc[nb]);
          __builtin_amdgcn_sched_barrier(0);
        }
        acc_ready(acc);
      }

      // ---- PV(t): O^T[c][head] += V^T[c][pos] . P^T[pos][head] over the pair's 64 heads ----
      // The value operand goes in as A and P as B, so the accumulators hold O
      // transposed: lane = head, register i of block cb = column 32cb +
      // 8(i/4) + 4g2 + (i%4) of this wave's half (a per-head factor is a
      // per-lane scalar). Step s = (ks, column block cb) waits for its value reads (count from
      // pv_later: LDS operations complete in order), runs the own-head and the
      // partner-head MFMA on them, then issues the reads of step s + kPvDepth
      // into the freed ring slot. After step kRotStep the four RoPE reads of
      // tile t+2 go out (once this wave's k_rope, cos and sin copies have
      // landed; past the segment they rotate the clamped rows of a tile that
      // is never used). Softmax(t+1) and the rotation take two slots per step.
      operands_ready(p_cur[0], p_cur[1]);
      u32x2 xe[4];  // FP8 cache: staged codes of half the wave's rows of tile t+2
      const uint32_t e_src = dbuf + fp8_stage_off(wave) + 8 * lane;
      const uint32_t e_dst = dbuf + ct_row_off(8 * wave) + 16 * lane;
      auto exp_piece = [&](auto slot_c) {
        constexpr int q = decltype(slot_c)::value - kExpSlot0;
        if constexpr (kFp8 && q >= 0 && q < 8) {
          if constexpr (q == 4)  // rows 4..7's reads (issued after slot 3) have landed
            asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(xe[0]), "+v"(xe[1]), "+v"(xe[2]), "+v"(xe[3]));
          fp8_exp_row<q>(L, e_dst, xe[q & 3]);
          if constexpr (q == 3) fp8_exp_issue<1>(e_src, xe);
        }
      };
      RotIn rot;
      float rot_k0[4], rot_k1[4], rot_a[4], rot_b[4];
      auto rot_piece = [&](auto slot_c) {
        // slot r: widen pairs e = 2r, 2r+1 (r < 2); products and sums of
        // pair r-2 (r = 2..5); store (r = 6)
        constexpr int r = decltype(slot_c)::value - kRotSlot0;
        if constexpr (r == 0) {
          // FP8 cache: step kExpWaitStep has waited for the RoPE reads
          if constexpr (kFp8) asm volatile("" : "+v"(rot.k8a), "+v"(rot.k8b), "+v"(rot.c), "+v"(rot.s));
          else rot_wait<KT, kFp8, rot_later()>(rot);
        }
        if constexpr (r >= 0 && r < 2) {
#pragma unroll
          for (int e = 2 * r; e < 2 * r + 2; ++e) {
            rot_k0[e] = rot_k<KT, kFp8>(rot, false, e);
            rot_k1[e] = rot_k<KT, kFp8>(rot, true, e);
            asm volatile("" : "+v"(rot_k0[e]), "+v"(rot_k1[e]));
          }
        }
        if constexpr (r >= 2 && r < 6) {
          constexpr int e = r - 2;
          rot_a[e] = rot_k0[e] * rot.c[e] - rot_k1[e] * rot.s[e];
          rot_b[e] = rot_k0[e] * rot.s[e] + rot_k1[e] * rot.c[e];
          asm volatile("" : "+v"(rot_a[e]), "+v"(rot_b[e]));
        }
        if constexpr (r == 6) rot_store<KT>(L, rot, rot_a, rot_b);
      };
      static_for<kPvSteps>([&](auto step_c) {
        constexpr int step = decltype(step_c)::value;
        constexpr int ks = step >> 3, cb = step & 7;
        TrPair& bc = tr[step % kPvDepth];
        if constexpr (step == 0) {
          wait_lgkm<pv_later(0)>(bc.x0, bc.x1, pp[0], pp[1]);
        } else if constexpr (kFp8 && step == kExpWaitStep) {
          static_assert(pv_wait_n(kExpWaitStep, true) == 0, "full wait");
          asm volatile("s_waitcnt lgkmcnt(0)"
                       : "+v"(bc.x0), "+v"(bc.x1), "+v"(xe[0]), "+v"(xe[1]), "+v"(xe[2]), "+v"(xe[3]), "+v"(rot.k8a),
                         "+v"(rot.k8b), "+v"(rot.c), "+v"(rot.s));
        } else {
          wait_lgkm<pv_wait_n(step, kFp8)>(bc.x0, bc.x1);
        }
        i16x8 bv;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          bv[e] = bc.x0[e];
          bv[4 + e] = bc.x1[e];
        }
        const vec bvec = __builtin_bit_cast(vec, bv);
        // the lead piece stays after the wait: hoisted above it, as the
        // compiler would, it leaves the MFMA right behind the wait, with a
        // wait state between them
        __builtin_amdgcn_sched_barrier(0);
        sm_lead(step_c);
        __builtin_amdgcn_sched_barrier(0);
        // A wave issues in order and an MFMA waits for the previous one to
        // leave the pipe, so VALU work placed between the two MFMAs runs while
        // the first executes; placed after both it would wait for the second
        // to issue.
        O_::mma_a(acc[cb], bvec, p_cur[ks]);
        __builtin_amdgcn_sched_barrier(0);
        sm_piece(std::integral_constant<int, 2 * step>());
        sm_mid(step_c);
        rot_piece(std::integral_constant<int, 2 * step>());
        exp_piece(std::integral_constant<int, 2 * step>());
        __builtin_amdgcn_sched_barrier(0);
        O_::mma_a(acc[8 + cb], bvec, pp[ks]);
        if constexpr (step + kPvDepth < kPvSteps) b_issue(bc, std::integral_constant<int, step + kPvDepth>());
        if constexpr (step >= kPostStep0 && step <= kPostStep1) __builtin_amdgcn_sched_barrier(0);
        if constexpr (step == kRotStep) {
          // this wave's k_rope / cos / sin copies of tile t+2 have landed (an
          // fp8 tile's k_rope parts come with every row copy)
          if constexpr (kFp8) wait_vm<0>();
          else wait_vm<kDmaPerWave - 3>();
          if constexpr (kFp8) rot = rot_issue<kFp8>(L, dbuf, wave, lane);
          else rot = rot_issue_at(L, dbuf + kRopeOff + lrot, kCosOff + 1024 * wave + 16 * lane);
          if constexpr (kFp8) fp8_exp_issue<0>(e_src, xe);
        }
        sm_piece(std::integral_constant<int, 2 * step + 1>());
        rot_piece(std::integral_constant<int, 2 * step + 1>());
        exp_piece(std::integral_constant<int, 2 * step + 1>());
        __builtin_amdgcn_sched_barrier(0);
      });
      // ---- publish P(t+1) and softmax(t+1)'s rescale for the partner ----
      {
        const int npar = (t + 1) & 1;
        const uint32_t ptab = kPtabOff + npar * kPtabPar + wave * 2048 + 16 * lane;
        typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
        p_cur[0] = __builtin_bit_cast(vec, u32x4{pw_next[0], pw_next[1], pw_next[2], pw_next[3]});
        p_cur[1] = __builtin_bit_cast(vec, u32x4{pw_next[4], pw_next[5], pw_next[6], pw_next[7]});
        lds_st(L, ptab, p_cur[0]);
        lds_st(L, ptab + 1024, p_cur[1]);
        // lanes 0..31 store the alpha of head lane, every lane from 32 on the
        // flag word (alpha slot 32) with the same value: one store, no exec mask
        const uint32_t natab = kAtabOff + npar * kAtabPar + wave * kAtabWave;
        lds_st(L, natab + 4 * min(lane, 32), lane < 32 ? alpha_pend : (resc_pend ? 1.f : 0.f));
      }
#ifdef LA_PHASE_STAMPS
      LA_TSTAMP(tt3);
#endif
      wait_vm<0>();  // this wave's copies of tile t+2 (issued in this iteration) have landed
      if constexpr (kPaged) tie(blk_cur);  // and the table entry loaded with them
#ifdef LA_PHASE_STAMPS
      LA_TSTAMP(tt4);
      if (t >= 0) {
        stamps_[11] += tt1 - tt0;
        stamps_[12] += tt2 - tt1;
        stamps_[13] += tt3 - tt2;
        stamps_[14] += tt4 - tt3;
        stamps_[15] += 1;
      }
#endif
      cur_b = nxt_b;
      nxt_b = dbuf_b;
      dbuf_b = kNBuf * kBufBytes - cur_b - nxt_b;
    }

    LA_STAMP(7);
    wait_vm<0>();  // the last iteration's copies (of a tile past the segment) have landed
    // ---- segment end: l over both lane halves; write the slot ----
    // This wave holds the pair's 64 heads (own: acc[0..7], partner:
    // acc[8..15]) over column half ch, transposed: lane = head (lane%32),
    // register i of block cb = column 32cb + 8(i/4) + 4g2 + (i%4). Each head's
    // half row goes out unnormalised as fp16 N * 2^-e, 2^(e-1) <= max |N| <
    // 2^e (every value below 1 in magnitude, 11 significant bits relative to
    // the half-row max); the max is lane-local over 128 values, then over the
    // two lane halves. The softmax owner writes m and m + log2(l).
    settle_acc(acc);
    const int le = lane_id();  // fresh: the prologue's lane index would come back from a spill slot
    const int g2 = le >> 5;
    const float l_tot = sum_halves(l_run);
    const int64_t slot = (int64_t)chunk + s;
    const int64_t hqg = slot * p.Hq + group * kHG;  // slot row of head 0 of the group
    if (le < 32 && 32 * wave + le < hg_heads) {
      p.part_lse[hqg + 32 * wave + le] = m_run + log2f(l_tot);
      p.part_m[hqg + 32 * wave + le] = m_run;
    }
    float mo = 0.f, mp = 0.f;
#pragma unroll
    for (int cb = 0; cb < 8; ++cb) {
      const f32x16 a = acc[cb], b = acc[8 + cb];
#pragma unroll
      for (int i = 0; i < 16; i += 2) {
        mo = max3abs(a[i], a[i + 1], mo);
        mp = max3abs(b[i], b[i + 1], mp);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    mo = max_halves(mo);
    mp = max_halves(mp);
    const int eo = __builtin_amdgcn_frexp_expf(mo);  // 0 for a zero row
    const int ep = __builtin_amdgcn_frexp_expf(mp);
    if (le < 32) {
      if (32 * wave + le < hg_heads) p.part_scale[2 * (hqg + 32 * wave + le) + ch] = __builtin_amdgcn_ldexpf(1.f, eo);
      if (32 * pw + le < hg_heads) p.part_scale[2 * (hqg + 32 * pw + le) + ch] = __builtin_amdgcn_ldexpf(1.f, ep);
    }
    const float mulo = __builtin_amdgcn_ldexpf(1.f, -eo), mulp = __builtin_amdgcn_ldexpf(1.f, -ep);
    // Write-out through LDS (the tile buffers are idle now): each wave stages
    // its 64 half rows as fp16 rows of kStagePitch bytes (own heads 0..31,
    // then the partner's), 8-B writes of the 4 consecutive columns a lane
    // holds per (block, i/4); then each round reads two whole rows back (16 B
    // per lane) and stores them: every store instruction writes eight full
    // 128-B lines.
    lds_barrier();  // every wave has finished with the tile buffers
    LA_STAMP(8);
    const uint32_t sbase = kStageBytes * wave;
    // stage(b): half rows b (0: own heads, staged rows 0..31; 1: the
    // partner's, rows 32..63), one 16-column block at a time
    auto stage = [&](auto b_c) {
      constexpr int b = decltype(b_c)::value;
#pragma unroll
      for (int cb = 0; cb < 8; ++cb) {
        const f32x16 v = acc[8 * b + cb] * (b == 0 ? mulo : mulp);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          i16x4 h4;
#pragma unroll
          for (int r = 0; r < 4; ++r) h4[r] = __builtin_bit_cast(short, (_Float16)v[4 * q + r]);
          lds_st(L, sbase + (32 * b + (le & 31)) * kStagePitch + (32 * cb + 8 * q + 4 * g2) * 2, h4);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    };
    const int lr = lane_id();  // fresh index: values derived earlier would come back from spill slots
    const uint32_t rd = sbase + (lr >> 5) * kStagePitch + 16 * (lr & 31);
    // read16(h, x): staged rows 32h + 2j (lanes 0..31) and 32h + 2j + 1
    // (lanes 32..63), j < 16, 16 B per lane
    auto read16 = [&](auto h_c, i16x8(&x)[16]) {
      constexpr int h = decltype(h_c)::value;
      static_for<16>([&](auto j_c) {
        constexpr int j = decltype(j_c)::value;
        x[j] = lds_rd128<i16x8, 2 * kStagePitch * (16 * h + j)>(L, rd);
      });
    };
    // The slot rows of this group in one raw buffer that ends at its last
    // valid head row, so a store of a row past it is dropped by the range
    // check (raw buffer stores outside num_records write nothing). A full
    // group (every benchmark shape) puts the row in the scalar offset: one
    // scalar add per store, no exec mask and no vector address arithmetic;
    // a partial one puts it in the vector offset, which the range check sees.
    const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
        reinterpret_cast<_Float16*>(p.part_o) + hqg * kDc, 0, hg_heads * kDc * 2, kBufferRsrcWord3);
    const int vlane = (lr >> 5) * (kDc * 2) + 512 * ch + 16 * (lr & 31);
    // row offsets of staged rows 0 and 32, made here (the empty asm) so the
    // per-store offsets below are one add each rather than 32 values
    // computed at kernel start and held in spill slots
    int own = 32 * wave * (kDc * 2), par = 32 * pw * (kDc * 2);
    asm volatile("" : "+s"(own), "+s"(par));
    auto store16 = [&](const int rows, const i16x8(&x)[16]) {
      if (hg_heads == kHG) {
        static_for<16>([&](auto j_c) {
          constexpr int j = decltype(j_c)::value;
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, x[j]), rsrc, vlane, rows + 2 * j * (kDc * 2),
                                                 kCpolSc1);
        });
      } else {
        static_for<16>([&](auto j_c) {
          constexpr int j = decltype(j_c)::value;
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, x[j]), rsrc, vlane + rows + 2 * j * (kDc * 2),
                                                 0, kCpolSc1);
        });
      }
    };
    // Two halves, so each half's LDS reads and stores overlap other work:
    // the own half rows' reads run while the partner's are converted and
    // staged, and their stores while the partner's reads run. Each read
    // lands in its own registers, held (the empty asm ties) until the
    // lgkmcnt(0) that covers it.
    stage(std::integral_constant<int, 0>());
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's own-half writes before their reads
    i16x8 xa[16];
    read16(std::integral_constant<int, 0>(), xa);
    stage(std::integral_constant<int, 1>());
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(xa[0]), "+v"(xa[1]), "+v"(xa[2]), "+v"(xa[3]), "+v"(xa[4]), "+v"(xa[5]), "+v"(xa[6]), "+v"(xa[7]));
    asm volatile("" : "+v"(xa[8]), "+v"(xa[9]), "+v"(xa[10]), "+v"(xa[11]), "+v"(xa[12]), "+v"(xa[13]), "+v"(xa[14]), "+v"(xa[15]));
    store16(own, xa);
    i16x8 xb[16];
    read16(std::integral_constant<int, 1>(), xb);  // the partner half's writes completed at the wait above
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(xb[0]), "+v"(xb[1]), "+v"(xb[2]), "+v"(xb[3]), "+v"(xb[4]), "+v"(xb[5]), "+v"(xb[6]), "+v"(xb[7]));
    asm volatile("" : "+v"(xb[8]), "+v"(xb[9]), "+v"(xb[10]), "+v"(xb[11]), "+v"(xb[12]), "+v"(xb[13]), "+v"(xb[14]), "+v"(xb[15]));
    store16(par, xb);
    LA_STAMP(9);
    lo = seg_hi;
    ++s;
  }
#ifdef LA_PHASE_STAMPS
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  LA_STAMP(10);
  if ((threadIdx.x & 63) == 0 && blockIdx.x < kStampBlocks)
    for (int i = 0; i < kStampSlots; ++i) g_attn_stamps[((size_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * kStampSlots + i] = stamps_[i];
#endif
}

// Copies-only variant of the attention kernel, for measuring the streaming
// ceiling of its copy schedule: the same grid and block mapping
// (block_coords), the same segment walk, and per tile the same 11 HBM->LDS
// copies per wave (issue_tile_dma: c_t rows, k_rope, cos, sin; non-temporal
// cache rows) into a ring of kRing tile buffers, with one barrier per tile and
// no compute, LDS reads or stores. Iteration t issues tile t + kRing - 1 and
// then waits for tile t + 1, so kRing - 1 tiles are in flight at the wait:
// kRing = 3 is the attention kernel's ring (it keeps one tile in flight at
// its end-of-iteration wait, two while it computes), kRing = 4 the deepest
// ring 160 KB of LDS holds. 16-bit contiguous caches only.
template <int kRing>
__global__ __launch_bounds__(kThreads) void stream_copies_kernel(DecodeProblem p, int groups) {
  static_assert(kRing >= 2 && kRing * kBufBytes + 2 * kT * 128 <= 160 * 1024, "ring fits the LDS");
  constexpr uint32_t kCs = kRing * kBufBytes;  // one cos / sin buffer (never read)
  extern __shared__ __attribute__((aligned(1024))) char lds_raw[];
  lchar* L = (lchar*)lds_raw;
  const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
  int chunk, group;
  block_coords(p.num_chunks, groups, &chunk, &group);
  if (chunk >= p.num_chunks) return;
  const int64_t end_all = seq_begin(p, p.num_seqs);
  int64_t lo = (int64_t)chunk * p.chunk_len;
  const int64_t hi = min(lo + (int64_t)p.chunk_len, end_all);
  lo = max(lo, seq_begin(p, 0));
  if (lo >= hi) return;
  int s = find_seq_mfma(p, lo);
  while (lo < hi) {
    const int64_t s_lo = seq_begin(p, s);
    lo = max(lo, s_lo);
    if (lo >= hi) break;
    const int64_t s_hi = seq_end(p, s);
    if (s_hi <= lo) {
      if (++s >= p.num_seqs) break;
      continue;
    }
    const int64_t seg_hi = min(hi, s_hi);
    SegCtx sg;
    sg.base = reinterpret_cast<const char*>(p.kv) + lo * kRowBytes;
    sg.pos0 = lo - s_lo;
    sg.last = (int)(seg_hi - lo - 1);
    sg.seq = s;
    sg.tab = nullptr;
    sg.tile0 = 0;
    const int ntiles = (sg.last + kT) / kT;
    lds_barrier();
    auto issue = [&](int k) {
      const TileDma d = tile_dma<false>(sg, k, tile_base<false, false>(p, sg, k, 0), wave, lane_id());
      const uint32_t buf = (uint32_t)(k % kRing) * kBufBytes;
      const int lane = lane_id();
      static_for<kDmaPerWave>([&](auto j) {
        constexpr int J = decltype(j)::value;
        if constexpr (J < 9) {
          issue_copy<J>(p, sg, k, L, buf, wave, lane, d);
        } else {  // cos / sin rows into the one table buffer
          const int row = 8 * wave + (lane >> 3);
          const int r = min(k * kT + row, sg.last);
          const uint32_t toff = (uint32_t)(rope_row(p, sg.pos0 + r) * (kDr / 2) * 4 + (lane & 7) * 16);
          const float* tab = J == 9 ? p.rope_cos : p.rope_sin;
          __builtin_amdgcn_global_load_lds(reinterpret_cast<const char*>(tab) + toff,
                                           (lds_void*)(L + kCs + (J == 9 ? 0 : kT * 128) + 8 * wave * 128), 16, 0, 0);
        }
      });
    };
    for (int k = 0; k < kRing - 1; ++k) issue(k);
    for (int t = 0; t < ntiles; ++t) {
      lds_barrier();  // every wave is done with buffer (t - 1) % kRing
      issue(t + kRing - 1);  // tiles past the segment re-read its last rows
      wait_vm_ext<kDmaPerWave * (kRing - 2)>();  // this wave's copies of tile t + 1 have landed
    }
    wait_vm<0>();
    lo = seg_hi;
    ++s;
  }
}

// q_prep = E([q_abs[row] (dc) | q_rope[row] (dR)] * scale_log2) in the
// operand-order layout (qprep_index); row = s * Hq + hq. One thread per 8
// consecutive elements (72 per row for dc = 512, dR = 64), i.e. per 16-B slot.
// zero_out: the decode output, which a latent-half merge adds into (zeroed
// grid-stride, before the early return).
template <typename KT>
__global__ __launch_bounds__(256) void prep_q_kernel(const float* __restrict__ q_abs, const float* __restrict__ q_rope,
                                                     float scale, typename Ops<KT>::elem* __restrict__ out,
                                                     int64_t rows, int Hq, float* __restrict__ zero_out,
                                                     int64_t zero_n) {
  typedef typename Ops<KT>::elem E;
  typedef typename Ops<KT>::vec vec;
  constexpr int kPer = (kDc + kDr) / 8;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (zero_out)
    for (int64_t z = i; z < zero_n; z += (int64_t)gridDim.x * 256) zero_out[z] = 0.f;
  if (i >= rows * kPer) return;
  const int64_t row = i / kPer;
  const int j = (int)(i - row * kPer);
  const float* src = j < kDc / 8 ? q_abs + row * kDc + 8 * j : q_rope + row * kDr + 8 * (j - kDc / 8);
  const f32x4 a = *reinterpret_cast<const f32x4*>(src);
  const f32x4 b = *reinterpret_cast<const f32x4*>(src + 4);
  vec v;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    v[e] = (E)(a[e] * scale);
    v[4 + e] = (E)(b[e] * scale);
  }
  const int64_t qrow = (row / Hq) * qprep_rows_per_seq(Hq) + row % Hq;
  *reinterpret_cast<vec*>(out + qprep_index(qrow, 8 * j)) = v;
}

template <typename KT, bool kPaged, bool kFp8 = false>
hipError_t launch_t(const DecodeProblem& p, hipStream_t stream, hipEvent_t ev_begin, hipEvent_t ev_end) {
  static bool attr_set = false;  // per instance; setting it twice is harmless
  if (!attr_set) {
    const void* fn = reinterpret_cast<const void*>(&decode_mfma_kernel<KT, kPaged, kFp8>);
    hipFuncAttributes fa;
    hipError_t e = hipFuncGetAttributes(&fa, fn);
    if (e != hipSuccess) return e;
    if (fa.sharedSizeBytes != 0) return hipErrorInvalidKernelFile;  // LDS offsets would not be addresses
    e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, kLdsBytes);
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  const int groups = (p.Hq + kHG - 1) / kHG;
  const int64_t blocks = mfma_grid_blocks(p.num_chunks, groups);
  if (ev_begin || ev_end) {
    // the events time this kernel's execution alone (no dispatch gap)
    hipExtLaunchKernelGGL((decode_mfma_kernel<KT, kPaged, kFp8>), dim3((unsigned)blocks), dim3(kThreads), kLdsBytes,
                          stream, ev_begin, ev_end, 0, p, groups);
  } else {
    hipLaunchKernelGGL((decode_mfma_kernel<KT, kPaged, kFp8>), dim3((unsigned)blocks), dim3(kThreads), kLdsBytes, stream,
                       p, groups);
  }
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
  if (p.kv_dtype != LA_DTYPE_BF16 && p.kv_dtype != LA_DTYPE_F16 && p.kv_dtype != LA_DTYPE_FP8_E4M3) return false;
  if (p.dc != kDc || p.dR != kDr || p.Hq % 16 != 0 || p.Hq <= 0) return false;
  if (p.rope_rows > (1 << 24) || (p.rope_rows == 0 && p.total_rows > (1 << 24))) return false;
  // uniform sequences: row indices fit in 31 bits (find_seq_mfma); offsets
  // are int32, so they always do
  if (!p.offsets && (int64_t)p.num_seqs * p.seq_len > INT32_MAX) return false;
  // paged: a 32-row tile must lie inside one block
  if (p.block_table && (p.block_size % kT != 0 || p.chunk_len % kT != 0)) return false;
  // 16-byte aligned cache rows, table rows and query rows
  if ((reinterpret_cast<uintptr_t>(p.kv) & 15) || (reinterpret_cast<uintptr_t>(p.rope_cos) & 15) ||
      (reinterpret_cast<uintptr_t>(p.rope_sin) & 15) || (reinterpret_cast<uintptr_t>(p.q_rope) & 15) ||
      (reinterpret_cast<uintptr_t>(p.q_abs) & 15))
    return false;
  return device_is_gfx950();
}

hipError_t launch_prep_q(const DecodeProblem& p, hipStream_t stream, float* zero_out, int64_t zero_n) {
  const int64_t rows = (int64_t)p.num_seqs * p.Hq;
  const int64_t threads = rows * ((kDc + kDr) / 8);
  if (threads == 0) return hipSuccess;
  const unsigned blocks = (unsigned)((threads + 255) / 256);
  if (p.kv_dtype != LA_DTYPE_F16)  // bf16 and fp8 caches run bf16 MFMAs
    hipLaunchKernelGGL(prep_q_kernel<__hip_bfloat16>, dim3(blocks), dim3(256), 0, stream, p.q_abs, p.q_rope,
                       p.scale_log2, reinterpret_cast<Ops<__hip_bfloat16>::elem*>(p.q_prep), rows, p.Hq, zero_out,
                       zero_n);
  else
    hipLaunchKernelGGL(prep_q_kernel<__half>, dim3(blocks), dim3(256), 0, stream, p.q_abs, p.q_rope, p.scale_log2,
                       reinterpret_cast<Ops<__half>::elem*>(p.q_prep), rows, p.Hq, zero_out, zero_n);
  return hipGetLastError();
}

hipError_t launch_stream_copies(const DecodeProblem& p, int ring, hipStream_t stream) {
  if (p.block_table || (p.kv_dtype != LA_DTYPE_BF16 && p.kv_dtype != LA_DTYPE_F16) || (ring != 3 && ring != 4))
    return hipErrorInvalidValue;
  const void* fn = ring == 3 ? reinterpret_cast<const void*>(&stream_copies_kernel<3>)
                             : reinterpret_cast<const void*>(&stream_copies_kernel<4>);
  const int lds = ring * kBufBytes + 2 * kT * 128;
  hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
  if (e != hipSuccess) return e;
  const int groups = (p.Hq + kHG - 1) / kHG;
  const int64_t blocks = mfma_grid_blocks(p.num_chunks, groups);
  if (ring == 3)
    hipLaunchKernelGGL(stream_copies_kernel<3>, dim3((unsigned)blocks), dim3(kThreads), lds, stream, p, groups);
  else
    hipLaunchKernelGGL(stream_copies_kernel<4>, dim3((unsigned)blocks), dim3(kThreads), lds, stream, p, groups);
  return hipGetLastError();
}

hipError_t launch_decode_mfma(const DecodeProblem& p, hipStream_t stream, hipEvent_t ev_begin, hipEvent_t ev_end) {
  if (p.block_table) {
    if (p.kv_dtype == LA_DTYPE_FP8_E4M3) return launch_t<__hip_bfloat16, true, true>(p, stream, ev_begin, ev_end);
    if (p.kv_dtype == LA_DTYPE_BF16) return launch_t<__hip_bfloat16, true>(p, stream, ev_begin, ev_end);
    return launch_t<__half, true>(p, stream, ev_begin, ev_end);
  }
  if (p.kv_dtype == LA_DTYPE_FP8_E4M3) return launch_t<__hip_bfloat16, false, true>(p, stream, ev_begin, ev_end);
  if (p.kv_dtype == LA_DTYPE_BF16) return launch_t<__hip_bfloat16, false>(p, stream, ev_begin, ev_end);
  return launch_t<__half, false>(p, stream, ev_begin, ev_end);
}

#ifdef LA_PHASE_STAMPS
// Phase-timing build: copies (clear == 0) the attention kernel's stamps of
// blocks 0 .. blocks-1 (4 waves x 12 slots each) to host, or zeroes them.
extern "C" int la_phase_attn_stamps(unsigned long long* host, int blocks, int clear) {
  const size_t n = sizeof(unsigned long long) * 4 * kStampSlots * (size_t)(blocks < kStampBlocks ? blocks : kStampBlocks);
  if (clear) {
    static unsigned long long zeros[kStampBlocks * 4 * kStampSlots];
    return (int)hipMemcpyToSymbol(HIP_SYMBOL(g_attn_stamps), zeros, sizeof(zeros), 0, hipMemcpyHostToDevice);
  }
  return (int)hipMemcpyFromSymbol(host, HIP_SYMBOL(g_attn_stamps), n, 0, hipMemcpyDeviceToHost);
}
#endif
}  // namespace la
