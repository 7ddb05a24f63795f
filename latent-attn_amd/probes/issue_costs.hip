// Issue costs beside an in-flight MFMA, one wave per SIMD (the attention
// kernel's occupancy): which instructions placed between two 32x32x16 bf16
// MFMAs hide under the matrix core's 32 cycles, and which wait for it.
//
// One workgroup of 1 or 4 waves; each step issues one MFMA (two AGPR
// accumulators, alternating) and then the variant's instructions; the result
// is shader-clock cycles per step (s_memtime around 2000 x 8 steps).
//
// Memory: LDS reads and writes stay inside the 8 KB array (byte offsets
// lane * 16 + at most 2048, 16-byte aligned); the copies read the wave's own
// 64 KB window of a 1 MB buffer (offset & 0xffff) into the wave's own 1 KB
// of LDS, with at most 40 in flight. Nothing depends on the values computed.
//
// Build and run (on the GPU box):
//   hipcc --offload-arch=gfx950 -O3 -std=c++17 -Xclang -target-feature -Xclang -packed-fp32-ops \
//     latent-attn_amd/probes/issue_costs.hip -o /tmp/issue_costs && /tmp/issue_costs
#include <hip/hip_runtime.h>
#include <cstdio>

typedef float f16v __attribute__((ext_vector_type(16)));
typedef int i4 __attribute__((ext_vector_type(4)));
typedef int i2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) void lds_void;

constexpr int kGlobalBytes = 1 << 20;
constexpr int kIters = 2000;

enum Variant {
  kMfma, kAdd3, kAdd6, kExp2, kExp3, kAddExp2, kMax3x2, kMulx2, kCndx2, kMov64x2, kRflx2, kCmpx2,
  kCvtPkBf16x2, kCvtPkF16x2, kPermx1, kDot2cBf16, kDot2Bf16, kDot2cF16, kTrRead2, kDsWrite64x2,
  kGlobalLds, kBufferLds, kGlobalLdsAlone, kBufferLdsAlone, kNumVariants
};
const char* const kNames[kNumVariants] = {
    "mfma only", "+ 3 v_add_f32", "+ 6 v_add_f32", "+ 2 v_exp_f32", "+ 3 v_exp_f32", "+ v_add_f32 + 2 v_exp_f32",
    "+ 2 v_max3_f32", "+ 2 v_mul_f32", "+ 2 v_cndmask_b32", "+ 2 v_mov_b64", "+ 2 v_readfirstlane_b32",
    "+ 2 v_cmp_gt_f32", "+ 2 v_cvt_pk_bf16_f32", "+ 2 v_cvt_pk_f16_f32", "+ 1 v_perm_b32",
    "+ 1 v_dot2c_f32_bf16", "+ 1 v_dot2_f32_bf16", "+ 1 v_dot2c_f32_f16",
    "+ 2 ds_read_b64_tr_b16, lgkmcnt(2)", "+ 2 ds_write_b64", "+ 1 global_load_lds_dwordx4",
    "+ 1 buffer_load_dwordx4 lds", "global_load_lds_dwordx4 alone", "buffer_load_dwordx4 lds alone"};

template <int K>
__global__ __launch_bounds__(256) void probe(unsigned long long* out, const char* g) {
  __shared__ __attribute__((aligned(1024))) char L[8192];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  for (int i = tid; i < 2048; i += blockDim.x) reinterpret_cast<int*>(L)[i] = i;
  __syncthreads();
  f16v acc0 = {}, acc1 = {};
  const i4 a = {tid, 1, 2, 3}, b = {4, 5, 6, tid};
  float x0 = tid * 1e-3f, x1 = x0 + 1, x2 = x0 + 2, x3 = x0 + 3, x4 = x0 + 4, x5 = x0 + 5;
  i2 d0 = {tid, 1}, d1 = {2, tid};
  unsigned la = 16u * (unsigned)lane;
  const char* gb = g + __builtin_amdgcn_readfirstlane(w) * 65536;
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(gb), 0, 65536, 0x00020000);
  unsigned long long t0, t1;
  asm volatile("s_memtime %0\n\ts_waitcnt lgkmcnt(0)" : "=s"(t0)::"memory");
  for (int i = 0; i < kIters; ++i) {
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      f16v& acc = (u & 1) ? acc1 : acc0;
      const unsigned off = ((unsigned)(i * 8 + u) * 1024u + 16u * lane) & 65535u;
      if constexpr (K != kGlobalLdsAlone && K != kBufferLdsAlone)
        asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
#define V4 "+v"(x0), "+v"(x1), "+v"(x2), "+v"(x3)
      if constexpr (K == kAdd3) asm volatile("v_add_f32 %0, 1.0, %0\n\tv_add_f32 %1, 1.0, %1\n\tv_add_f32 %2, 1.0, %2" : V4);
      if constexpr (K == kAdd6)
        asm volatile("v_add_f32 %0, 1.0, %0\n\tv_add_f32 %1, 1.0, %1\n\tv_add_f32 %2, 1.0, %2\n\t"
                     "v_add_f32 %3, 1.0, %3\n\tv_add_f32 %4, 1.0, %4\n\tv_add_f32 %5, 1.0, %5"
                     : "+v"(x0), "+v"(x1), "+v"(x2), "+v"(x3), "+v"(x4), "+v"(x5));
      if constexpr (K == kExp2) asm volatile("v_exp_f32 %0, %0\n\tv_exp_f32 %1, %1" : V4);
      if constexpr (K == kExp3) asm volatile("v_exp_f32 %0, %0\n\tv_exp_f32 %1, %1\n\tv_exp_f32 %2, %2" : V4);
      if constexpr (K == kAddExp2) asm volatile("v_add_f32 %0, 1.0, %0\n\tv_exp_f32 %1, %1\n\tv_exp_f32 %2, %2" : V4);
      if constexpr (K == kMax3x2) asm volatile("v_max3_f32 %0, %1, %2, %3\n\tv_max3_f32 %1, %2, %3, %0" : V4);
      if constexpr (K == kMulx2) asm volatile("v_mul_f32 %0, %1, %2\n\tv_mul_f32 %1, %2, %3" : V4);
      if constexpr (K == kCndx2) asm volatile("v_cndmask_b32 %0, %1, %2, vcc\n\tv_cndmask_b32 %1, %2, %3, vcc" : V4 :: "vcc");
      if constexpr (K == kMov64x2) asm volatile("v_mov_b64 %0, %1\n\tv_mov_b64 %1, %0" : "+v"(d0), "+v"(d1));
      if constexpr (K == kRflx2) asm volatile("v_readfirstlane_b32 s40, %0\n\tv_readfirstlane_b32 s41, %1" : V4 :: "s40", "s41");
      if constexpr (K == kCmpx2) asm volatile("v_cmp_gt_f32 vcc, %0, %1\n\tv_cmp_gt_f32 s[42:43], %2, %3" : V4 :: "vcc", "s42", "s43");
      if constexpr (K == kCvtPkBf16x2) asm volatile("v_cvt_pk_bf16_f32 %0, %2, %3\n\tv_cvt_pk_bf16_f32 %1, %2, %3" : "=&v"(d0[0]), "=&v"(d0[1]), "+v"(x0), "+v"(x1));
      if constexpr (K == kCvtPkF16x2) asm volatile("v_cvt_pk_f16_f32 %0, %2, %3\n\tv_cvt_pk_f16_f32 %1, %2, %3" : "=&v"(d0[0]), "=&v"(d0[1]), "+v"(x0), "+v"(x1));
      if constexpr (K == kPermx1) asm volatile("v_perm_b32 %0, %1, %2, %3" : "=v"(d1[0]) : "v"(x0), "v"(x1), "v"(la));
      if constexpr (K == kDot2cBf16) asm volatile("v_dot2c_f32_bf16 %0, %1, %1" : "+v"(x2), "+v"(la));
      if constexpr (K == kDot2Bf16) asm volatile("v_dot2_f32_bf16 %0, %1, %1, %0" : "+v"(x2), "+v"(la));
      if constexpr (K == kDot2cF16) asm volatile("v_dot2c_f32_f16 %0, %1, %1" : "+v"(x2), "+v"(la));
      if constexpr (K == kTrRead2)
        asm volatile("ds_read_b64_tr_b16 %0, %2 offset:0\n\tds_read_b64_tr_b16 %1, %2 offset:1024\n\ts_waitcnt lgkmcnt(2)"
                     : "=v"(d0), "=v"(d1), "+v"(la));
      if constexpr (K == kDsWrite64x2)
        asm volatile("ds_write_b64 %0, %1 offset:2048\n\tds_write_b64 %0, %2 offset:4096" : "+v"(la), "+v"(d0), "+v"(d1) :: "memory");
      if constexpr (K == kGlobalLds || K == kGlobalLdsAlone) __builtin_amdgcn_global_load_lds(gb + off, (lds_void*)(L + 1024 * w), 16, 0, 0);
      if constexpr (K == kBufferLds || K == kBufferLdsAlone)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void*)(L + 1024 * w), 16, off, 0, 0, 0);
#undef V4
    }
    if constexpr (K >= kGlobalLds) asm volatile("s_waitcnt vmcnt(32)" ::: "memory");
  }
  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_memtime %0\n\ts_waitcnt lgkmcnt(0)" : "=s"(t1)::"memory");
  float sink = x0 + x1 + x2 + x3 + x4 + x5 + (float)(d0[0] + d0[1] + d1[0] + d1[1]);
#pragma unroll
  for (int k = 0; k < 16; ++k) sink += acc0[k] + acc1[k];
  if (lane == 0) out[w] = (t1 - t0) | (sink == 12345.f ? 1ull << 63 : 0);
}

typedef void (*Kernel)(unsigned long long*, const char*);
template <int K>
void fill(Kernel* ks) {
  ks[K] = probe<K>;
  if constexpr (K + 1 < kNumVariants) fill<K + 1>(ks);
}

int main() {
  Kernel ks[kNumVariants];
  fill<0>(ks);
  unsigned long long* d = nullptr;
  char* g = nullptr;
  if (hipMalloc(&d, 4 * sizeof(unsigned long long)) != hipSuccess) return 1;
  if (hipMalloc(&g, kGlobalBytes) != hipSuccess) return 1;
  if (hipMemset(g, 0, kGlobalBytes) != hipSuccess) return 1;
  printf("| Per step: one 32x32x16 bf16 MFMA ... | 1 wave: cycles per step | 4 waves (one per SIMD) |\n|---|---|---|\n");
  for (int v = 0; v < kNumVariants; ++v) {
    double c[2];
    for (int wv = 0; wv < 2; ++wv) {
      const int threads = wv ? 256 : 64;
      for (int rep = 0; rep < 2; ++rep) {
        hipLaunchKernelGGL(ks[v], dim3(1), dim3(threads), 0, 0, d, g);
        if (hipDeviceSynchronize() != hipSuccess) { printf("launch failed\n"); return 1; }
      }
      unsigned long long h[4] = {};
      if (hipMemcpy(h, d, sizeof(h[0]) * (threads / 64), hipMemcpyDeviceToHost) != hipSuccess) return 1;
      c[wv] = (double)(h[0] & ~(1ull << 63)) / (kIters * 8.0);
    }
    printf("| %s | %.1f | %.1f |\n", kNames[v], c[0], c[1]);
  }
  return 0;
}
