// A C++ caller of the drop-in headers written the way the reference's own
// C++ test is (reference tests/test_correctness.cu): inputs from srand(42) /
// rand() uniform in [-scale, scale) (kv 0.05, W_UK / W_UV 0.02, q 0.1;
// :15-23, :111-115), RoPE tables from cosf / sinf of pos / 10000^(2i/dR)
// (:118-124), the absorbed query built on the host (:29-46), then a
// FusedMLAParams filled field by field and launch_fused_mla (:182-199), over
// the reference's matrix: DeepSeek-V2 at kv_len 512 / 2048 / 8192, 16 heads at
// 512 / 2048, 64 heads at 512 / 2048 (:238-257). Also one
// launch_batched_fused_mla over a shared cache and a LatentKVCache filled with
// append_host.
//
// Usage: reference_caller <out_dir>. Writes each case's inputs and output as
// raw little-endian arrays (<tag>_<name>.bin) for the Python test
// (tests/test_gpu_cpp_caller.py), which checks them against the float64
// oracle. Exit status 0 when every launch succeeded and the cache rows read
// back exactly.
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "fused_mla.cuh"
#include "fused_mla_batched.cuh"
#include "mla_config.cuh"

#define HIP_CHECK(x)                                                                     \
  do {                                                                                   \
    hipError_t e_ = (x);                                                                 \
    if (e_ != hipSuccess) {                                                              \
      std::fprintf(stderr, "%s:%d %s: %s\n", __FILE__, __LINE__, #x, hipGetErrorString(e_)); \
      std::exit(1);                                                                      \
    }                                                                                    \
  } while (0)

static std::string g_dir;

static void fill_random_fp16(__half* dst, int n, float scale) {
  for (int i = 0; i < n; ++i) dst[i] = __float2half((float(rand()) / RAND_MAX - 0.5f) * 2.0f * scale);
}

static void fill_random_fp32(float* dst, int n, float scale) {
  for (int i = 0; i < n; ++i) dst[i] = (float(rand()) / RAND_MAX - 0.5f) * 2.0f * scale;
}

static void dump(const std::string& tag, const char* name, const void* p, size_t bytes) {
  const std::string path = g_dir + "/" + tag + "_" + name + ".bin";
  FILE* f = std::fopen(path.c_str(), "wb");
  if (!f || std::fwrite(p, 1, bytes, f) != bytes) {
    std::fprintf(stderr, "cannot write %s\n", path.c_str());
    std::exit(1);
  }
  std::fclose(f);
}

static void compute_q_absorbed_host(const float* q_nope, const __half* W_UK, float* q_absorbed, int nh, int dn,
                                    int dc) {
  for (int h = 0; h < nh; ++h)
    for (int c = 0; c < dc; ++c) {
      float acc = 0.0f;
      for (int i = 0; i < dn; ++i) acc += q_nope[h * dn + i] * __half2float(W_UK[(size_t)(h * dn + i) * dc + c]);
      q_absorbed[h * dc + c] = acc;
    }
}

static void rope_tables(int S, int dR, float* cs, float* sn) {
  for (int pos = 0; pos < S; ++pos)
    for (int i = 0; i < dR / 2; ++i) {
      const float theta = (float)pos / powf(10000.0f, 2.0f * i / dR);
      cs[pos * (dR / 2) + i] = cosf(theta);
      sn[pos * (dR / 2) + i] = sinf(theta);
    }
}

template <typename T>
static T* to_device(const std::vector<T>& h) {
  T* d = nullptr;
  HIP_CHECK(hipMalloc(&d, h.size() * sizeof(T)));
  HIP_CHECK(hipMemcpy(d, h.data(), h.size() * sizeof(T), hipMemcpyHostToDevice));
  return d;
}

// One single-token case, dumped under tag.
static void run_single(const MLAConfig& cfg, int S, const std::string& tag) {
  const int dc = cfg.kv_lora_rank, dR = cfg.qk_rope_head_dim, nh = cfg.num_heads, dn = cfg.qk_nope_head_dim,
            dv = cfg.v_head_dim, stride = dc + dR;
  std::vector<__half> kv((size_t)S * stride), W_UK((size_t)nh * dn * dc), W_UV((size_t)nh * dv * dc);
  std::vector<float> q_nope(nh * dn), q_rope(nh * dR), q_abs(nh * dc), cs(S * dR / 2), sn(S * dR / 2),
      out(nh * dv, 0.f);
  fill_random_fp16(kv.data(), (int)kv.size(), 0.05f);
  fill_random_fp16(W_UK.data(), (int)W_UK.size(), 0.02f);
  fill_random_fp16(W_UV.data(), (int)W_UV.size(), 0.02f);
  fill_random_fp32(q_nope.data(), (int)q_nope.size(), 0.1f);
  fill_random_fp32(q_rope.data(), (int)q_rope.size(), 0.1f);
  rope_tables(S, dR, cs.data(), sn.data());
  compute_q_absorbed_host(q_nope.data(), W_UK.data(), q_abs.data(), nh, dn, dc);

  __half* d_kv = to_device(kv);
  __half* d_W_UV = to_device(W_UV);
  float* d_q_absorbed = to_device(q_abs);
  float* d_q_rope = to_device(q_rope);
  float* d_rope_cos = to_device(cs);
  float* d_rope_sin = to_device(sn);
  float* d_out_fused = to_device(out);

  FusedMLAParams params;
  params.kv_cache = d_kv;
  params.seq_len = S;
  params.q_absorbed = d_q_absorbed;
  params.q_rope = d_q_rope;
  params.W_UV = d_W_UV;
  params.rope_cos = d_rope_cos;
  params.rope_sin = d_rope_sin;
  params.output = d_out_fused;
  params.cfg = &cfg;
  HIP_CHECK(launch_fused_mla(params));
  HIP_CHECK(hipDeviceSynchronize());
  HIP_CHECK(hipMemcpy(out.data(), d_out_fused, out.size() * sizeof(float), hipMemcpyDeviceToHost));

  dump(tag, "kv", kv.data(), kv.size() * 2);
  dump(tag, "wuk", W_UK.data(), W_UK.size() * 2);
  dump(tag, "wuv", W_UV.data(), W_UV.size() * 2);
  dump(tag, "qn", q_nope.data(), q_nope.size() * 4);
  dump(tag, "qr", q_rope.data(), q_rope.size() * 4);
  dump(tag, "qa", q_abs.data(), q_abs.size() * 4);
  dump(tag, "cos", cs.data(), cs.size() * 4);
  dump(tag, "sin", sn.data(), sn.size() * 4);
  dump(tag, "out", out.data(), out.size() * 4);
  for (void* p : {(void*)d_kv, (void*)d_W_UV, (void*)d_q_absorbed, (void*)d_q_rope, (void*)d_rope_cos,
                  (void*)d_rope_sin, (void*)d_out_fused})
    HIP_CHECK(hipFree(p));
  std::printf("%s: launch_fused_mla nh=%d S=%d ok\n", tag.c_str(), nh, S);
}

// B tokens over one shared cache through launch_batched_fused_mla.
static void run_batched(const MLAConfig& cfg, int S, int B, const std::string& tag) {
  const int dc = cfg.kv_lora_rank, dR = cfg.qk_rope_head_dim, nh = cfg.num_heads, dv = cfg.v_head_dim;
  std::vector<__half> kv((size_t)S * (dc + dR)), W_UV((size_t)nh * dv * dc);
  std::vector<float> q_abs((size_t)B * nh * dc), q_rope((size_t)B * nh * dR), cs(S * dR / 2), sn(S * dR / 2),
      out((size_t)B * nh * dv, 0.f);
  fill_random_fp16(kv.data(), (int)kv.size(), 0.05f);
  fill_random_fp16(W_UV.data(), (int)W_UV.size(), 0.02f);
  fill_random_fp32(q_abs.data(), (int)q_abs.size(), 0.1f);
  fill_random_fp32(q_rope.data(), (int)q_rope.size(), 0.1f);
  rope_tables(S, dR, cs.data(), sn.data());
  __half* d_kv = to_device(kv);
  __half* d_W_UV = to_device(W_UV);
  float* d_qa = to_device(q_abs);
  float* d_qr = to_device(q_rope);
  float* d_cos = to_device(cs);
  float* d_sin = to_device(sn);
  float* d_out = to_device(out);
  BatchedFusedMLAParams p;
  p.kv_cache = d_kv;
  p.seq_len = S;
  p.batch_size = B;
  p.q_absorbed = d_qa;
  p.q_rope = d_qr;
  p.W_UV = d_W_UV;
  p.rope_cos = d_cos;
  p.rope_sin = d_sin;
  p.output = d_out;
  p.cfg = &cfg;
  // with a caller workspace this time, sized for the fp16 / fp16 pair
  const size_t ws_bytes = fused_mla_workspace_size(S, B, cfg);
  HIP_CHECK(hipMalloc(&p.workspace, ws_bytes));
  p.workspace_bytes = ws_bytes;
  HIP_CHECK(launch_batched_fused_mla(p));
  HIP_CHECK(hipDeviceSynchronize());
  HIP_CHECK(hipMemcpy(out.data(), d_out, out.size() * sizeof(float), hipMemcpyDeviceToHost));
  dump(tag, "kv", kv.data(), kv.size() * 2);
  dump(tag, "wuv", W_UV.data(), W_UV.size() * 2);
  dump(tag, "qa", q_abs.data(), q_abs.size() * 4);
  dump(tag, "qr", q_rope.data(), q_rope.size() * 4);
  dump(tag, "cos", cs.data(), cs.size() * 4);
  dump(tag, "sin", sn.data(), sn.size() * 4);
  dump(tag, "out", out.data(), out.size() * 4);
  for (void* q : {(void*)d_kv, (void*)d_W_UV, (void*)d_qa, (void*)d_qr, (void*)d_cos, (void*)d_sin, (void*)d_out,
                  p.workspace})
    HIP_CHECK(hipFree(q));
  std::printf("%s: launch_batched_fused_mla B=%d S=%d ok\n", tag.c_str(), B, S);
}

// LatentKVCache: append_host row by row, read back, compare bit for bit;
// one append past max_seq_len must throw "KV cache full".
static bool run_cache(const MLAConfig& cfg) {
  const int max_len = 48, n = 40, stride = cfg.kv_lora_rank + cfg.qk_rope_head_dim;
  __half* d = nullptr;
  HIP_CHECK(hipMalloc(&d, (size_t)max_len * stride * sizeof(__half)));
  HIP_CHECK(hipMemset(d, 0, (size_t)max_len * stride * sizeof(__half)));
  LatentKVCache cache(d, max_len, cfg);
  std::vector<__half> rows((size_t)max_len * stride);
  fill_random_fp16(rows.data(), (int)rows.size(), 0.05f);
  for (int i = 0; i < n; ++i)
    cache.append_host(rows.data() + (size_t)i * stride, rows.data() + (size_t)i * stride + cfg.kv_lora_rank, cfg);
  std::vector<__half> back((size_t)max_len * stride);
  HIP_CHECK(hipMemcpy(back.data(), d, back.size() * sizeof(__half), hipMemcpyDeviceToHost));
  bool ok = cache.current_len == n && std::memcmp(back.data(), rows.data(), (size_t)n * stride * 2) == 0;
  for (size_t i = (size_t)n * stride; i < back.size(); ++i) ok = ok && __half2float(back[i]) == 0.f;
  for (int i = n; i < max_len; ++i)
    cache.append_host(rows.data() + (size_t)i * stride, rows.data() + (size_t)i * stride + cfg.kv_lora_rank, cfg);
  bool threw = false;
  try {
    cache.append_host(rows.data(), rows.data() + cfg.kv_lora_rank, cfg);
  } catch (const std::runtime_error& e) {
    threw = std::string(e.what()) == "KV cache full";
  }
  ok = ok && threw && cache.current_len == max_len && cache.row(3) == d + 3 * stride;
  HIP_CHECK(hipFree(d));
  std::printf("LatentKVCache append_host: %s\n", ok ? "ok" : "MISMATCH");
  return ok;
}

int main(int argc, char** argv) {
  if (argc != 2) {
    std::fprintf(stderr, "usage: %s <out_dir>\n", argv[0]);
    return 2;
  }
  g_dir = argv[1];
  srand(42);
  MLAConfig cfg_v2 = MLAConfig::deepseek_v2();
  cfg_v2.validate();
  for (int kv_len : {512, 2048, 8192}) run_single(cfg_v2, kv_len, "v2_" + std::to_string(kv_len));
  MLAConfig cfg_small = cfg_v2;
  cfg_small.num_heads = 16;
  for (int kv_len : {512, 2048}) run_single(cfg_small, kv_len, "h16_" + std::to_string(kv_len));
  cfg_small.num_heads = 64;
  for (int kv_len : {512, 2048}) run_single(cfg_small, kv_len, "h64_" + std::to_string(kv_len));
  run_batched(cfg_v2, 1024, 4, "batched");
  return run_cache(cfg_v2) ? 0 : 1;
}
