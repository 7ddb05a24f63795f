// extern "C" entry points of liblatent_attn_hip.so (declared in
// include/latent_attn.h): argument checking, split-KV planning, workspace
// carving and kernel dispatch. Host code only; the kernels live in
// la_generic.hip and la_mfma.hip.
#include "la_internal.hpp"

#include <algorithm>
#include <cmath>
#include <mutex>
#include <vector>

namespace la {
namespace {

thread_local int g_last_hip_error = 0;

int record_hip(hipError_t e) {
  g_last_hip_error = (int)e;
  return LA_ERROR_HIP;
}

bool valid_dtype(int d) { return d == LA_DTYPE_F32 || d == LA_DTYPE_F16 || d == LA_DTYPE_BF16; }
// latent caches may also be FP8 E4M3 (weights may not)
bool valid_cache_dtype(int d) { return valid_dtype(d) || d == LA_DTYPE_FP8_E4M3; }

// Same conditions as MLAConfig::validate (src/mla_config.cuh:35-40) plus the
// rotate-half requirement of an even rope dimension.
bool valid_cfg(const la_mla_config* c) {
  if (!c) return false;
  if (c->kv_lora_rank <= 0 || c->qk_nope_head_dim <= 0 || c->qk_rope_head_dim <= 0) return false;
  if (c->num_heads <= 0 || c->v_head_dim <= 0) return false;
  return (c->qk_rope_head_dim % 2) == 0;
}

int cu_count() {
  static std::mutex mu;
  static std::vector<int> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  std::lock_guard<std::mutex> lock(mu);
  if ((int)cache.size() <= dev) cache.resize(dev + 1, 0);
  if (cache[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cache[dev] = n;
  }
  return cache[dev];
}

constexpr size_t kAlign = 256;
size_t align_up(size_t x) { return (x + kAlign - 1) / kAlign * kAlign; }

enum Variant { kAuto = 0, kGeneric = 1, kMfma = 2 };

struct Plan {
  bool mfma = false;
  int chunk_len = 0;
  int num_chunks = 0;
  int num_slots = 0;
  bool proj_mfma = false;
  size_t part_scale_off = 0;
  bool absorb_mfma = false;  // q_nope . W_UK on the MFMA kernel
  bool absorb_prep = false;  // ... writing the attention kernel's 16-bit Q rows directly
  size_t q_abs_off = 0, q_prep_off = 0, part_o_off = 0, part_lse_off = 0, total = 0;
};

// Fills the problem (without workspace pointers) and the plan. The args'
// chunk_rows / kernel_variant fields are tuning overrides (0 = automatic).
int prepare(const la_decode_args* a, DecodeProblem* p, Plan* plan) {
  if (!a || !valid_cfg(&a->cfg)) return LA_ERROR_INVALID_VALUE;
  const int chunk_rows = a->chunk_rows;
  const int variant = a->kernel_variant;
  if (chunk_rows < 0 || variant < kAuto || variant > kMfma || a->rope_rows < 0) return LA_ERROR_INVALID_VALUE;
  if (a->num_seqs < 0 || a->queries_per_seq < 1 || a->total_rows < 0) return LA_ERROR_INVALID_VALUE;
  if (!valid_cache_dtype(a->kv_dtype) || !valid_dtype(a->w_uv_dtype)) return LA_ERROR_INVALID_VALUE;
  const bool paged = a->block_table != nullptr;
  if (paged) {
    // pool of total_rows rows in blocks; sequences are virtual regions of
    // blocks_per_seq blocks whose filled length comes from seq_lens
    if (a->block_size <= 0 || a->blocks_per_seq <= 0 || a->seq_offsets || !a->seq_lens ||
        a->total_rows % a->block_size != 0 || (int64_t)a->blocks_per_seq * a->block_size > INT32_MAX ||
        a->total_rows > (int64_t)UINT32_MAX ||  // pool rows are 32-bit in the MFMA kernel
        (a->num_seqs > 0 && a->total_rows < a->block_size))  // a pool without a block: nothing to clamp into
      return LA_ERROR_INVALID_VALUE;
  } else if (!a->seq_offsets && (a->seq_len < 0 || (int64_t)a->num_seqs * a->seq_len > a->total_rows)) {
    return LA_ERROR_INVALID_VALUE;
  }
  const bool absorb = a->q_nope != nullptr;
  if (absorb == (a->q_absorbed != nullptr)) return LA_ERROR_INVALID_VALUE;
  if (absorb && (!a->W_UK || !valid_dtype(a->w_uk_dtype))) return LA_ERROR_INVALID_VALUE;
  const la_mla_config& c = a->cfg;

  *p = DecodeProblem{};
  p->kv = a->kv_cache;
  p->kv_dtype = a->kv_dtype;
  p->row_elems = c.kv_lora_rank + c.qk_rope_head_dim;
  p->total_rows = a->total_rows;
  p->num_seqs = a->num_seqs;
  p->seq_len = a->seq_offsets ? 0 : a->seq_len;
  p->offsets = a->seq_offsets;
  p->lens = a->seq_lens;
  if (paged) {
    p->block_table = a->block_table;
    p->block_size = a->block_size;
    p->blocks_per_seq = a->blocks_per_seq;
    p->pool_blocks = a->total_rows / a->block_size;
    p->pool_last = (int)std::min<int64_t>(std::max<int64_t>(p->pool_blocks - 1, 0), INT32_MAX);
    set_tile_divisor(*p, (uint32_t)std::max(a->block_size / 32, 1));
    p->seq_len = a->blocks_per_seq * a->block_size;       // virtual region per sequence
    p->total_rows = (int64_t)a->num_seqs * p->seq_len;    // the virtual row space the plan covers
  }
  p->qps = a->queries_per_seq;
  p->nh = c.num_heads;
  p->Hq = a->queries_per_seq * c.num_heads;
  p->q_abs = a->q_absorbed;
  p->q_rope = a->q_rope;
  p->W_UV = a->W_UV;
  p->wuv_dtype = a->w_uv_dtype;
  p->rope_cos = a->rope_cos;
  p->rope_sin = a->rope_sin;
  p->rope_rows = a->rope_rows;
  p->out = a->output;
  p->dc = c.kv_lora_rank;
  p->dR = c.qk_rope_head_dim;
  p->dv = c.v_head_dim;
  p->scale_log2 = (float)(kLog2e / std::sqrt((double)(c.qk_nope_head_dim + c.qk_rope_head_dim)));

  if (a->num_seqs == 0) {
    *plan = Plan{};
    return LA_SUCCESS;
  }
  if (!a->q_rope || !a->W_UV || !a->rope_cos || !a->rope_sin || !a->output) return LA_ERROR_INVALID_VALUE;
  if (a->total_rows > 0 && !a->kv_cache) return LA_ERROR_INVALID_VALUE;

  Plan pl;
  // An FP8 E4M3 cache runs on the MFMA kernel too (its tiles are expanded to
  // bf16 in LDS); the VALU kernel (kernel_variant 1) reads it as well.
  const bool mfma_ok = mfma_supported(*p);
  if (variant == kMfma && !mfma_ok) return LA_ERROR_NOT_SUPPORTED;
  if (variant == kGeneric || !mfma_ok) {
    if (!generic_supported(*p)) return LA_ERROR_NOT_SUPPORTED;
    pl.mfma = false;
  } else {
    pl.mfma = true;
  }

  const int64_t total = paged ? p->total_rows : a->seq_offsets ? a->total_rows : (int64_t)a->num_seqs * a->seq_len;
  const int ncu = cu_count();
  int64_t L;
  if (chunk_rows > 0) {
    L = chunk_rows;
  } else {
    int64_t groups = pl.mfma ? (p->Hq + mfma_heads_per_group() - 1) / mfma_heads_per_group() : p->Hq;
    int64_t target_blocks = pl.mfma ? ncu : 4LL * ncu;
    int64_t chunks = std::max<int64_t>(1, target_blocks / std::max<int64_t>(1, groups));
    L = (total + chunks - 1) / chunks;
    // MFMA path: each workgroup (one chunk, one group of up to 128 query
    // heads) writes a partial row of dc fp16 values per head; keep them
    // below the bytes the workgroup streams from a 16-bit cache (rows of
    // dc + dR), so short batches (B = 1) do not trade a cheaper attention
    // launch for a merge that reads more than the cache: 128 heads need at
    // least 114 rows (128 after rounding). The floor counts rows, so for an
    // FP8 cache (rows of half the bytes) the partials may reach twice the
    // cache bytes. Head groups share a chunk's rows (several queries over
    // one cache), each writing its own partials, so the floor is per group.
    if (pl.mfma) {
      const int64_t hg = std::min<int64_t>(p->Hq, mfma_heads_per_group());
      L = std::max<int64_t>(L, (hg * c.kv_lora_rank + c.kv_lora_rank + c.qk_rope_head_dim - 1) /
                                   (c.kv_lora_rank + c.qk_rope_head_dim));
    }
    L = (L + 63) / 64 * 64;
    L = std::max<int64_t>(L, 64);
  }
  if (L > (int64_t)1 << 30) L = (int64_t)1 << 30;
  if (pl.mfma && L > mfma_max_chunk_rows()) L = mfma_max_chunk_rows();
  if (paged && pl.mfma) L = (L + 63) / 64 * 64;  // MFMA tiles start block-aligned
  const int64_t nchunks = total > 0 ? (total + L - 1) / L : 0;
  if (nchunks > (int64_t)1 << 30) return LA_ERROR_INVALID_VALUE;
  pl.chunk_len = (int)L;
  pl.num_chunks = (int)nchunks;
  pl.num_slots = nchunks > 0 ? (int)(nchunks + a->num_seqs - 1) : 0;

  const int64_t tokens = (int64_t)a->num_seqs * a->queries_per_seq;
  pl.absorb_mfma = absorb && absorb_mfma_supported(a->w_uk_dtype, c.num_heads, c.qk_nope_head_dim, c.kv_lora_rank) &&
                   (reinterpret_cast<uintptr_t>(a->q_nope) & 15) == 0 &&
                   (reinterpret_cast<uintptr_t>(a->W_UK) & 15) == 0;
  pl.absorb_prep = pl.mfma && pl.absorb_mfma;
  size_t off = 0;
  if (absorb && !pl.absorb_prep) {
    pl.q_abs_off = off;
    off += align_up((size_t)tokens * c.num_heads * c.kv_lora_rank * sizeof(float));
  }
  if (pl.mfma) {
    pl.q_prep_off = off;
    off += align_up((size_t)a->num_seqs * qprep_rows_per_seq(p->Hq) * kQPrepRow * 2);
  }
  // the MFMA kernel writes its partial rows as scaled fp16, the VALU kernel as fp32
  p->part_f16 = pl.mfma ? 1 : 0;
  pl.part_o_off = off;
  off += align_up((size_t)pl.num_slots * p->Hq * c.kv_lora_rank * (pl.mfma ? 2 : 4));
  if (pl.mfma) {
    pl.part_scale_off = off;  // two per row (column halves), then part_m: one per row
    off += align_up((size_t)pl.num_slots * p->Hq * 3 * sizeof(float));
  }
  pl.part_lse_off = off;
  off += align_up((size_t)pl.num_slots * p->Hq * sizeof(float));
  pl.proj_mfma = project_mfma_supported(*p);
  pl.total = off;

  p->chunk_len = pl.chunk_len;
  p->num_chunks = pl.num_chunks;
  p->num_slots = pl.num_slots;
  *plan = pl;
  return LA_SUCCESS;
}

// The latent-half merge: few query rows leave most CUs idle in the full-row
// merge, so it is split over the two latent halves, which add into the
// output (zeroed first by the kernel that writes the attention kernel's
// 16-bit queries: the absorb kernel, or prep_q when the queries come
// absorbed and there is at least one chunk).
bool merge_halves(const DecodeProblem& p, const Plan& plan) {
  return plan.proj_mfma && plan.mfma && (plan.absorb_prep || plan.num_chunks > 0) &&
         merge_project_blocks(p) < cu_count();
}

// ev_b / ev_e (optional) are recorded around the attention kernel, which runs
// max(repeat, 1) times between them.
int run(const la_decode_args* a, hipStream_t stream, hipEvent_t ev_b = nullptr, hipEvent_t ev_e = nullptr,
        int repeat = 1) {
  if (repeat < 0) return LA_ERROR_INVALID_VALUE;
  DecodeProblem p;
  Plan plan;
  int st = prepare(a, &p, &plan);
  if (st != LA_SUCCESS) return st;
  if (a->num_seqs == 0) return LA_SUCCESS;

  char* ws = static_cast<char*>(a->workspace);
  bool owned = false;
  if (plan.total > 0) {
    if (ws) {
      if (a->workspace_bytes < plan.total) return LA_ERROR_WORKSPACE;
    } else {
      void* m = nullptr;
      hipError_t e = hipMallocAsync(&m, plan.total, stream);
      if (e != hipSuccess) return record_hip(e);
      ws = static_cast<char*>(m);
      owned = true;
    }
  }
  auto finish = [&](hipError_t e) -> int {
    if (owned) {
      hipError_t f = hipFreeAsync(ws, stream);
      if (e == hipSuccess) e = f;
    }
    return e == hipSuccess ? (int)LA_SUCCESS : record_hip(e);
  };

  const la_mla_config& c = a->cfg;
  const int64_t tokens = (int64_t)a->num_seqs * a->queries_per_seq;
  if (plan.mfma) p.q_prep = ws + plan.q_prep_off;
  // Few query rows leave most CUs idle in the full-row merge: split it over
  // the two latent halves, which add into the output. The kernel that writes
  // the attention kernel's 16-bit queries (the absorb kernel, or prep_q when
  // the queries come absorbed) runs first and zeroes the output.
  const bool merge_halves = la::merge_halves(p, plan);
  float* const zero_out = merge_halves ? a->output : nullptr;
  const int64_t zero_n = merge_halves ? tokens * c.num_heads * c.v_head_dim : 0;
  if (a->q_nope) {
    hipError_t e = hipSuccess;
    if (plan.absorb_prep) {
      // absorbed, scaled 16-bit Q rows for the attention kernel in one pass
      // q_prep in the MFMAs' 16-bit type: fp16 for an fp16 cache, bf16 otherwise
      e = launch_absorb_mfma(a->q_nope, a->W_UK, a->w_uk_dtype, p.q_prep, p.kv_dtype == LA_DTYPE_F16 ? 2 : 1,
                             a->q_rope, p.scale_log2, c.qk_rope_head_dim, (int)tokens, c.num_heads,
                             c.qk_nope_head_dim, c.kv_lora_rank, a->queries_per_seq, stream, zero_out, zero_n);
    } else {
      float* qa = reinterpret_cast<float*>(ws + plan.q_abs_off);
      e = plan.absorb_mfma ? launch_absorb_mfma(a->q_nope, a->W_UK, a->w_uk_dtype, qa, 0, nullptr, 1.f, 0,
                                                (int)tokens, c.num_heads, c.qk_nope_head_dim, c.kv_lora_rank, 1,
                                                stream)
                           : launch_absorb(a->q_nope, a->W_UK, a->w_uk_dtype, qa, (int)tokens, c.num_heads,
                                           c.qk_nope_head_dim, c.kv_lora_rank, stream);
      p.q_abs = qa;
    }
    if (e != hipSuccess) return finish(e);
  }
  p.part_o = reinterpret_cast<float*>(ws + plan.part_o_off);
  p.part_lse = reinterpret_cast<float*>(ws + plan.part_lse_off);
  p.part_scale = plan.mfma ? reinterpret_cast<float*>(ws + plan.part_scale_off) : nullptr;
  p.part_m = plan.mfma ? p.part_scale + (size_t)plan.num_slots * p.Hq * 2 : nullptr;
  if (plan.num_chunks > 0) {
    if (plan.mfma && !plan.absorb_prep) {
      hipError_t e = launch_prep_q(p, stream, zero_out, zero_n);
      if (e != hipSuccess) return finish(e);
    }
    // the optional events bracket the attention kernel alone
    hipError_t e = hipSuccess;
    const int reps = repeat > 1 ? repeat : 1;
    if (plan.mfma && reps == 1) {
      e = launch_decode_mfma(p, stream, ev_b, ev_e);  // recorded by the launch itself
    } else {
      if (ev_b) e = hipEventRecord(ev_b, stream);
      for (int r = 0; r < reps && e == hipSuccess; ++r)
        e = plan.mfma ? launch_decode_mfma(p, stream, nullptr, nullptr) : launch_decode_generic(p, stream);
      if (e == hipSuccess && ev_e) e = hipEventRecord(ev_e, stream);
    }
    if (e != hipSuccess) return finish(e);
  }
  return finish(plan.proj_mfma ? launch_combine_project_mfma(p, stream, merge_halves)
                                : launch_combine_project(p, stream));
}

la_decode_args shared_cache_args(const void* kv_cache, int kv_dtype, int seq_len, int batch, const float* q_absorbed,
                                 const float* q_rope, const void* W_UV, int w_uv_dtype, const float* rope_cos,
                                 const float* rope_sin, float* output, const la_mla_config* cfg, void* workspace,
                                 size_t workspace_bytes) {
  la_decode_args a{};
  a.rope_rows = seq_len;
  a.kv_cache = kv_cache;
  a.kv_dtype = kv_dtype;
  a.total_rows = seq_len;
  a.num_seqs = 1;
  a.seq_len = seq_len;
  a.seq_offsets = nullptr;
  a.queries_per_seq = batch;
  a.q_absorbed = q_absorbed;
  a.q_rope = q_rope;
  a.W_UV = W_UV;
  a.w_uv_dtype = w_uv_dtype;
  a.rope_cos = rope_cos;
  a.rope_sin = rope_sin;
  a.output = output;
  if (cfg) a.cfg = *cfg;
  a.workspace = workspace;
  a.workspace_bytes = workspace_bytes;
  return a;
}

// Scratch of la_mla_decode_noalloc: one array per GPU, in the code object,
// held until the process ends. Host code never uses the array's name as an
// address (on the host it is only a stand-in for the device symbol): the
// device address comes from hipGetSymbolAddress, once per device, with that
// device current, and is kept per device.
constexpr size_t kNoAllocScratchBytes = (size_t)64 << 20;
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

}  // namespace

static __device__ __align__(256) char scratch[kNoAllocScratchBytes];

namespace {

// The current device's scratch address (looked up on its first use there).
int scratch_ptr(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return record_hip(e);
  if (dev < 0 || dev >= kMaxDevices) return LA_ERROR_NOT_SUPPORTED;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return record_hip(e);
    if (!ptr) return LA_ERROR_HIP;
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return LA_SUCCESS;
}

}  // namespace
}  // namespace la

extern "C" {

const char* la_status_string(int status) {
  switch (status) {
    case LA_SUCCESS: return "success";
    case LA_ERROR_INVALID_VALUE: return "invalid value";
    case LA_ERROR_NOT_SUPPORTED: return "not supported";
    case LA_ERROR_WORKSPACE: return "workspace too small";
    case LA_ERROR_HIP: return "HIP runtime error";
    default: return "unknown status";
  }
}

int la_last_hip_error(void) { return la::g_last_hip_error; }

int la_abi_version(void) { return LA_ABI_VERSION; }

size_t la_mla_decode_workspace_size(const la_decode_args* args) {
  la::DecodeProblem p;
  la::Plan plan;
  if (la::prepare(args, &p, &plan) != LA_SUCCESS) return 0;
  return plan.total;
}

int la_mla_decode_plan(const la_decode_args* args, la_plan_info* info) {
  if (!info) return LA_ERROR_INVALID_VALUE;
  la::DecodeProblem p;
  la::Plan plan;
  const int st = la::prepare(args, &p, &plan);
  if (st != LA_SUCCESS) return st;
  *info = la_plan_info{};
  info->workspace_bytes = plan.total;
  if (args->num_seqs == 0) return LA_SUCCESS;
  info->attention = plan.mfma ? LA_PLAN_ATTENTION_MFMA : LA_PLAN_ATTENTION_VALU;
  info->chunk_rows = plan.chunk_len;
  info->num_chunks = plan.num_chunks;
  info->num_slots = plan.num_slots;
  info->head_groups = plan.mfma ? (p.Hq + la::mfma_heads_per_group() - 1) / la::mfma_heads_per_group() : p.Hq;
  if (!plan.proj_mfma) info->merge = LA_PLAN_MERGE_VALU;
  else info->merge = la::merge_halves(p, plan) ? LA_PLAN_MERGE_MFMA_HALVES : LA_PLAN_MERGE_MFMA;
  if (!args->q_nope) info->absorb = LA_PLAN_ABSORB_NONE;
  else if (plan.absorb_prep) info->absorb = LA_PLAN_ABSORB_MFMA_QPREP;
  else info->absorb = plan.absorb_mfma ? LA_PLAN_ABSORB_MFMA : LA_PLAN_ABSORB_VALU;
  return LA_SUCCESS;
}

int la_mla_decode(const la_decode_args* args, void* stream) { return la::run(args, static_cast<hipStream_t>(stream)); }

int la_mla_decode_profiled(const la_decode_args* args, void* stream, void* event_begin, void* event_end,
                           int32_t repeat) {
  return la::run(args, static_cast<hipStream_t>(stream), static_cast<hipEvent_t>(event_begin),
                 static_cast<hipEvent_t>(event_end), repeat);
}

int la_stream_ceiling(const la_decode_args* args, int32_t ring, void* stream, void* event_begin, void* event_end,
                      int32_t repeat) {
  if (ring != 3 && ring != 4 || repeat < 0) return LA_ERROR_INVALID_VALUE;
  la::DecodeProblem p;
  la::Plan plan;
  const int st = la::prepare(args, &p, &plan);
  if (st != LA_SUCCESS) return st;
  if (!plan.mfma || p.block_table || (p.kv_dtype != LA_DTYPE_BF16 && p.kv_dtype != LA_DTYPE_F16))
    return LA_ERROR_NOT_SUPPORTED;
  if (plan.num_chunks == 0) return LA_SUCCESS;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t e = hipSuccess;
  if (event_begin) e = hipEventRecord(static_cast<hipEvent_t>(event_begin), s);
  for (int r = 0; r < (repeat > 1 ? repeat : 1) && e == hipSuccess; ++r) e = la::launch_stream_copies(p, ring, s);
  if (e == hipSuccess && event_end) e = hipEventRecord(static_cast<hipEvent_t>(event_end), s);
  return e == hipSuccess ? (int)LA_SUCCESS : la::record_hip(e);
}

int la_mla_decode_noalloc(const la_decode_args* args, void* stream) {
  la::DecodeProblem p;
  la::Plan plan;
  const int st = la::prepare(args, &p, &plan);
  if (st != LA_SUCCESS) return st;
  if (plan.total > la::kNoAllocScratchBytes) return LA_ERROR_WORKSPACE;
  la_decode_args a = *args;
  a.workspace = nullptr;
  a.workspace_bytes = la::kNoAllocScratchBytes;
  if (plan.total > 0) {
    const int sp = la::scratch_ptr(&a.workspace);
    if (sp != LA_SUCCESS) return sp;
  }  // else: no workspace is needed and none is passed
  return la::run(&a, static_cast<hipStream_t>(stream));
}

size_t la_mla_decode_noalloc_max_bytes(void) { return la::kNoAllocScratchBytes; }

int la_fused_mla(const void* kv_cache, int kv_dtype, int seq_len, const float* q_absorbed, const float* q_rope,
                 const void* W_UV, int w_uv_dtype, const float* rope_cos, const float* rope_sin, float* output,
                 const la_mla_config* cfg, void* workspace, size_t workspace_bytes, void* stream) {
  if (!cfg || seq_len < 0 || !q_absorbed) return LA_ERROR_INVALID_VALUE;
  la_decode_args a = la::shared_cache_args(kv_cache, kv_dtype, seq_len, 1, q_absorbed, q_rope, W_UV, w_uv_dtype,
                                           rope_cos, rope_sin, output, cfg, workspace, workspace_bytes);
  return la::run(&a, static_cast<hipStream_t>(stream));
}

int la_batched_fused_mla(const void* kv_cache, int kv_dtype, int seq_len, int batch_size, const float* q_absorbed,
                         const float* q_rope, const void* W_UV, int w_uv_dtype, const float* rope_cos,
                         const float* rope_sin, float* output, const la_mla_config* cfg, void* workspace,
                         size_t workspace_bytes, void* stream) {
  if (!cfg || seq_len < 0 || batch_size <= 0 || !q_absorbed) return LA_ERROR_INVALID_VALUE;
  la_decode_args a = la::shared_cache_args(kv_cache, kv_dtype, seq_len, batch_size, q_absorbed, q_rope, W_UV,
                                           w_uv_dtype, rope_cos, rope_sin, output, cfg, workspace, workspace_bytes);
  return la::run(&a, static_cast<hipStream_t>(stream));
}

size_t la_fused_mla_workspace_size_dt(int seq_len, int batch_size, const la_mla_config* cfg, int kv_dtype,
                                      int w_uv_dtype) {
  if (!cfg || seq_len < 0 || batch_size <= 0) return 0;
  // Only plan-relevant fields are read. Which kernel family runs also depends
  // on pointer alignment, so return the larger of the two families' plans.
  alignas(256) static const char dummy[256] = {0};
  const float* d = reinterpret_cast<const float*>(dummy);
  size_t best = 0;
  for (int variant : {1, 2}) {
    la_decode_args a = la::shared_cache_args(dummy, kv_dtype, seq_len, batch_size, d, d, dummy, w_uv_dtype, d, d,
                                             const_cast<float*>(d), cfg, nullptr, 0);
    a.kernel_variant = variant;
    la::DecodeProblem p;
    la::Plan plan;
    if (la::prepare(&a, &p, &plan) == LA_SUCCESS && plan.total > best) best = plan.total;
  }
  return best;
}

size_t la_fused_mla_workspace_size(int seq_len, int batch_size, const la_mla_config* cfg) {
  // every cache dtype with every weight dtype
  size_t best = 0;
  for (int kv : {LA_DTYPE_F16, LA_DTYPE_BF16, LA_DTYPE_F32, LA_DTYPE_FP8_E4M3})
    for (int w : {LA_DTYPE_F16, LA_DTYPE_BF16, LA_DTYPE_F32})
      best = std::max(best, la_fused_mla_workspace_size_dt(seq_len, batch_size, cfg, kv, w));
  return best;
}

size_t la_naive_mla_workspace_size(int seq_len, const la_mla_config* cfg) {
  if (!la::valid_cfg(cfg) || seq_len < 0) return 0;
  return la::naive_workspace_bytes(seq_len, cfg->num_heads, cfg->qk_nope_head_dim, cfg->v_head_dim);
}

int la_naive_mla(const void* kv_cache, int kv_dtype, int seq_len, const void* W_UK, int w_uk_dtype, const void* W_UV,
                 int w_uv_dtype, const float* q_nope, const float* q_rope, const float* rope_cos,
                 const float* rope_sin, float* output, const la_mla_config* cfg, void* workspace,
                 size_t workspace_bytes, void* stream) {
  if (!la::valid_cfg(cfg) || seq_len < 0 || !la::valid_cache_dtype(kv_dtype) || !la::valid_dtype(w_uk_dtype) ||
      !la::valid_dtype(w_uv_dtype))
    return LA_ERROR_INVALID_VALUE;
  if (!W_UK || !W_UV || !q_nope || !q_rope || !rope_cos || !rope_sin || !output || (seq_len > 0 && !kv_cache))
    return LA_ERROR_INVALID_VALUE;
  const size_t need = la::naive_workspace_bytes(seq_len, cfg->num_heads, cfg->qk_nope_head_dim, cfg->v_head_dim);
  const hipStream_t st = static_cast<hipStream_t>(stream);
  la::NaiveProblem p{};
  p.kv = kv_cache;
  p.kv_dtype = kv_dtype;
  p.S = seq_len;
  p.W_UK = W_UK;
  p.wuk_dtype = w_uk_dtype;
  p.W_UV = W_UV;
  p.wuv_dtype = w_uv_dtype;
  p.q_nope = q_nope;
  p.q_rope = q_rope;
  p.rope_cos = rope_cos;
  p.rope_sin = rope_sin;
  p.rope_rows = seq_len;  // the reference indexes cos/sin by position < seq_len (src/fused_mla.cu:158-159)
  p.out = output;
  p.nh = cfg->num_heads;
  p.dn = cfg->qk_nope_head_dim;
  p.dR = cfg->qk_rope_head_dim;
  p.dc = cfg->kv_lora_rank;
  p.dv = cfg->v_head_dim;
  p.scale = (float)(1.0 / std::sqrt((double)(cfg->qk_nope_head_dim + cfg->qk_rope_head_dim)));
  void* ws = workspace;
  bool owned = false;
  if (ws) {
    if (workspace_bytes < need) return LA_ERROR_WORKSPACE;
  } else if (need > 0) {
    hipError_t e = hipMallocAsync(&ws, need, st);
    if (e != hipSuccess) return la::record_hip(e);
    owned = true;
  }
  hipError_t e = la::launch_naive(p, ws, st);
  if (owned) {
    hipError_t f = hipFreeAsync(ws, st);
    if (e == hipSuccess) e = f;
  }
  return e == hipSuccess ? (int)LA_SUCCESS : la::record_hip(e);
}

int la_append_kv(const la_append_args* a, void* stream) {
  if (!a || !la::valid_cfg(&a->cfg) || !la::valid_cache_dtype(a->kv_dtype) || !la::valid_cache_dtype(a->src_dtype))
    return LA_ERROR_INVALID_VALUE;
  if (a->num_seqs < 0 || a->tokens_per_seq < 0 || a->total_rows < 0 || a->rope_rows < 0) return LA_ERROR_INVALID_VALUE;
  const bool paged = a->block_table != nullptr;
  if (paged) {
    if (a->block_size <= 0 || a->blocks_per_seq <= 0 || a->seq_offsets || a->total_rows % a->block_size != 0 ||
        (a->num_seqs > 0 && a->total_rows < a->block_size))  // a pool without a block: nothing to clamp into
      return LA_ERROR_INVALID_VALUE;
  } else if (!a->seq_offsets && (a->seq_capacity < 0 || (int64_t)a->num_seqs * a->seq_capacity > a->total_rows)) {
    return LA_ERROR_INVALID_VALUE;
  }
  if (a->num_seqs == 0) return LA_SUCCESS;
  if (!a->seq_lens || (a->total_rows > 0 && !a->kv_cache)) return LA_ERROR_INVALID_VALUE;
  if (a->tokens_per_seq > 0 && (!a->c_t || !a->k_rope)) return LA_ERROR_INVALID_VALUE;
  // per-sequence element counts stay within the kernel's 32-bit indexing
  if ((int64_t)a->tokens_per_seq * (a->cfg.kv_lora_rank + a->cfg.qk_rope_head_dim) > INT32_MAX ||
      (a->q_rope && (int64_t)a->queries_per_seq * a->cfg.num_heads * a->cfg.qk_rope_head_dim > INT32_MAX))
    return LA_ERROR_INVALID_VALUE;
  // the vectorised query rotation reads 16-B chunks of q_rope and the tables
  if (a->q_rope && (a->cfg.qk_rope_head_dim / 2) % 4 == 0 &&
      ((reinterpret_cast<uintptr_t>(a->q_rope) | reinterpret_cast<uintptr_t>(a->rope_cos) |
        reinterpret_cast<uintptr_t>(a->rope_sin)) & 15))
    return LA_ERROR_INVALID_VALUE;
  if (a->q_rope && (a->queries_per_seq < 1 || a->queries_per_seq > a->tokens_per_seq || !a->rope_cos ||
                    !a->rope_sin || (int64_t)a->num_seqs * a->queries_per_seq * a->cfg.num_heads > INT32_MAX))
    return LA_ERROR_INVALID_VALUE;
  la::AppendProblem p{};
  p.kv = a->kv_cache;
  p.kv_dtype = a->kv_dtype;
  p.total_rows = a->total_rows;
  p.num_seqs = a->num_seqs;
  p.capacity = a->seq_offsets ? 0 : a->seq_capacity;
  p.offsets = a->seq_offsets;
  p.lens = a->seq_lens;
  p.tokens = a->tokens_per_seq;
  p.c_t = a->c_t;
  p.k_rope = a->k_rope;
  p.src_dtype = a->src_dtype;
  p.q_rope = a->q_rope;
  p.qps = a->q_rope ? a->queries_per_seq : 0;
  p.nh = a->cfg.num_heads;
  p.rope_cos = a->rope_cos;
  p.rope_sin = a->rope_sin;
  p.rope_rows = a->rope_rows;
  p.status = a->status;
  p.dc = a->cfg.kv_lora_rank;
  p.dR = a->cfg.qk_rope_head_dim;
  if (paged) {
    p.block_table = a->block_table;
    p.block_size = a->block_size;
    p.blocks_per_seq = a->blocks_per_seq;
    p.pool_blocks = a->total_rows / a->block_size;
  }
  const hipError_t e = la::launch_append(p, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? (int)LA_SUCCESS : la::record_hip(e);
}

int la_absorb_q(const float* q_nope, const void* W_UK, int w_uk_dtype, float* q_absorbed, int tokens,
                const la_mla_config* cfg, void* stream) {
  if (!la::valid_cfg(cfg) || tokens < 0 || !la::valid_dtype(w_uk_dtype)) return LA_ERROR_INVALID_VALUE;
  if (tokens == 0) return LA_SUCCESS;
  if (!q_nope || !W_UK || !q_absorbed) return LA_ERROR_INVALID_VALUE;
  const bool mfma = la::absorb_mfma_supported(w_uk_dtype, cfg->num_heads, cfg->qk_nope_head_dim, cfg->kv_lora_rank) &&
                    (reinterpret_cast<uintptr_t>(q_nope) & 15) == 0 && (reinterpret_cast<uintptr_t>(W_UK) & 15) == 0;
  hipError_t e = mfma ? la::launch_absorb_mfma(q_nope, W_UK, w_uk_dtype, q_absorbed, 0, nullptr, 1.f, 0, tokens,
                                               cfg->num_heads, cfg->qk_nope_head_dim, cfg->kv_lora_rank, 1,
                                               static_cast<hipStream_t>(stream))
                      : la::launch_absorb(q_nope, W_UK, w_uk_dtype, q_absorbed, tokens, cfg->num_heads,
                                          cfg->qk_nope_head_dim, cfg->kv_lora_rank, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? (int)LA_SUCCESS : la::record_hip(e);
}

}  // extern "C"
