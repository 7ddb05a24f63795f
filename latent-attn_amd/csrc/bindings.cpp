// latent_attn._C -- PyTorch-ROCm extension over the C ABI of
// liblatent_attn_hip.so (include/latent_attn.h).
//
// Mirrors the reference bindings (csrc/bindings.cpp:249-256 in the reference
// repo): same function names, argument order, shape checks and error
// messages, output allocated as float32 on kv_cache's device, launched on the
// current stream. Differences: the 16-bit dtype may be float16 (reference
// contract) or bfloat16, float32 caches/weights select the fp32 path, a
// device guard is taken, and two functions are added (mla_decode_forward,
// absorb_q_forward). No tensor math happens here; all compute is in the HIP
// library.
#include <torch/extension.h>
#include <c10/hip/HIPStream.h>

#include <stdexcept>
#include <string>

#include "latent_attn.h"

namespace {

// MLAConfig::validate (src/mla_config.cuh:35-40): std::invalid_argument.
la_mla_config config_from_args(int d_model, int kv_lora_rank, int qk_nope_head_dim, int qk_rope_head_dim,
                               int num_heads, int v_head_dim) {
  la_mla_config c{d_model, kv_lora_rank, qk_nope_head_dim, qk_rope_head_dim, num_heads, v_head_dim};
  if (kv_lora_rank <= 0 || qk_nope_head_dim <= 0 || qk_rope_head_dim <= 0)
    throw std::invalid_argument("MLA dims must be positive");
  if (num_heads <= 0 || v_head_dim <= 0) throw std::invalid_argument("num_heads and v_head_dim must be positive");
  if (qk_rope_head_dim % 2 != 0) throw std::invalid_argument("qk_rope_head_dim must be even (rotate-half RoPE)");
  return c;
}

int dtype_tag(const torch::Tensor& t) {
  switch (t.scalar_type()) {
    case torch::kFloat32: return LA_DTYPE_F32;
    case torch::kFloat16: return LA_DTYPE_F16;
    case torch::kBFloat16: return LA_DTYPE_BF16;
    case torch::kFloat8_e4m3fn: return LA_DTYPE_FP8_E4M3;
    default: return -1;
  }
}

// Caches (and the rows appended to them) may be FP8 E4M3 besides the 16- and
// 32-bit types; weights may not (check_weight).
void check_storage(const torch::Tensor& t, const char* name) {
  TORCH_CHECK(dtype_tag(t) >= 0, name, " must be float16, bfloat16, float32 or float8_e4m3fn, got ", t.dtype());
  TORCH_CHECK(t.is_contiguous(), name, " must be contiguous");
  TORCH_CHECK(t.is_cuda(), name, " must be on CUDA");
}

void check_weight(const torch::Tensor& t, const char* name) {
  TORCH_CHECK(dtype_tag(t) >= 0 && dtype_tag(t) != LA_DTYPE_FP8_E4M3, name,
              " must be float16, bfloat16 or float32, got ", t.dtype());
  TORCH_CHECK(t.is_contiguous(), name, " must be contiguous");
  TORCH_CHECK(t.is_cuda(), name, " must be on CUDA");
}

void check_fp32_contiguous(const torch::Tensor& t, const char* name) {
  TORCH_CHECK(t.dtype() == torch::kFloat32, name, " must be float32, got ", t.dtype());
  TORCH_CHECK(t.is_contiguous(), name, " must be contiguous");
  TORCH_CHECK(t.is_cuda(), name, " must be on CUDA");
}

void check_same_device(const torch::Tensor& ref, const torch::Tensor& t, const char* name) {
  TORCH_CHECK(t.device() == ref.device(), name, " must be on the same device as kv_cache");
}

void check_rope(const torch::Tensor& cos, const torch::Tensor& sin, int64_t rows, const la_mla_config& c) {
  TORCH_CHECK(cos.dim() == 2 && sin.dim() == 2, "rope_cos / rope_sin must be 2D (seq_len, qk_rope_head_dim/2)");
  TORCH_CHECK(cos.size(1) == c.qk_rope_head_dim / 2 && sin.size(1) == c.qk_rope_head_dim / 2,
              "rope_cos / rope_sin dim1 must be ", c.qk_rope_head_dim / 2);
  TORCH_CHECK(cos.size(0) >= rows && sin.size(0) >= rows, "rope_cos / rope_sin need at least ", rows, " rows");
}

void check_status(int st, const char* what) {
  if (st == LA_SUCCESS) return;
  std::string msg = std::string(what) + " failed: " + la_status_string(st);
  if (st == LA_ERROR_HIP) msg += std::string(" (") + hipGetErrorString((hipError_t)la_last_hip_error()) + ")";
  TORCH_CHECK(false, msg);
}

torch::Tensor workspace(const torch::Tensor& like, size_t bytes) {
  return torch::empty({(int64_t)std::max<size_t>(bytes, 1)}, like.options().dtype(torch::kUInt8));
}

void* current_stream() { return (void*)c10::hip::getCurrentHIPStream().stream(); }

}  // namespace

// fused_mla_forward -- reference csrc/bindings.cpp:126-176
//   kv_cache (seq_len, dc+dR); q_absorbed (nh, dc) f32; q_rope (nh, dR) f32;
//   W_UV (nh*dv, dc); rope tables (>= seq_len, dR/2) f32 -> (nh, dv) f32
torch::Tensor fused_mla_forward(torch::Tensor kv_cache, torch::Tensor q_absorbed, torch::Tensor q_rope,
                                torch::Tensor W_UV, torch::Tensor rope_cos, torch::Tensor rope_sin, int d_model,
                                int kv_lora_rank, int qk_nope_head_dim, int qk_rope_head_dim, int num_heads,
                                int v_head_dim) {
  check_storage(kv_cache, "kv_cache");
  check_fp32_contiguous(q_absorbed, "q_absorbed");
  check_fp32_contiguous(q_rope, "q_rope");
  check_weight(W_UV, "W_UV");
  check_fp32_contiguous(rope_cos, "rope_cos");
  check_fp32_contiguous(rope_sin, "rope_sin");
  la_mla_config cfg =
      config_from_args(d_model, kv_lora_rank, qk_nope_head_dim, qk_rope_head_dim, num_heads, v_head_dim);

  TORCH_CHECK(kv_cache.dim() == 2, "kv_cache must be 2D (seq_len, kv_lora_rank + qk_rope_head_dim)");
  const int64_t seq_len = kv_cache.size(0);
  TORCH_CHECK(kv_cache.size(1) == kv_lora_rank + qk_rope_head_dim, "kv_cache dim1 mismatch");
  TORCH_CHECK(q_absorbed.dim() == 2 && q_absorbed.size(0) == num_heads && q_absorbed.size(1) == kv_lora_rank,
              "q_absorbed shape mismatch");
  TORCH_CHECK(q_rope.dim() == 2 && q_rope.size(0) == num_heads && q_rope.size(1) == qk_rope_head_dim,
              "q_rope shape mismatch");
  TORCH_CHECK(W_UV.dim() == 2 && W_UV.size(0) == (int64_t)num_heads * v_head_dim && W_UV.size(1) == kv_lora_rank,
              "W_UV shape mismatch");
  check_rope(rope_cos, rope_sin, seq_len, cfg);
  for (auto* t : {&q_absorbed, &q_rope, &W_UV, &rope_cos, &rope_sin}) check_same_device(kv_cache, *t, "inputs");
  TORCH_CHECK(seq_len <= INT32_MAX, "seq_len too large");

  const at::DeviceGuard guard(kv_cache.device());
  auto output = torch::empty({num_heads, v_head_dim}, kv_cache.options().dtype(torch::kFloat32));
  const size_t ws_bytes = la_fused_mla_workspace_size_dt((int)seq_len, 1, &cfg, dtype_tag(kv_cache), dtype_tag(W_UV));
  auto ws = workspace(kv_cache, ws_bytes);
  int st = la_fused_mla(kv_cache.data_ptr(), dtype_tag(kv_cache), (int)seq_len, q_absorbed.data_ptr<float>(),
                        q_rope.data_ptr<float>(), W_UV.data_ptr(), dtype_tag(W_UV), rope_cos.data_ptr<float>(),
                        rope_sin.data_ptr<float>(), output.data_ptr<float>(), &cfg, ws.data_ptr(), ws_bytes,
                        current_stream());
  check_status(st, "launch_fused_mla");
  return output;
}

// batched_fused_mla_forward -- reference csrc/bindings.cpp:188-244
//   B query tokens over one shared cache -> (B, nh, dv) f32
torch::Tensor batched_fused_mla_forward(torch::Tensor kv_cache, torch::Tensor q_absorbed, torch::Tensor q_rope,
                                        torch::Tensor W_UV, torch::Tensor rope_cos, torch::Tensor rope_sin,
                                        int d_model, int kv_lora_rank, int qk_nope_head_dim, int qk_rope_head_dim,
                                        int num_heads, int v_head_dim) {
  check_storage(kv_cache, "kv_cache");
  check_fp32_contiguous(q_absorbed, "q_absorbed");
  check_fp32_contiguous(q_rope, "q_rope");
  check_weight(W_UV, "W_UV");
  check_fp32_contiguous(rope_cos, "rope_cos");
  check_fp32_contiguous(rope_sin, "rope_sin");
  la_mla_config cfg =
      config_from_args(d_model, kv_lora_rank, qk_nope_head_dim, qk_rope_head_dim, num_heads, v_head_dim);

  TORCH_CHECK(q_absorbed.dim() == 3, "q_absorbed must be 3D (batch, num_heads, kv_lora_rank)");
  TORCH_CHECK(q_rope.dim() == 3, "q_rope must be 3D (batch, num_heads, qk_rope_head_dim)");
  const int64_t batch = q_absorbed.size(0);
  TORCH_CHECK(kv_cache.dim() == 2, "kv_cache must be 2D (seq_len, kv_lora_rank + qk_rope_head_dim)");
  const int64_t seq_len = kv_cache.size(0);
  TORCH_CHECK(batch > 0, "batch_size must be positive, got ", batch);
  TORCH_CHECK(q_rope.size(0) == batch, "q_rope batch dim must match q_absorbed batch dim: ", q_rope.size(0), " vs ",
              batch);
  TORCH_CHECK(q_absorbed.size(1) == num_heads && q_absorbed.size(2) == kv_lora_rank,
              "q_absorbed shape mismatch: expected (", batch, ", ", num_heads, ", ", kv_lora_rank, ") got (",
              q_absorbed.size(0), ", ", q_absorbed.size(1), ", ", q_absorbed.size(2), ")");
  TORCH_CHECK(q_rope.size(1) == num_heads && q_rope.size(2) == qk_rope_head_dim, "q_rope shape mismatch");
  TORCH_CHECK(kv_cache.size(1) == kv_lora_rank + qk_rope_head_dim, "kv_cache dim1 mismatch");
  TORCH_CHECK(W_UV.dim() == 2 && W_UV.size(0) == (int64_t)num_heads * v_head_dim && W_UV.size(1) == kv_lora_rank,
              "W_UV shape mismatch");
  check_rope(rope_cos, rope_sin, seq_len, cfg);
  for (auto* t : {&q_absorbed, &q_rope, &W_UV, &rope_cos, &rope_sin}) check_same_device(kv_cache, *t, "inputs");
  TORCH_CHECK(seq_len <= INT32_MAX && batch <= INT32_MAX / num_heads, "problem too large");

  const at::DeviceGuard guard(kv_cache.device());
  auto output = torch::empty({batch, num_heads, v_head_dim}, kv_cache.options().dtype(torch::kFloat32));
  const size_t ws_bytes =
      la_fused_mla_workspace_size_dt((int)seq_len, (int)batch, &cfg, dtype_tag(kv_cache), dtype_tag(W_UV));
  auto ws = workspace(kv_cache, ws_bytes);
  int st = la_batched_fused_mla(kv_cache.data_ptr(), dtype_tag(kv_cache), (int)seq_len, (int)batch,
                                q_absorbed.data_ptr<float>(), q_rope.data_ptr<float>(), W_UV.data_ptr(),
                                dtype_tag(W_UV), rope_cos.data_ptr<float>(), rope_sin.data_ptr<float>(),
                                output.data_ptr<float>(), &cfg, ws.data_ptr(), ws_bytes, current_stream());
  check_status(st, "launch_batched_fused_mla");
  return output;
}

// mla_decode_forward -- the full decode step the north star adds: per-sequence
// caches, query absorption inside, split-KV + log-sum-exp combine, W_UV.
//   kv_cache: (B, S, dc+dR) uniform, or (T, dc+dR) packed with seq_offsets
//   seq_offsets: None or int32 (B+1,) device tensor of row offsets
//   q_nope (B, nh, dn) f32; q_rope (B, nh, dR) f32 (already rotated)
//   W_UK (nh*dn, dc); W_UV (nh*dv, dc); rope tables (>= longest seq, dR/2)
//   returns (B, nh, dv) f32. chunk_rows / kernel_variant: tuning overrides.
//   seq_lens: None or int32 (B,) device tensor; sequence b is the first
//   seq_lens[b] rows of its region (a capacity cache filled by append_kv).
namespace {

// Shared by mla_decode_forward and mla_decode_absorbed_forward: checks the
// cache / sequence / table arguments, fills the descriptor and runs it.
torch::Tensor run_decode(la_decode_args& a, const torch::Tensor& kv_cache, const torch::Tensor& q_rope,
                         const torch::Tensor& W_UV, const torch::Tensor& rope_cos, const torch::Tensor& rope_sin,
                         const c10::optional<torch::Tensor>& seq_offsets, const c10::optional<torch::Tensor>& seq_lens,
                         const la_mla_config& cfg, int64_t batch, int chunk_rows, int kernel_variant,
                         const c10::optional<torch::Tensor>& block_table, int block_size) {
  const int64_t row = cfg.kv_lora_rank + cfg.qk_rope_head_dim;
  TORCH_CHECK(q_rope.dim() == 3 && q_rope.size(0) == batch && q_rope.size(1) == cfg.num_heads &&
                  q_rope.size(2) == cfg.qk_rope_head_dim,
              "q_rope must be (batch, num_heads, qk_rope_head_dim)");
  TORCH_CHECK(W_UV.dim() == 2 && W_UV.size(0) == (int64_t)cfg.num_heads * cfg.v_head_dim &&
                  W_UV.size(1) == cfg.kv_lora_rank,
              "W_UV shape mismatch");
  TORCH_CHECK(batch <= INT32_MAX / cfg.num_heads, "batch too large");
  a.kv_cache = kv_cache.data_ptr();
  a.kv_dtype = dtype_tag(kv_cache);
  a.num_seqs = (int32_t)batch;
  a.queries_per_seq = 1;
  int64_t longest = 0;
  if (block_table.has_value() && block_table->defined()) {
    const auto& bt = *block_table;
    TORCH_CHECK(bt.dtype() == torch::kInt32 && bt.is_contiguous() && bt.is_cuda() && bt.dim() == 2 &&
                    bt.size(0) == batch,
                "block_table must be a contiguous int32 CUDA tensor (batch, blocks_per_seq)");
    TORCH_CHECK(!(seq_offsets.has_value() && seq_offsets->defined()), "block_table and seq_offsets exclude each other");
    TORCH_CHECK(seq_lens.has_value() && seq_lens->defined(), "a paged cache needs seq_lens");
    TORCH_CHECK(block_size > 0 && kv_cache.dim() == 2 && kv_cache.size(1) == row && kv_cache.size(0) % block_size == 0,
                "paged kv_cache must be a (num_blocks * block_size, ", row, ") pool");
    TORCH_CHECK(batch == 0 || kv_cache.size(0) >= block_size, "paged kv_cache pool needs at least one block");
    check_same_device(kv_cache, bt, "block_table");
    a.total_rows = kv_cache.size(0);
    a.block_table = bt.data_ptr<int32_t>();
    a.block_size = block_size;
    a.blocks_per_seq = (int32_t)bt.size(1);
  } else if (seq_offsets.has_value() && seq_offsets->defined()) {
    const auto& off = *seq_offsets;
    TORCH_CHECK(off.dtype() == torch::kInt32 && off.is_contiguous() && off.is_cuda(),
                "seq_offsets must be a contiguous int32 CUDA tensor");
    TORCH_CHECK(off.dim() == 1 && off.size(0) == batch + 1, "seq_offsets must have batch + 1 entries");
    check_same_device(kv_cache, off, "seq_offsets");
    TORCH_CHECK(kv_cache.dim() == 2 && kv_cache.size(1) == row, "packed kv_cache must be (total_rows, ", row, ")");
    a.total_rows = kv_cache.size(0);
    a.seq_offsets = off.data_ptr<int32_t>();
    // Sequences are at most total_rows long; positions past the table clamp.
    longest = 0;
  } else {
    TORCH_CHECK(kv_cache.dim() == 3 && kv_cache.size(0) == batch && kv_cache.size(2) == row,
                "kv_cache must be (batch, seq_len, ", row, ") when seq_offsets is None");
    TORCH_CHECK(kv_cache.size(1) <= INT32_MAX, "seq_len too large");
    a.seq_len = (int32_t)kv_cache.size(1);
    a.total_rows = batch * kv_cache.size(1);
    longest = kv_cache.size(1);
  }
  a.rope_rows = rope_cos.size(0);
  if (seq_lens.has_value() && seq_lens->defined()) {
    const auto& len = *seq_lens;
    TORCH_CHECK(len.dtype() == torch::kInt32 && len.is_contiguous() && len.is_cuda(),
                "seq_lens must be a contiguous int32 CUDA tensor");
    TORCH_CHECK(len.dim() == 1 && len.size(0) == batch, "seq_lens must have batch entries");
    check_same_device(kv_cache, len, "seq_lens");
    a.seq_lens = len.data_ptr<int32_t>();
    longest = 0;  // lengths live on the device; positions past the table clamp
  }
  check_rope(rope_cos, rope_sin, longest, cfg);
  for (auto* t : {&q_rope, &W_UV, &rope_cos, &rope_sin}) check_same_device(kv_cache, *t, "inputs");
  a.q_rope = q_rope.data_ptr<float>();
  a.W_UV = W_UV.data_ptr();
  a.w_uv_dtype = dtype_tag(W_UV);
  a.rope_cos = rope_cos.data_ptr<float>();
  a.rope_sin = rope_sin.data_ptr<float>();
  a.cfg = cfg;
  a.chunk_rows = chunk_rows;
  a.kernel_variant = kernel_variant;

  const at::DeviceGuard guard(kv_cache.device());
  auto output = torch::empty({batch, cfg.num_heads, cfg.v_head_dim}, kv_cache.options().dtype(torch::kFloat32));
  a.output = output.data_ptr<float>();
  const size_t ws_bytes = la_mla_decode_workspace_size(&a);
  TORCH_CHECK(ws_bytes > 0 || batch == 0, "mla_decode: unsupported arguments");
  auto ws = workspace(kv_cache, ws_bytes);
  a.workspace = ws.data_ptr();
  a.workspace_bytes = ws_bytes;
  check_status(la_mla_decode(&a, current_stream()), "la_mla_decode");
  return output;
}

}  // namespace

torch::Tensor mla_decode_forward(torch::Tensor kv_cache, torch::Tensor q_nope, torch::Tensor q_rope,
                                 torch::Tensor W_UK, torch::Tensor W_UV, torch::Tensor rope_cos,
                                 torch::Tensor rope_sin, c10::optional<torch::Tensor> seq_offsets, int d_model,
                                 int kv_lora_rank, int qk_nope_head_dim, int qk_rope_head_dim, int num_heads,
                                 int v_head_dim, int chunk_rows, int kernel_variant,
                                 c10::optional<torch::Tensor> seq_lens, c10::optional<torch::Tensor> block_table,
                                 int block_size) {
  check_storage(kv_cache, "kv_cache");
  check_fp32_contiguous(q_nope, "q_nope");
  check_fp32_contiguous(q_rope, "q_rope");
  check_weight(W_UK, "W_UK");
  check_weight(W_UV, "W_UV");
  check_fp32_contiguous(rope_cos, "rope_cos");
  check_fp32_contiguous(rope_sin, "rope_sin");
  la_mla_config cfg =
      config_from_args(d_model, kv_lora_rank, qk_nope_head_dim, qk_rope_head_dim, num_heads, v_head_dim);
  TORCH_CHECK(q_nope.dim() == 3 && q_nope.size(1) == num_heads && q_nope.size(2) == qk_nope_head_dim,
              "q_nope must be (batch, num_heads, qk_nope_head_dim)");
  TORCH_CHECK(W_UK.dim() == 2 && W_UK.size(0) == (int64_t)num_heads * qk_nope_head_dim && W_UK.size(1) == kv_lora_rank,
              "W_UK shape mismatch");
  check_same_device(kv_cache, q_nope, "q_nope");
  check_same_device(kv_cache, W_UK, "W_UK");
  la_decode_args a{};
  a.q_nope = q_nope.data_ptr<float>();
  a.W_UK = W_UK.data_ptr();
  a.w_uk_dtype = dtype_tag(W_UK);
  return run_decode(a, kv_cache, q_rope, W_UV, rope_cos, rope_sin, seq_offsets, seq_lens, cfg, q_nope.size(0),
                    chunk_rows, kernel_variant, block_table, block_size);
}

// mla_decode_absorbed_forward -- the same step for queries already absorbed
// (q_absorbed (B, nh, dc) f32, e.g. x . W_Q_absorbed^T as the reference's
// LatentAttentionLayer computes them, latent_attn/__init__.py:124-126).
torch::Tensor mla_decode_absorbed_forward(torch::Tensor kv_cache, torch::Tensor q_absorbed, torch::Tensor q_rope,
                                          torch::Tensor W_UV, torch::Tensor rope_cos, torch::Tensor rope_sin,
                                          c10::optional<torch::Tensor> seq_offsets, int d_model, int kv_lora_rank,
                                          int qk_nope_head_dim, int qk_rope_head_dim, int num_heads, int v_head_dim,
                                          int chunk_rows, int kernel_variant, c10::optional<torch::Tensor> seq_lens,
                                          c10::optional<torch::Tensor> block_table, int block_size) {
  check_storage(kv_cache, "kv_cache");
  check_fp32_contiguous(q_absorbed, "q_absorbed");
  check_fp32_contiguous(q_rope, "q_rope");
  check_weight(W_UV, "W_UV");
  check_fp32_contiguous(rope_cos, "rope_cos");
  check_fp32_contiguous(rope_sin, "rope_sin");
  la_mla_config cfg =
      config_from_args(d_model, kv_lora_rank, qk_nope_head_dim, qk_rope_head_dim, num_heads, v_head_dim);
  TORCH_CHECK(q_absorbed.dim() == 3 && q_absorbed.size(1) == num_heads && q_absorbed.size(2) == kv_lora_rank,
              "q_absorbed must be (batch, num_heads, kv_lora_rank)");
  check_same_device(kv_cache, q_absorbed, "q_absorbed");
  la_decode_args a{};
  a.q_absorbed = q_absorbed.data_ptr<float>();
  return run_decode(a, kv_cache, q_rope, W_UV, rope_cos, rope_sin, seq_offsets, seq_lens, cfg, q_absorbed.size(0),
                    chunk_rows, kernel_variant, block_table, block_size);
}

// append_kv_forward -- device-side LatentKVCache::append_host
// (src/mla_config.cuh:57-72) for a batch: appends c_t (B, T, dc) and k_rope
// (B, T, dR) (one dtype, any of the three) at each sequence's length in
// kv_cache ((B, capacity, dc+dR), or packed (rows, dc+dR) with seq_offsets
// (B+1,) int32 regions), advances seq_lens (B,) int32 in place and, when
// q_rope ((B*qps, nh, dR) f32) is given, rotates it in place for the
// positions of the last qps appended tokens. status: optional int32 (1,)
// device flag set to 1 when a sequence has no room.
void append_kv_forward(torch::Tensor kv_cache, torch::Tensor seq_lens, torch::Tensor c_t, torch::Tensor k_rope,
                       c10::optional<torch::Tensor> q_rope, c10::optional<torch::Tensor> rope_cos,
                       c10::optional<torch::Tensor> rope_sin, c10::optional<torch::Tensor> seq_offsets,
                       c10::optional<torch::Tensor> status, int d_model, int kv_lora_rank, int qk_nope_head_dim,
                       int qk_rope_head_dim, int num_heads, int v_head_dim, c10::optional<torch::Tensor> block_table,
                       int block_size) {
  check_storage(kv_cache, "kv_cache");
  check_storage(c_t, "c_t");
  check_storage(k_rope, "k_rope");
  la_mla_config cfg =
      config_from_args(d_model, kv_lora_rank, qk_nope_head_dim, qk_rope_head_dim, num_heads, v_head_dim);
  const int64_t row = kv_lora_rank + qk_rope_head_dim;
  TORCH_CHECK(seq_lens.dtype() == torch::kInt32 && seq_lens.is_contiguous() && seq_lens.is_cuda() &&
                  seq_lens.dim() == 1,
              "seq_lens must be a contiguous 1D int32 CUDA tensor");
  const int64_t batch = seq_lens.size(0);
  TORCH_CHECK(batch <= INT32_MAX, "batch too large");
  TORCH_CHECK(c_t.dim() == 3 && c_t.size(0) == batch && c_t.size(2) == kv_lora_rank,
              "c_t must be (batch, tokens, kv_lora_rank)");
  const int64_t tokens = c_t.size(1);
  TORCH_CHECK(tokens <= INT32_MAX, "too many tokens");
  TORCH_CHECK(k_rope.dim() == 3 && k_rope.size(0) == batch && k_rope.size(1) == tokens &&
                  k_rope.size(2) == qk_rope_head_dim,
              "k_rope must be (batch, tokens, qk_rope_head_dim)");
  TORCH_CHECK(k_rope.dtype() == c_t.dtype(), "c_t and k_rope must have the same dtype");
  for (auto* t : {&seq_lens, &c_t, &k_rope}) check_same_device(kv_cache, *t, "inputs");

  la_append_args a{};
  a.kv_cache = kv_cache.data_ptr();
  a.kv_dtype = dtype_tag(kv_cache);
  a.num_seqs = (int32_t)batch;
  a.seq_lens = seq_lens.data_ptr<int32_t>();
  a.tokens_per_seq = (int32_t)tokens;
  a.c_t = c_t.data_ptr();
  a.k_rope = k_rope.data_ptr();
  a.src_dtype = dtype_tag(c_t);
  a.cfg = cfg;
  if (block_table.has_value() && block_table->defined()) {
    const auto& bt = *block_table;
    TORCH_CHECK(bt.dtype() == torch::kInt32 && bt.is_contiguous() && bt.is_cuda() && bt.dim() == 2 &&
                    bt.size(0) == batch,
                "block_table must be a contiguous int32 CUDA tensor (batch, blocks_per_seq)");
    TORCH_CHECK(!(seq_offsets.has_value() && seq_offsets->defined()), "block_table and seq_offsets exclude each other");
    TORCH_CHECK(block_size > 0 && kv_cache.dim() == 2 && kv_cache.size(1) == row && kv_cache.size(0) % block_size == 0,
                "paged kv_cache must be a (num_blocks * block_size, ", row, ") pool");
    TORCH_CHECK(batch == 0 || kv_cache.size(0) >= block_size, "paged kv_cache pool needs at least one block");
    check_same_device(kv_cache, bt, "block_table");
    a.total_rows = kv_cache.size(0);
    a.block_table = bt.data_ptr<int32_t>();
    a.block_size = block_size;
    a.blocks_per_seq = (int32_t)bt.size(1);
  } else if (seq_offsets.has_value() && seq_offsets->defined()) {
    const auto& off = *seq_offsets;
    TORCH_CHECK(off.dtype() == torch::kInt32 && off.is_contiguous() && off.is_cuda(),
                "seq_offsets must be a contiguous int32 CUDA tensor");
    TORCH_CHECK(off.dim() == 1 && off.size(0) == batch + 1, "seq_offsets must have batch + 1 entries");
    check_same_device(kv_cache, off, "seq_offsets");
    TORCH_CHECK(kv_cache.dim() == 2 && kv_cache.size(1) == row, "packed kv_cache must be (total_rows, ", row, ")");
    a.total_rows = kv_cache.size(0);
    a.seq_offsets = off.data_ptr<int32_t>();
  } else {
    TORCH_CHECK(kv_cache.dim() == 3 && kv_cache.size(0) == batch && kv_cache.size(2) == row,
                "kv_cache must be (batch, capacity, ", row, ") when seq_offsets is None");
    TORCH_CHECK(kv_cache.size(1) <= INT32_MAX, "capacity too large");
    a.seq_capacity = (int32_t)kv_cache.size(1);
    a.total_rows = batch * kv_cache.size(1);
  }
  if (q_rope.has_value() && q_rope->defined()) {
    const auto& q = *q_rope;
    check_fp32_contiguous(q, "q_rope");
    TORCH_CHECK(batch > 0 && q.dim() == 3 && q.size(0) % batch == 0 && q.size(1) == num_heads &&
                    q.size(2) == qk_rope_head_dim,
                "q_rope must be (batch * queries_per_seq, num_heads, qk_rope_head_dim)");
    TORCH_CHECK(rope_cos.has_value() && rope_sin.has_value() && rope_cos->defined() && rope_sin->defined(),
                "rope_cos / rope_sin are required with q_rope");
    check_fp32_contiguous(*rope_cos, "rope_cos");
    check_fp32_contiguous(*rope_sin, "rope_sin");
    check_rope(*rope_cos, *rope_sin, 1, cfg);
    check_same_device(kv_cache, q, "q_rope");
    check_same_device(kv_cache, *rope_cos, "rope_cos");
    check_same_device(kv_cache, *rope_sin, "rope_sin");
    const int64_t qps = q.size(0) / batch;
    TORCH_CHECK(qps <= tokens, "queries_per_seq (", qps, ") must not exceed the appended tokens (", tokens, ")");
    a.q_rope = q.data_ptr<float>();
    a.queries_per_seq = (int32_t)qps;
    a.rope_cos = rope_cos->data_ptr<float>();
    a.rope_sin = rope_sin->data_ptr<float>();
    a.rope_rows = rope_cos->size(0);
  }
  if (status.has_value() && status->defined()) {
    TORCH_CHECK(status->dtype() == torch::kInt32 && status->is_cuda() && status->numel() >= 1,
                "status must be an int32 CUDA tensor");
    check_same_device(kv_cache, *status, "status");
    a.status = status->data_ptr<int32_t>();
  }
  const at::DeviceGuard guard(kv_cache.device());
  check_status(la_append_kv(&a, current_stream()), "la_append_kv");
}

// absorb_q_forward -- q_abs[t,h,c] = sum_i q_nope[t,h,i] W_UK[h*dn+i, c]
// (reference tests/test_correctness.cu:29-46, tests/test_python.py:97-99).
torch::Tensor absorb_q_forward(torch::Tensor q_nope, torch::Tensor W_UK, int d_model, int kv_lora_rank,
                               int qk_nope_head_dim, int qk_rope_head_dim, int num_heads, int v_head_dim) {
  check_fp32_contiguous(q_nope, "q_nope");
  check_weight(W_UK, "W_UK");
  la_mla_config cfg =
      config_from_args(d_model, kv_lora_rank, qk_nope_head_dim, qk_rope_head_dim, num_heads, v_head_dim);
  TORCH_CHECK(q_nope.dim() >= 2 && q_nope.size(-1) == qk_nope_head_dim && q_nope.size(-2) == num_heads,
              "q_nope must be (..., num_heads, qk_nope_head_dim)");
  TORCH_CHECK(W_UK.dim() == 2 && W_UK.size(0) == (int64_t)num_heads * qk_nope_head_dim && W_UK.size(1) == kv_lora_rank,
              "W_UK shape mismatch");
  check_same_device(q_nope, W_UK, "W_UK");
  const int64_t tokens = q_nope.numel() / ((int64_t)num_heads * qk_nope_head_dim);
  TORCH_CHECK(tokens <= INT32_MAX, "too many tokens");
  auto sizes = q_nope.sizes().vec();
  sizes.back() = kv_lora_rank;
  const at::DeviceGuard guard(q_nope.device());
  auto out = torch::empty(sizes, q_nope.options());
  check_status(la_absorb_q(q_nope.data_ptr<float>(), W_UK.data_ptr(), dtype_tag(W_UK), out.data_ptr<float>(),
                           (int)tokens, &cfg, current_stream()),
               "la_absorb_q");
  return out;
}

// naive_mla_forward -- reference csrc/bindings.cpp:53-114 signature:
// decompress-then-attend on the GPU (la_naive_mla: K_nope and V materialised
// in fp32, RoPE, softmax, P V), independent of the absorbed kernels.
torch::Tensor naive_mla_forward(torch::Tensor kv_cache, torch::Tensor W_UK, torch::Tensor W_UV,
                                torch::Tensor q_nope, torch::Tensor q_rope, torch::Tensor rope_cos,
                                torch::Tensor rope_sin, int d_model, int kv_lora_rank, int qk_nope_head_dim,
                                int qk_rope_head_dim, int num_heads, int v_head_dim) {
  check_storage(kv_cache, "kv_cache");
  check_weight(W_UK, "W_UK");
  check_weight(W_UV, "W_UV");
  check_fp32_contiguous(q_nope, "q_nope");
  check_fp32_contiguous(q_rope, "q_rope");
  check_fp32_contiguous(rope_cos, "rope_cos");
  check_fp32_contiguous(rope_sin, "rope_sin");
  config_from_args(d_model, kv_lora_rank, qk_nope_head_dim, qk_rope_head_dim, num_heads, v_head_dim);
  TORCH_CHECK(kv_cache.dim() == 2 && kv_cache.size(1) == kv_lora_rank + qk_rope_head_dim, "kv_cache dim1 must be ",
              kv_lora_rank + qk_rope_head_dim);
  TORCH_CHECK(q_nope.dim() == 2 && q_nope.size(0) == num_heads && q_nope.size(1) == qk_nope_head_dim,
              "q_nope shape mismatch");
  TORCH_CHECK(q_rope.dim() == 2 && q_rope.size(0) == num_heads && q_rope.size(1) == qk_rope_head_dim,
              "q_rope shape mismatch");
  TORCH_CHECK(W_UK.dim() == 2 && W_UK.size(0) == (int64_t)num_heads * qk_nope_head_dim && W_UK.size(1) == kv_lora_rank,
              "W_UK shape mismatch");
  TORCH_CHECK(W_UV.dim() == 2 && W_UV.size(0) == (int64_t)num_heads * v_head_dim && W_UV.size(1) == kv_lora_rank,
              "W_UV shape mismatch");
  TORCH_CHECK(kv_cache.size(0) <= INT32_MAX, "seq_len too large");
  const int seq_len = (int)kv_cache.size(0);
  la_mla_config cfg =
      config_from_args(d_model, kv_lora_rank, qk_nope_head_dim, qk_rope_head_dim, num_heads, v_head_dim);
  check_rope(rope_cos, rope_sin, seq_len, cfg);
  for (auto* t : {&W_UK, &W_UV, &q_nope, &q_rope, &rope_cos, &rope_sin}) check_same_device(kv_cache, *t, "inputs");
  const at::DeviceGuard guard(kv_cache.device());
  auto out = torch::empty({num_heads, v_head_dim}, kv_cache.options().dtype(torch::kFloat32));
  const size_t ws_bytes = la_naive_mla_workspace_size(seq_len, &cfg);
  auto ws = workspace(kv_cache, ws_bytes);
  check_status(la_naive_mla(kv_cache.data_ptr(), dtype_tag(kv_cache), seq_len, W_UK.data_ptr(), dtype_tag(W_UK),
                            W_UV.data_ptr(), dtype_tag(W_UV), q_nope.data_ptr<float>(), q_rope.data_ptr<float>(),
                            rope_cos.data_ptr<float>(), rope_sin.data_ptr<float>(), out.data_ptr<float>(), &cfg,
                            ws.data_ptr(), ws_bytes, current_stream()),
               "la_naive_mla");
  return out;
}

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  m.def("naive_mla_forward", &naive_mla_forward, "MLA forward from q_nope and W_UK (decompress-then-attend result)");
  m.def("fused_mla_forward", &fused_mla_forward,
        "Fused absorbed MLA forward (single token, online softmax in latent space)");
  m.def("batched_fused_mla_forward", &batched_fused_mla_forward,
        "Batched fused MLA forward (batch tokens, shared KV cache)");
  m.def("mla_decode_forward", &mla_decode_forward,
        "Batched MLA decode step over per-sequence or ragged caches (absorb, split-KV, combine, W_UV)",
        py::arg("kv_cache"), py::arg("q_nope"), py::arg("q_rope"), py::arg("W_UK"), py::arg("W_UV"),
        py::arg("rope_cos"), py::arg("rope_sin"), py::arg("seq_offsets"), py::arg("d_model"),
        py::arg("kv_lora_rank"), py::arg("qk_nope_head_dim"), py::arg("qk_rope_head_dim"), py::arg("num_heads"),
        py::arg("v_head_dim"), py::arg("chunk_rows") = 0, py::arg("kernel_variant") = 0,
        py::arg("seq_lens") = py::none(), py::arg("block_table") = py::none(), py::arg("block_size") = 0);
  m.def("mla_decode_absorbed_forward", &mla_decode_absorbed_forward,
        "Batched MLA decode step for pre-absorbed queries (split-KV, combine, W_UV)", py::arg("kv_cache"),
        py::arg("q_absorbed"), py::arg("q_rope"), py::arg("W_UV"), py::arg("rope_cos"), py::arg("rope_sin"),
        py::arg("seq_offsets"), py::arg("d_model"), py::arg("kv_lora_rank"), py::arg("qk_nope_head_dim"),
        py::arg("qk_rope_head_dim"), py::arg("num_heads"), py::arg("v_head_dim"), py::arg("chunk_rows") = 0,
        py::arg("kernel_variant") = 0, py::arg("seq_lens") = py::none(), py::arg("block_table") = py::none(),
        py::arg("block_size") = 0);
  m.def("append_kv_forward", &append_kv_forward,
        "Device-side append of latent rows at each sequence's length, with the query's RoPE",
        py::arg("kv_cache"), py::arg("seq_lens"), py::arg("c_t"), py::arg("k_rope"), py::arg("q_rope"),
        py::arg("rope_cos"), py::arg("rope_sin"), py::arg("seq_offsets"), py::arg("status"), py::arg("d_model"),
        py::arg("kv_lora_rank"), py::arg("qk_nope_head_dim"), py::arg("qk_rope_head_dim"), py::arg("num_heads"),
        py::arg("v_head_dim"), py::arg("block_table") = py::none(), py::arg("block_size") = 0);
  m.def("absorb_q_forward", &absorb_q_forward, "q_absorbed = q_nope . W_UK per head");
}
