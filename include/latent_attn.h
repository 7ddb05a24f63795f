/*
 * latent_attn.h -- C ABI of the MI355X (gfx950) multi-head latent attention
 * decode library (liblatent_attn_hip.so).
 *
 * Plain C: pointers, sizes, integer tags. No torch or HIP types appear in the
 * signatures; a stream is passed as `void*` (a hipStream_t, NULL = default
 * stream). Every entry point is asynchronous on that stream, returns an
 * la_status, and never calls exit(). Device pointers are non-owning.
 *
 * Reference interfaces replaced (paths relative to the reference repo):
 *   la_fused_mla          <- launch_fused_mla          src/fused_mla.cuh:51,
 *                            src/fused_mla.cu:271-296
 *   la_batched_fused_mla  <- launch_batched_fused_mla  src/fused_mla_batched.cuh:35,
 *                            src/fused_mla_batched.cu:109-130
 *   la_naive_mla          <- naive_mla_forward         csrc/bindings.cpp:53-114,
 *                            src/naive_mla.cu:91-245 (decompress-then-attend)
 *   la_absorb_q           <- host absorption loop tests/test_correctness.cu:29-46
 *                            and einsum tests/test_python.py:97-99
 *   la_mla_decode         <- the decode step the north star adds on top of the
 *                            reference API (per-sequence / ragged caches, split-KV
 *                            with log-sum-exp combine, fused W_UV projection)
 *   la_mla_config         <- MLAConfig                 src/mla_config.cuh:7-13
 *                            (same six ints in the same order)
 *   la_append_kv          <- LatentKVCache::append_host src/mla_config.cuh:57-72
 *                            (host-to-device copies of one row plus a stream
 *                            synchronize per token), done on the device for
 *                            every sequence at once, with the query's RoPE
 *
 * Layouts (all row-major, contiguous):
 *   latent cache row   [c_t (kv_lora_rank) | k_rope (qk_rope_head_dim)]
 *                      (src/mla_config.cuh:43-48)
 *   W_UK               (num_heads*qk_nope_head_dim, kv_lora_rank)
 *   W_UV               (num_heads*v_head_dim, kv_lora_rank); head h owns rows
 *                      [h*v_head_dim, (h+1)*v_head_dim)   (src/fused_mla.cu:258-267)
 *   rope_cos/rope_sin  (rows >= longest sequence, qk_rope_head_dim/2) float32,
 *                      indexed by the key's position inside its sequence;
 *                      rotate-half pairing (i, i + d_R/2)   (src/fused_mla.cu:34-54)
 *   q_rope             already rotated for the query position (the reference
 *                      never rotates q; src/fused_mla.cu:34-54)
 *   scale              1/sqrt(qk_nope_head_dim + qk_rope_head_dim), applied
 *                      inside (src/fused_mla.cu:284)
 *   outputs            float32 (.., num_heads, v_head_dim)
 *
 * An empty sequence (length 0) produces a zero output row (the reference's
 * kernel would divide by zero there; its PyTorch reference sums an empty set).
 */
#ifndef LATENT_ATTN_H
#define LATENT_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LA_ABI_VERSION 4

typedef enum la_status {
  LA_SUCCESS = 0,
  LA_ERROR_INVALID_VALUE = 1, /* null pointer, bad shape or config         */
  LA_ERROR_NOT_SUPPORTED = 2, /* no kernel for this dtype / dims / device   */
  LA_ERROR_WORKSPACE = 3,     /* caller workspace smaller than required     */
  LA_ERROR_HIP = 4            /* a HIP call failed: see la_last_hip_error() */
} la_status;

typedef enum la_dtype {
  LA_DTYPE_F32 = 0,
  LA_DTYPE_F16 = 1,
  LA_DTYPE_BF16 = 2,
  /* OCP FP8 E4M3 ("e4m3fn": bias 7, no infinities, 0x7F / 0xFF NaN, max
   * 448), latent caches only (kv_dtype of decode, append and naive; not
   * weights). The MFMA decode kernel reads the 576-B rows and expands each
   * tile to bf16 in LDS (exact); kernel_variant 1 reads them on the VALU
   * kernel. Values written by la_append_kv round to nearest even and
   * saturate at +-448. */
  LA_DTYPE_FP8_E4M3 = 3
} la_dtype;

/* Same fields and order as the reference MLAConfig (src/mla_config.cuh:7-13). */
typedef struct la_mla_config {
  int32_t d_model;
  int32_t kv_lora_rank;     /* d_c */
  int32_t qk_nope_head_dim; /* d_n */
  int32_t qk_rope_head_dim; /* d_R */
  int32_t num_heads;
  int32_t v_head_dim;
} la_mla_config;

/* Arguments of one decode step (la_mla_decode). */
typedef struct la_decode_args {
  /* packed latent cache: total_rows rows of (kv_lora_rank + qk_rope_head_dim) */
  const void* kv_cache;
  int32_t kv_dtype; /* la_dtype */
  int64_t total_rows;
  /* sequences: num_seqs caches inside kv_cache.
   * seq_offsets == NULL: sequence s owns rows [s*seq_len, (s+1)*seq_len).
   * otherwise seq_offsets is a DEVICE int32 array of num_seqs+1 non-decreasing
   * row offsets with seq_offsets[num_seqs] <= total_rows. */
  int32_t num_seqs;
  int32_t seq_len;
  const int32_t* seq_offsets;
  /* query tokens sharing each sequence's cache (1 for ordinary decode; the
   * reference's shared-cache batched form is num_seqs = 1, queries_per_seq = B).
   * Query token t = s*queries_per_seq + j. */
  int32_t queries_per_seq;
  /* queries: either q_nope (+ W_UK, absorbed inside) or q_absorbed.
   * q_nope (tokens, num_heads, qk_nope_head_dim) f32; W_UK see header comment.
   * q_absorbed (tokens, num_heads, kv_lora_rank) f32. Exactly one of q_nope /
   * q_absorbed must be non-NULL. */
  const float* q_nope;
  const void* W_UK;
  int32_t w_uk_dtype;
  const float* q_absorbed;
  const float* q_rope; /* (tokens, num_heads, qk_rope_head_dim) f32 */
  const void* W_UV;
  int32_t w_uv_dtype;
  const float* rope_cos;
  const float* rope_sin;
  /* rows in rope_cos / rope_sin; 0 = unchecked (caller guarantees at least
   * the longest sequence). Positions past it read the last row instead of
   * faulting. */
  int64_t rope_rows;
  /* (tokens, num_heads, v_head_dim) f32; must not overlap an input (a call
   * with few query rows zeroes it first and adds partial products into it) */
  float* output;
  la_mla_config cfg;
  /* scratch for split partials (and the absorbed query when q_nope is given).
   * NULL: the library takes stream-ordered memory (hipMallocAsync) and returns
   * it on the same stream. */
  void* workspace;
  size_t workspace_bytes;
  /* tuning / test overrides, 0 = automatic:
   * chunk_rows     rows per split-KV chunk
   * kernel_variant 1 = VALU kernel, 2 = MFMA kernel (LA_ERROR_NOT_SUPPORTED if
   *                the shape has none) */
  int32_t chunk_rows;
  int32_t kernel_variant;
  /* optional DEVICE int32 array of num_seqs lengths (as la_append_kv keeps
   * them): sequence s is the first seq_lens[s] rows of its region above
   * (clamped into it; rows past it are unfilled capacity and are not read).
   * NULL: each sequence is its whole region. The split plan covers the
   * regions, so capacity far beyond the lengths costs idle blocks. */
  const int32_t* seq_lens;
  /* optional paged cache (block tables): kv_cache is then a pool of
   * total_rows rows in blocks of block_size rows (total_rows a multiple of
   * block_size), and position p of sequence s lives in pool row
   * block_table[s*blocks_per_seq + p/block_size]*block_size + p%block_size
   * (DEVICE int32 table, num_seqs*blocks_per_seq entries; ids outside the
   * pool are clamped into it). seq_lens is required, seq_offsets must be
   * NULL, seq_len is ignored. block_size a multiple of 32 keeps the MFMA
   * kernel (others run on the VALU kernel). NULL: contiguous cache. */
  const int32_t* block_table;
  int32_t block_size;
  int32_t blocks_per_seq;
} la_decode_args;

/* Arguments of la_append_kv. */
typedef struct la_append_args {
  /* latent cache, laid out as for la_decode_args: sequence s owns the region
   * [s*seq_capacity, (s+1)*seq_capacity) (seq_offsets == NULL) or
   * [seq_offsets[s], seq_offsets[s+1]) (DEVICE int32, num_seqs+1), and its
   * first seq_lens[s] rows are filled. */
  void* kv_cache;
  int32_t kv_dtype; /* la_dtype */
  int64_t total_rows;
  int32_t num_seqs;
  int32_t seq_capacity;
  const int32_t* seq_offsets;
  int32_t* seq_lens; /* DEVICE int32, num_seqs; advanced by tokens_per_seq */
  /* new rows: c_t (num_seqs, tokens_per_seq, kv_lora_rank) and k_rope
   * (num_seqs, tokens_per_seq, qk_rope_head_dim) in src_dtype, k_rope NOT
   * rotated (the attention rotates keys by their position, as the
   * reference's cache holds them). Row j of sequence s lands at position
   * seq_lens[s] + j. */
  int32_t tokens_per_seq;
  const void* c_t;
  const void* k_rope;
  int32_t src_dtype; /* la_dtype */
  /* optional: q_rope (num_seqs*queries_per_seq, num_heads, qk_rope_head_dim)
   * f32, rotated in place (rotate-half, src/fused_mla.cu:43-51) for its
   * position: query j of sequence s is the token at position
   * seq_lens[s] + tokens_per_seq - queries_per_seq + j (the last
   * queries_per_seq appended tokens; queries_per_seq <= tokens_per_seq).
   * When qk_rope_head_dim/2 is a multiple of 4, q_rope, rope_cos and rope_sin
   * must be 16-byte aligned. NULL: no query rotation. */
  float* q_rope;
  int32_t queries_per_seq;
  const float* rope_cos; /* (rope_rows, qk_rope_head_dim/2) f32 */
  const float* rope_sin;
  int64_t rope_rows; /* 0 = unchecked; positions past it use the last row */
  /* optional DEVICE int32: set to 1 when a sequence has no room for
   * tokens_per_seq more rows (that sequence is left unchanged: no rows, no
   * length change, no query rotation); never cleared by the library. */
  int32_t* status;
  la_mla_config cfg;
  /* optional paged cache, as in la_decode_args: kv_cache is a pool of
   * total_rows rows in blocks of block_size rows, sequence s has
   * blocks_per_seq blocks listed in the DEVICE int32 block_table (capacity
   * blocks_per_seq*block_size); seq_offsets must be NULL and seq_capacity is
   * ignored. NULL: contiguous cache. */
  const int32_t* block_table;
  int32_t block_size;
  int32_t blocks_per_seq;
} la_append_args;

/* Human-readable name of an la_status value. */
const char* la_status_string(int status);

/* Last hipError_t recorded by a failing call on this host thread (0 = none). */
int la_last_hip_error(void);

/* Library ABI version (LA_ABI_VERSION). */
int la_abi_version(void);

/* Bytes of workspace la_mla_decode needs for these arguments on the current
 * device (the fields kv_cache/q/output pointers are not read). */
size_t la_mla_decode_workspace_size(const la_decode_args* args);

/* One decode step: [absorb] -> split-KV latent attention -> log-sum-exp
 * combine -> W_UV projection. */
int la_mla_decode(const la_decode_args* args, void* stream);

/* The plan la_mla_decode would run for `args` on the current device. No
 * counterpart in the reference (its launch has no split plan); for callers
 * that size or schedule around the step and for tests. */
enum {
  LA_PLAN_ATTENTION_VALU = 1, /* decode_generic_kernel (any dtype and head shape) */
  LA_PLAN_ATTENTION_MFMA = 2  /* decode_mfma_kernel (kv_lora_rank 512, rope 64, 16-bit or FP8 cache, gfx950) */
};
enum {
  LA_PLAN_MERGE_VALU = 1,        /* combine_project_kernel */
  LA_PLAN_MERGE_MFMA = 2,        /* merge_project_kernel: full partial rows per workgroup */
  LA_PLAN_MERGE_MFMA_HALVES = 3  /* merge_project_half_kernel: latent halves added into the output */
};
enum {
  LA_PLAN_ABSORB_NONE = 0,       /* queries come absorbed (q_absorbed) */
  LA_PLAN_ABSORB_VALU = 1,       /* absorb_kernel into fp32 q_abs */
  LA_PLAN_ABSORB_MFMA = 2,       /* absorb_mfma_kernel into fp32 q_abs */
  LA_PLAN_ABSORB_MFMA_QPREP = 3  /* absorb_mfma_kernel straight into the attention kernel's 16-bit queries */
};
typedef struct la_plan_info {
  int32_t attention;   /* LA_PLAN_ATTENTION_* (0 when num_seqs == 0) */
  int32_t chunk_rows;  /* rows per split-KV chunk */
  int32_t num_chunks;
  int32_t num_slots;   /* partial slots per query head: num_chunks + num_seqs - 1 */
  int32_t head_groups; /* query-head groups per chunk (workgroups = num_chunks x head_groups, rounded for the XCDs) */
  int32_t merge;       /* LA_PLAN_MERGE_* */
  int32_t absorb;      /* LA_PLAN_ABSORB_* */
  size_t workspace_bytes; /* la_mla_decode_workspace_size(args) */
} la_plan_info;
int la_mla_decode_plan(const la_decode_args* args, la_plan_info* info);

/* la_mla_decode for profilers and benchmarks that time the split-KV attention
 * kernel alone. No counterpart in the reference. event_begin / event_end:
 * optional hipEvent_t handles recorded on `stream` right before and right
 * after the attention kernel (NULL = not recorded). repeat > 1 launches the
 * attention kernel that many times back to back between the two events (each
 * launch rewrites the same partial slots, so the result is unchanged), so the
 * events time launches whose dispatch overlaps the previous one; 0 or 1 =
 * once; negative = LA_ERROR_INVALID_VALUE. */
int la_mla_decode_profiled(const la_decode_args* args, void* stream, void* event_begin, void* event_end,
                           int32_t repeat);

/* Streaming-ceiling measurement of the attention kernel's copy schedule. No
 * counterpart in the reference; for benchmarks and profilers. Runs, with the
 * plan la_mla_decode would use for `args`, a copies-only variant of the MFMA
 * attention kernel: the same grid and block mapping and, per 32-position
 * tile, the same HBM->LDS copies of every wave (cache rows, k_rope rows,
 * RoPE table rows) into a ring of `ring` tile buffers (3: the kernel's own
 * ring; 4: the deepest one 160 KB of LDS holds), with one barrier per tile
 * and no compute. It reads the cache and the tables and writes nothing to
 * device memory (the output and workspace are untouched). repeat and the
 * optional events behave as in la_mla_decode_profiled. Returns
 * LA_ERROR_NOT_SUPPORTED unless args select the MFMA kernel on a contiguous
 * BF16 / F16 cache. */
int la_stream_ceiling(const la_decode_args* args, int32_t ring, void* stream, void* event_begin, void* event_end,
                      int32_t repeat);

/* la_mla_decode without any allocation. No counterpart in the reference: for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc). The scratch the
 * step needs (16-bit queries, split partials) comes from a static device
 * array of la_mla_decode_noalloc_max_bytes() bytes (64 MiB) that each GPU the
 * library runs on holds until the process ends; args->workspace and
 * workspace_bytes are ignored. Steps needing more than that return
 * LA_ERROR_WORKSPACE before any device work (la_mla_decode_workspace_size
 * gives the need). Every call on one GPU shares that GPU's array: calls that
 * overlap on one GPU (two streams, two threads) race and must be serialised
 * by the caller. Nothing in the array needs to start at zero; it keeps the
 * last call's contents. */
int la_mla_decode_noalloc(const la_decode_args* args, void* stream);
size_t la_mla_decode_noalloc_max_bytes(void);

/* Drop-in for launch_fused_mla (src/fused_mla.cuh:51): one query token over
 * one cache of seq_len rows. kv_cache / W_UV dtypes: F16 (the reference
 * contract), BF16 or F32. */
int la_fused_mla(const void* kv_cache, int kv_dtype, int seq_len, const float* q_absorbed, const float* q_rope,
                 const void* W_UV, int w_uv_dtype, const float* rope_cos, const float* rope_sin, float* output,
                 const la_mla_config* cfg, void* workspace, size_t workspace_bytes, void* stream);

/* Drop-in for launch_batched_fused_mla (src/fused_mla_batched.cuh:35):
 * batch_size query tokens over one SHARED cache. q_absorbed (B, nh, dc),
 * q_rope (B, nh, dR), output (B, nh, dv). */
int la_batched_fused_mla(const void* kv_cache, int kv_dtype, int seq_len, int batch_size, const float* q_absorbed,
                         const float* q_rope, const void* W_UV, int w_uv_dtype, const float* rope_cos,
                         const float* rope_sin, float* output, const la_mla_config* cfg, void* workspace,
                         size_t workspace_bytes, void* stream);

/* Workspace bytes la_fused_mla / la_batched_fused_mla need (batch_size 1 for
 * la_fused_mla): the largest over every cache and weight dtype. */
size_t la_fused_mla_workspace_size(int seq_len, int batch_size, const la_mla_config* cfg);

/* The same for one cache / weight dtype pair (la_dtype values): what the
 * torch extension and the C++ drop-in allocate. */
size_t la_fused_mla_workspace_size_dt(int seq_len, int batch_size, const la_mla_config* cfg, int kv_dtype,
                                      int w_uv_dtype);

/* Decompress-then-attend on the GPU, the reference's naive path
 * (naive_mla_forward, csrc/bindings.cpp:53-114; math of
 * tests/test_python.py:26-63): K_nope = c_t W_UK^T, V = c_t W_UV^T, RoPE on
 * k_rope, softmax, P V, all fp32, computed independently of the absorbed
 * kernels (a GPU check for shapes where a CPU restatement is slow). One query:
 * q_nope (num_heads, qk_nope_head_dim), q_rope (num_heads, qk_rope_head_dim)
 * f32 (already rotated); output (num_heads, v_head_dim) f32; rope tables have
 * >= seq_len rows. Workspace: la_naive_mla_workspace_size bytes (fp32 K_nope,
 * V and scores), or NULL for a stream-ordered allocation. The reference's
 * cuBLAS call reads K/V transposed (its naive path is wrong); this one is not. */
int la_naive_mla(const void* kv_cache, int kv_dtype, int seq_len, const void* W_UK, int w_uk_dtype, const void* W_UV,
                 int w_uv_dtype, const float* q_nope, const float* q_rope, const float* rope_cos,
                 const float* rope_sin, float* output, const la_mla_config* cfg, void* workspace,
                 size_t workspace_bytes, void* stream);
size_t la_naive_mla_workspace_size(int seq_len, const la_mla_config* cfg);

/* Appends tokens_per_seq rows to every sequence's cache on the device and
 * advances seq_lens (replaces LatentKVCache::append_host,
 * src/mla_config.cuh:57-72: no host copies, no synchronize, no host-side
 * length), then rotates the queries' q_rope for their positions. */
int la_append_kv(const la_append_args* args, void* stream);

/* Query absorption q_abs[t,h,c] = sum_i q_nope[t,h,i] * W_UK[h*dn+i, c]
 * (tests/test_correctness.cu:29-46). q_nope (tokens, nh, dn) f32,
 * q_absorbed (tokens, nh, dc) f32. */
int la_absorb_q(const float* q_nope, const void* W_UK, int w_uk_dtype, float* q_absorbed, int tokens,
                const la_mla_config* cfg, void* stream);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* LATENT_ATTN_H */
