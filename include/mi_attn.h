/*
 * mi_attn.h — C ABI of the MI355X (gfx950) causal GQA attention path.
 *
 * This is the drop-in boundary for metal-infer's attention hot path
 * (stratorys/metal-infer-rs; every citation below is relative to that
 * repository's root). A Rust `extern "C"` façade in a HIP backend of
 * metal-infer-core binds exactly these symbols.
 *
 * Conventions
 *  - Every fallible call returns an mi_status. On failure a human-readable
 *    message is kept per thread and returned by mi_last_error().
 *  - Tensors cross the boundary as plain descriptors (mi_tensor): a device
 *    address, dtype, rank, shape and element strides. No handle owns them;
 *    the caller keeps the memory alive until the batch that uses it has been
 *    waited on (the same contract as ops.rs:1311-1313).
 *  - A batch is an in-order sequence of kernels on the context's HIP stream
 *    (the counterpart of one MTLCommandBuffer). Each operation is enqueued
 *    on the stream when it is called, so the GPU may start before commit;
 *    commit closes the batch and wait / finish block until it is done.
 *    Outputs are readable only after wait.
 *  - The library owns only scratch memory (a per-batch arena) and the
 *    KV caches it creates; everything else is caller-owned.
 *  - Contexts are single-threaded, like MetalContext (`!Send + !Sync`).
 */
#ifndef MI_ATTN_H
#define MI_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MI_ATTN_ABI_VERSION 1
#define MI_MAX_RANK 4

/* Status codes; 1..11 map 1:1 onto CoreError
 * (crates/metal-infer-core/src/error.rs:5-32). */
typedef enum mi_status {
  MI_OK = 0,
  MI_ERR_NO_DEVICE = 1,         /* CoreError::NoDevice */
  MI_ERR_RESOURCE = 2,          /* CoreError::Resource (allocation, stream) */
  MI_ERR_SHADER = 3,            /* CoreError::Shader (code object missing) */
  MI_ERR_PIPELINE = 4,          /* CoreError::Pipeline (launch rejected) */
  MI_ERR_MISSING_KERNEL = 5,    /* CoreError::MissingKernel */
  MI_ERR_COMMAND = 6,           /* CoreError::Command (GPU error at wait) */
  MI_ERR_UNKNOWN_COMMAND = 7,   /* CoreError::UnknownCommand */
  MI_ERR_SHAPE = 8,             /* CoreError::Shape */
  MI_ERR_DTYPE = 9,             /* CoreError::DType */
  MI_ERR_DATA_LENGTH = 10,      /* CoreError::DataLength */
  MI_ERR_PROFILING = 11,        /* CoreError::Profiling */
  MI_ERR_INVALID_ARGUMENT = 12, /* null handle/pointer (Rust's types rule
                                   these out; no CoreError counterpart) */
  MI_ERR_CACHE_CAPACITY = 13    /* ModelError::CacheCapacity
                                   (crates/metal-infer-models/src/error.rs) */
} mi_status;

/* DType (crates/metal-infer-core/src/tensor.rs:11-33). */
typedef enum mi_dtype { MI_F16 = 0, MI_F32 = 1, MI_U32 = 2 } mi_dtype;

/* AttentionKind (crates/metal-infer-core/src/ops.rs:12-19). */
typedef enum mi_attention_kind {
  MI_ATTN_REFERENCE = 0,
  MI_ATTN_TILED = 1,
  MI_ATTN_FLASH_PREFILL = 2,
  MI_ATTN_DECODE_SPLIT_KV = 3,
  MI_ATTN_FLASH_DECODE = 4
} mi_attention_kind;

/* Tensor (tensor.rs:35-42) as a plain descriptor. `data` is the device
 * address of logical element 0 (any byte offset already applied). Strides
 * are in elements; the fast kernels need stride[rank-1] == 1. */
typedef struct mi_tensor {
  void *data;
  int32_t dtype;
  int32_t rank;
  int64_t shape[MI_MAX_RANK];
  int64_t stride[MI_MAX_RANK];
} mi_tensor;

/* AttentionConfig (ops.rs:29-36); `causal` is 0 or 1. */
typedef struct mi_attention_config {
  uint32_t query_heads;
  uint32_t kv_heads;
  uint32_t head_dim;
  uint32_t causal;
  uint32_t query_offset;
} mi_attention_config;

/* QkNormRopeCacheConfig (ops.rs:38-43). */
typedef struct mi_qk_norm_rope_cache_config {
  uint32_t offset;
  float theta;
  float epsilon;
} mi_qk_norm_rope_cache_config;

/* DispatchStats (context.rs:31-35), in nanoseconds. */
typedef struct mi_dispatch_stats {
  uint64_t gpu_ns;
  uint64_t wall_ns;
} mi_dispatch_stats;

/* KernelDispatchProfile (context.rs:37-41). */
typedef struct mi_kernel_profile {
  char kernel[64];
  double gpu_ns;
} mi_kernel_profile;

/* What mi_attention_plan decided (host-only; no device work). */
typedef struct mi_attention_plan_info {
  char kernel[64];        /* kernel family that would run */
  uint32_t grid[3];       /* workgroups */
  uint32_t block_threads; /* threads per workgroup */
  uint32_t block_keys;    /* split-K keys per workgroup (0 = no split) */
  uint32_t splits;        /* key splits per (row, KV head) */
  uint64_t scratch_bytes; /* split-K partials drawn from the batch arena */
} mi_attention_plan_info;

typedef struct mi_context mi_context;
typedef struct mi_batch mi_batch;
typedef struct mi_kv_cache mi_kv_cache;
typedef struct mi_graph mi_graph;

/* ------------------------------------------------------------ library -- */

/* Message for the last failing call on this thread ("" if none). */
const char *mi_last_error(void);
/* Returns MI_ATTN_ABI_VERSION. */
uint32_t mi_abi_version(void);
/* CoreError-style text for a status ("invalid tensor shape", ...). */
const char *mi_status_name(int32_t status);

/* ------------------------------------------------------------ context -- */

/* MetalContext::new (context.rs:216-248): binds HIP device `device`,
 * creates the context's stream (default priority) and loads the kernels. */
mi_status mi_context_create(int32_t device, mi_context **out);
void mi_context_destroy(mi_context *ctx);
/* MetalContext::device_name (context.rs:250-252). */
mi_status mi_context_device_name(const mi_context *ctx, char *buf, size_t len);
/* MetalContext::allocated_bytes (context.rs:340-342): device bytes held by
 * tensors, caches and scratch arenas of this context. */
uint64_t mi_context_allocated_bytes(const mi_context *ctx);
/* Number of compute units (used to size split-K grids). */
uint32_t mi_context_compute_units(const mi_context *ctx);

/* ------------------------------------------------------------ tensors -- */

/* MetalContext::empty (context.rs:740-754): a fresh contiguous device
 * tensor. Zero-sized or zero-rank shapes are a Shape error
 * (checked_elements, context.rs:1141-1153). */
mi_status mi_tensor_empty(mi_context *ctx, const int64_t *shape, int32_t rank,
                          int32_t dtype, mi_tensor *out);
/* Releases memory from mi_tensor_empty (no-op on views and NULL data). */
mi_status mi_tensor_free(mi_context *ctx, mi_tensor *tensor);
/* tensor_f16_bits / tensor_u32 (context.rs:776-817): synchronous host ->
 * device copy into a contiguous tensor; `bytes` must equal its byte length
 * (DataLength error otherwise). */
mi_status mi_tensor_upload(mi_context *ctx, const mi_tensor *tensor,
                           const void *host, size_t bytes);
/* with_f16_bits / to_u32_vec (tensor.rs:212-260): synchronous device ->
 * host copy of a tensor in logical (row-major) order, gathering strided
 * views. Only valid after the writing batch has been waited on. */
mi_status mi_tensor_download(mi_context *ctx, const mi_tensor *tensor,
                             void *host, size_t bytes);
/* Tensor::prefix (tensor.rs:133-157): same storage, first dimension cut to
 * `first_dimension` (1..capacity). Keeps strides, so head-major cache views
 * stay head-major. */
mi_status mi_tensor_prefix(const mi_tensor *tensor, int64_t first_dimension,
                           mi_tensor *out);
/* Tensor::reshape (tensor.rs:112-131) of a contiguous tensor. */
mi_status mi_tensor_reshape(const mi_tensor *tensor, const int64_t *shape,
                            int32_t rank, mi_tensor *out);

/* ------------------------------------------------------------ batches -- */

/* MetalContext::begin_batch (context.rs:703-738): claims an idle scratch
 * arena (or makes a new one) and opens an in-order batch. */
mi_status mi_batch_begin(mi_context *ctx, mi_batch **out);
/* CommandBatch::empty (context.rs:962-1022): a contiguous tensor leased from
 * the batch's arena (256-B aligned, first fit). The lease lives until
 * mi_scratch_release; freed ranges are reused by later work of the same
 * batch, which is safe because a batch executes in order. */
mi_status mi_batch_empty(mi_batch *batch, const int64_t *shape, int32_t rank,
                         int32_t dtype, mi_tensor *out);
/* Drop for ScratchLease (context.rs:1094-1117): returns the range to the
 * arena that leased it and merges neighbours. Valid before or after the
 * leasing batch has been waited on (a lease outlives its batch, like the
 * Tensor that CommandBatch::attention returns). */
mi_status mi_scratch_release(mi_context *ctx, const mi_tensor *tensor);
/* CommandBatch::commit (context.rs:1032-1045): non-blocking. */
mi_status mi_batch_commit(mi_batch *batch);
/* PendingBatch::wait (context.rs:1053-1083): blocks until the batch is
 * done, reports GPU and wall time, releases the arena and frees `batch`.
 * A GPU error is MI_ERR_COMMAND. */
mi_status mi_batch_wait(mi_batch *batch, mi_dispatch_stats *stats);
/* CommandBatch::finish (context.rs:1047-1049) = commit + wait. */
mi_status mi_batch_finish(mi_batch *batch, mi_dispatch_stats *stats);
/* Drop for an uncommitted CommandBatch (context.rs:1119-1128): nothing it
 * encoded runs... except work already handed to the stream, which is
 * drained before the arena is released. A capturing batch's recording is
 * discarded. Frees `batch`. */
void mi_batch_abandon(mi_batch *batch);
/* The hipStream_t the batch launches on (for interop and timing). */
void *mi_batch_stream(mi_batch *batch);

/* ------------------------------------------------------------- graphs -- */

/* Captured decode steps. The reference re-encodes a Metal command buffer for
 * every token (crates/metal-infer-models/src/qwen3.rs:475-555); on MI355X a
 * step's few small kernels are launch-bound, so a caller may record them
 * once and replay them. mi_batch_begin_capture opens a batch whose kernels
 * are recorded into a HIP graph (stream capture, relaxed mode) instead of
 * running. Only enqueueing calls belong in it (attention, copy_into_cache,
 * qk_norm_rope_cache(_value), rms_norm, rope, matmul, mi_batch_empty); no
 * upload, download or wait.
 * mi_batch_end_capture consumes the batch and returns the graph, which keeps
 * the batch's scratch arena (so tensors leased during capture stay valid and
 * every replay writes the same addresses). Each replay reads and writes the
 * tensors, offsets and cache slots that were current at capture. */
mi_status mi_batch_begin_capture(mi_context *ctx, mi_batch **out);
mi_status mi_batch_end_capture(mi_batch *batch, mi_graph **out);
/* Enqueues one replay on the context's stream (in order with batches). */
mi_status mi_graph_launch(mi_context *ctx, mi_graph *graph);
/* Waits for the stream, then frees the graph and releases its arena. */
void mi_graph_destroy(mi_graph *graph);
/* Blocks until everything enqueued on the context's stream has finished;
 * a GPU error is MI_ERR_COMMAND. */
mi_status mi_context_synchronize(mi_context *ctx);

/* ---------------------------------------------------------- profiling -- */

/* set_kernel_profiling / take_kernel_profiles (context.rs:602-700): when
 * enabled, every kernel a batch launches carries start / stop HIP events
 * bound to its dispatch (hipExtLaunchKernelGGL), and its execution time is
 * reported per launch after wait. A split-K attention records its split
 * pass ("attn_rows") and merge pass ("attn_merge") separately. */
mi_status mi_context_set_kernel_profiling(mi_context *ctx, int32_t enabled);
mi_status mi_context_take_kernel_profiles(mi_context *ctx,
                                          mi_kernel_profile *out,
                                          size_t capacity, size_t *count);

/* ---------------------------------------------------------- attention -- */

/* CommandBatch::attention (ops.rs:979-994 -> 1050-1247).
 * q [T, Hq, D], k/v [L, Hkv, D] f16 (any strides with unit innermost
 * stride; head-major cache prefixes are read in place), out [T, Hq, D] f16
 * caller-provided. Validation and error text follow ops.rs:1065-1150, with
 * one deliberate extension: FlashDecode accepts every GQA ratio (the
 * reference kernel is hard-wired to Hq == 2 * Hkv, ops.rs:1141-1145).
 * FlashPrefill runs its MFMA kernel when q, k, v and out have 16-byte
 * aligned rows (base and outer strides multiples of 8 elements); other
 * views take the rows kernel, with the same results. */
mi_status mi_attention(mi_batch *batch, const mi_tensor *q, const mi_tensor *k,
                       const mi_tensor *v, const mi_attention_config *config,
                       int32_t kind, const mi_tensor *out);
/* attention_flash_decode_with_block (ops.rs:996-1005): threads = 256. */
mi_status mi_attention_flash_decode_with_block(
    mi_batch *batch, const mi_tensor *q, const mi_tensor *k, const mi_tensor *v,
    const mi_attention_config *config, uint32_t block_keys,
    const mi_tensor *out);
/* attention_flash_decode_with_configuration (ops.rs:1007-1026):
 * block_keys in {32, 64, 128, 256}, threads in {128, 256}. */
mi_status mi_attention_flash_decode_with_configuration(
    mi_batch *batch, const mi_tensor *q, const mi_tensor *k, const mi_tensor *v,
    const mi_attention_config *config, uint32_t block_keys, uint32_t threads,
    const mi_tensor *out);
/* Host-only dry run of mi_attention's validation and kernel choice
 * (ops.rs:1065-1150). block_keys/threads = 0 picks the defaults. The
 * choice assumes an output with 16-byte aligned rows. */
mi_status mi_attention_plan(const mi_context *ctx, const mi_tensor *q,
                            const mi_tensor *k, const mi_tensor *v,
                            const mi_attention_config *config, int32_t kind,
                            uint32_t block_keys, uint32_t threads,
                            mi_attention_plan_info *info);

/* Batched split-K decode: B sequences, one new query each. No counterpart
 * in the reference (its decode is single-sequence). q [B, Hq, D]; k/v
 * [B, C, Hkv, D] views (C = per-sequence capacity); lengths: device u32 [B]
 * (values above C are clamped to C; a sequence of length 0 gets NaN, the
 * reference's 0/0); causal over each sequence (query at position
 * lengths[b] - 1). out [B, Hq, D]. config->query_offset is ignored.
 * block_keys = 0 picks the default: at head_dim 128 and B <= 1024 an MFMA
 * kernel whose workgroups share all sequences' keys equally (stream-K),
 * otherwise the rows kernel over a flat (sequence, KV head, split) grid.
 * block_keys > 0 runs the rows kernel with splits of that many keys. */
mi_status mi_attention_decode_batched(mi_batch *batch, const mi_tensor *q,
                                      const mi_tensor *k, const mi_tensor *v,
                                      const mi_tensor *lengths,
                                      const mi_attention_config *config,
                                      uint32_t block_keys,
                                      const mi_tensor *out);

/* mi_attention_decode_batched without any allocation. No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). Same arguments, kernels, results and errors as
 * mi_attention_decode_batched, except that the split-K partials live in a
 * fixed per-GPU buffer of 16 MiB (kept until the process ends) instead of
 * the batch arena: a call whose partials need more fails with
 * MI_ERR_RESOURCE (the default head_dim-128 plan fits about 7,500 units of
 * one sequence, one KV head and 4 query heads, in a compact partial layout
 * past about 840 of them, with the same results), and its launches carry no
 * kernel-profiling events. Every
 * call on one GPU shares that buffer; calls in one stream's order are safe.
 * A call from a second context while the first context's last eager call is
 * still unfinished fails with MI_ERR_RESOURCE instead of racing it; calls
 * recorded into graphs are not tracked, so overlapping replays race. */
mi_status mi_attention_decode_batched_noalloc(mi_batch *batch, const mi_tensor *q,
                                              const mi_tensor *k, const mi_tensor *v,
                                              const mi_tensor *lengths,
                                              const mi_attention_config *config,
                                              uint32_t block_keys, const mi_tensor *out);

/* FlashDecode (block, threads) for a KV length
 * (flash_decode_configuration_for_length, context.rs:258-267): the tuned
 * entry, or untuned (128, 256). Untuned, mi_attention's FlashDecode runs the
 * library default instead: 128-key splits on 512-thread workgroups with the
 * split merge inside the launch; passing a configuration explicitly selects
 * the reference-sized threadgroup and a separate merge launch. */
mi_status mi_flash_decode_configuration_for_length(const mi_context *ctx,
                                                   uint64_t length,
                                                   uint32_t *block_keys,
                                                   uint32_t *threads);
/* MetalContext::tune_flash_decode (context.rs:269-338): for each of the
 * reference's lengths, times the library default and each of the
 * reference's (block, threads) pairs on constant synthetic caches, and
 * records a pair only where it beats the default by 3%; elsewhere the
 * default stays. Runs on every device and every GQA ratio (the reference
 * only tunes on an M4 Pro with Hq == 2 * Hkv). Replaces an earlier table. */
mi_status mi_tune_flash_decode(mi_context *ctx, uint32_t query_heads,
                               uint32_t kv_heads, uint32_t head_dim);

/* attention_kind_for_tokens (crates/metal-infer-models/src/qwen3.rs:799-822)
 * generalised: FlashDecode serves every GQA ratio. Returns a kind. */
int32_t mi_attention_kind_for_tokens(int32_t configured, uint64_t tokens,
                                     uint64_t active_length,
                                     uint64_t query_heads_per_kv);

/* ----------------------------------------------------------- KV cache -- */

/* CommandBatch::copy_into_cache (ops.rs:1249-1285): writes source
 * [T, Hkv, D] into cache [capacity, Hkv, D] (any strides, e.g. a head-major
 * cache view) at position `offset`. Shape error if offset + T > capacity. */
mi_status mi_copy_into_cache(mi_batch *batch, const mi_tensor *source,
                             const mi_tensor *cache, uint64_t offset);

/* CommandBatch::qk_norm_rope_cache (ops.rs:917-977): per-head RMSNorm with
 * q_weight / k_weight [D], RoPE at position offset + token, Q to q_out
 * [T, Hq, D], K straight into key_cache [capacity, Hkv, D] at `offset`. */
mi_status mi_qk_norm_rope_cache(mi_batch *batch, const mi_tensor *q,
                                const mi_tensor *k, const mi_tensor *q_weight,
                                const mi_tensor *k_weight,
                                const mi_tensor *key_cache,
                                const mi_qk_norm_rope_cache_config *config,
                                const mi_tensor *q_out);

/* qk_norm_rope_cache followed by copy_into_cache of the value rows, in one
 * launch. No counterpart in the reference: forward_layer issues the two back
 * to back for every layer and token (crates/metal-infer-models/src/
 * qwen3.rs:704-728), and on MI355X one kernel fewer per layer shortens a
 * captured decode step. value [T, Hkv, D] goes to value_cache
 * [capacity, Hkv, D] at config->offset; every other argument, and every
 * error, is as for mi_qk_norm_rope_cache and mi_copy_into_cache. */
mi_status mi_qk_norm_rope_cache_value(mi_batch *batch, const mi_tensor *q,
                                      const mi_tensor *k, const mi_tensor *value,
                                      const mi_tensor *q_weight,
                                      const mi_tensor *k_weight,
                                      const mi_tensor *key_cache,
                                      const mi_tensor *value_cache,
                                      const mi_qk_norm_rope_cache_config *config,
                                      const mi_tensor *q_out);

/* One decode token's attention step in one launch: qk_norm_rope_cache, the
 * value's copy_into_cache and FlashDecode attention over the cache prefix
 * [0, qk_config->offset] (key_cache / value_cache [capacity, Hkv, D]), the
 * three calls forward_layer issues per layer and token (crates/
 * metal-infer-models/src/qwen3.rs:704-750; ops.rs:917-994, 1249-1285). No
 * counterpart in the reference as one call. q / k / value are [1, H, D];
 * the rotated query is not returned; out [1, Hq, D] gets the attention.
 * config->query_offset must equal qk_config->offset. Errors are those of the
 * three calls. At head_dim 128 with 16-byte aligned rows (and the library's
 * default decode split) the query and key transforms run inside the
 * attention kernel; otherwise the three calls' kernels run in order. */
mi_status mi_decode_step_attention(mi_batch *batch, const mi_tensor *q,
                                   const mi_tensor *k, const mi_tensor *value,
                                   const mi_tensor *q_weight,
                                   const mi_tensor *k_weight,
                                   const mi_tensor *key_cache,
                                   const mi_tensor *value_cache,
                                   const mi_qk_norm_rope_cache_config *qk_config,
                                   const mi_attention_config *config,
                                   const mi_tensor *out);

/* ------------------------------------------------ attention neighbours -- */

/* The steps on either side of attention in Qwen3's forward_layer
 * (crates/metal-infer-models/src/qwen3.rs:717-752): the unfused Q/K path
 * (rms_norm, rope, copy_into_cache) and the o_proj matmul of the attention
 * output. Outputs are caller-provided, like mi_attention's. */

/* CommandBatch::rms_norm (ops.rs:722-755): out = f16(x * scale * weight) per
 * row of the last dimension, scale = 1 / sqrt(mean(x^2) + epsilon) in f32.
 * input of rank 1..4 (unit innermost stride), weight [width], out of the
 * input's shape. */
mi_status mi_rms_norm(mi_batch *batch, const mi_tensor *input,
                      const mi_tensor *weight, float epsilon,
                      const mi_tensor *out);
/* CommandBatch::rope (ops.rs:882-915): input [T, H, D] with even D; pair
 * (i, i + D/2) of token t rotated by (offset + t) * theta^(-2i/D). out has
 * the input's shape. */
mi_status mi_rope(mi_batch *batch, const mi_tensor *input, uint64_t offset,
                  float theta, const mi_tensor *out);
/* CommandBatch::matmul (ops.rs:242-373): out[m, n] = f16(sum_k input[m, k] *
 * weight[n, k]) with f32 accumulation (weight in the checkpoint's
 * [out_features, in_features] layout). Up to 8 rows run the library's
 * HBM-streaming few-row kernel; more rows run a hipBLASLt f16 GEMM with f32
 * compute, planned once per shape (or the few-row kernel over groups of 8
 * rows when hipBLASLt has no solution for the shape). */
mi_status mi_matmul(mi_batch *batch, const mi_tensor *input,
                    const mi_tensor *weight, const mi_tensor *out);

/* KvCache::new (crates/metal-infer-models/src/qwen3.rs:75-100): one device
 * allocation holding, per layer, key and value as [Hkv, capacity, D]
 * (head-major). Capacity 0 is an error, as in the reference. */
mi_status mi_kv_cache_create(mi_context *ctx, uint32_t layers,
                             uint32_t kv_heads, uint32_t head_dim,
                             uint64_t capacity, mi_kv_cache **out);
void mi_kv_cache_destroy(mi_kv_cache *cache);
/* KvCache::len / capacity / reset (qwen3.rs:102-116). */
uint64_t mi_kv_cache_len(const mi_kv_cache *cache);
uint64_t mi_kv_cache_capacity(const mi_kv_cache *cache);
void mi_kv_cache_reset(mi_kv_cache *cache);
/* `cache.filled = n` (qwen3.rs:632, rollback at :401-409); n > capacity is
 * MI_ERR_CACHE_CAPACITY. */
mi_status mi_kv_cache_set_len(mi_kv_cache *cache, uint64_t filled);
/* LayerCache (qwen3.rs:36-40): logical [capacity, Hkv, D] views of one
 * layer's key and value storage, strides {D, capacity * D, 1}. */
mi_status mi_kv_cache_layer(const mi_kv_cache *cache, uint32_t layer,
                            mi_tensor *key, mi_tensor *value);

#ifdef __cplusplus
}
#endif

#endif /* MI_ATTN_H */
