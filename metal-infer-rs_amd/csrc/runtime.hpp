// Host runtime behind the C ABI: context, device memory, scratch arenas,
// batches and per-kernel profiling. Counterpart of
// crates/metal-infer-core/src/context.rs, designed for HIP: one in-order
// stream per context, device memory from hipMalloc, and HIP events for
// batch and per-kernel GPU time.
#pragma once

#include <hip/hip_runtime.h>

#include <chrono>
#include <cstdint>
#include <memory>
#include <string>
#include <unordered_map>
#include <unordered_set>
#include <vector>

#include "kernels.hpp"
#include "mi_attn.h"

struct mi_kv_cache;

namespace mi {

struct GemmState;

// Records `message` as this thread's last error and returns `status`.
mi_status fail(mi_status status, const std::string &message);
mi_status hip_fail(mi_status status, const char *what, hipError_t err);
void clear_error();
const std::string &last_error_string();

size_t dtype_size(int32_t dtype);
const char *dtype_name(int32_t dtype);

// One arena chunk: a device allocation with a sorted free list of
// [start, end) byte ranges (context.rs:173-190).
struct ScratchChunk {
  void *base = nullptr;
  size_t size = 0;
  std::vector<std::pair<size_t, size_t>> free;
};

// A scratch arena; a batch holds one exclusively while it is in flight
// (context.rs:715-729).
struct ScratchPool {
  std::vector<ScratchChunk> chunks;
  bool busy = false;
};

struct Lease {
  ScratchPool *pool;
  size_t chunk;
  size_t start;
  size_t end;
};

// Arena chunks are at least this large (the reference uses 1 MiB chunks
// for Metal's shared memory; split-K partials of a 32-sequence decode are
// tens of MiB, so chunks start bigger here).
constexpr size_t kScratchChunkBytes = 32ull << 20;
constexpr size_t kScratchAlignment = 256;

// One row of the tuned FlashDecode table: lengths up to `limit` run with
// (block_keys, threads); threads == 0 keeps the library default there.
struct FlashDecodeEntry {
  uint64_t limit;
  uint32_t block_keys;
  uint32_t threads;
};

struct Context {
  int device = 0;
  hipStream_t stream = nullptr;
  std::string name;
  uint32_t compute_units = 0;
  uint64_t allocated = 0;
  std::vector<std::unique_ptr<ScratchPool>> pools;
  std::unordered_map<uintptr_t, Lease> leases;
  std::unordered_map<uintptr_t, size_t> tensors;  // mi_tensor_empty sizes
  bool profiling = false;
  std::vector<mi_kernel_profile> profiles;
  std::vector<FlashDecodeEntry> flash_decode;  // tuned table, sorted
  // Arrival counters of split-K prefill (one per row tile and KV head). Zero
  // between kernels: the last split to arrive resets its counter.
  uint32_t *split_counters = nullptr;
  uint32_t split_counter_count = 0;

  // Live KV caches; destroying the context releases their storage and
  // detaches them, so a cache destroyed later only frees its handle.
  std::unordered_set<mi_kv_cache *> caches;
  // Live captured graphs (same ownership rule as caches).
  std::unordered_set<mi_graph *> graphs;
  // hipBLASLt handle and per-shape GEMM plans, made at the first matmul
  // with more rows than the few-row kernel takes.
  GemmState *gemm = nullptr;
  // Recorded on `stream` after each eager no-allocation call.
  hipEvent_t noalloc_done = nullptr;
};

// Frees the context's hipBLASLt handle and plans (after its stream drained).
void release_gemm(Context *ctx);

struct LaunchRecord {
  std::string kernel;
  hipEvent_t start;
  hipEvent_t end;
};

struct Batch {
  Context *ctx = nullptr;
  ScratchPool *pool = nullptr;
  hipEvent_t start = nullptr;
  hipEvent_t end = nullptr;
  bool committed = false;
  bool capturing = false;  // kernels are recorded into a HIP graph
  std::chrono::steady_clock::time_point commit_time;
  std::vector<LaunchRecord> launches;
};

// Leases `bytes` from the batch's arena (first fit, 256-B aligned).
mi_status scratch_alloc(Batch *batch, size_t bytes, void **out);
mi_status scratch_free(Context *ctx, void *ptr);

// Where one operation's scratch (split-K partials) comes from: the batch
// arena when `fixed` is null, else the fixed device buffer `fixed` of
// `limit` bytes (the no-allocation entry point). Launches of an operation
// with a fixed buffer carry no profiling events either, so it calls no
// allocating HIP routine.
struct ScratchSource {
  void *fixed = nullptr;
  size_t limit = 0;
};
// scratch_take: the arena lease, or the fixed buffer when `bytes` fits it
// (MI_ERR_RESOURCE naming both sizes when it does not). scratch_give
// returns an arena lease; nothing for the fixed buffer.
mi_status scratch_take(Batch *batch, const ScratchSource &src, size_t bytes, void **out);
void scratch_give(Context *ctx, const ScratchSource &src, void *ptr);

// The no-allocation entry point's fixed scratch: a file-scope device array
// of kNoAllocScratchBytes (csrc/noalloc.hip), one copy per GPU, held until
// the process ends. noalloc_init resolves its address on `device` (which
// must be current) once per device; noalloc_scratch returns that address,
// or null when it was never resolved.
constexpr size_t kNoAllocScratchBytes = 16ull << 20;
mi_status noalloc_init(int device);
void *noalloc_scratch(int device);
// Cross-context use of that array: noalloc_acquire fails with
// MI_ERR_RESOURCE while another context's last eager call is unfinished,
// else makes `ctx` its user; noalloc_mark records ctx's completion event
// after its launches (skipped under capture); noalloc_forget drops a
// destroyed context.
mi_status noalloc_acquire(Context *ctx, bool capturing);
void noalloc_mark(Context *ctx, bool capturing);
void noalloc_forget(const Context *ctx);


// Launches through `fn` on the batch stream. With kernel profiling on, the
// launch carries start / stop events bound to the kernel's dispatch (see
// kernels::Launch). `fn` returns the launch's hipError_t.
template <typename Fn>
mi_status launch(Batch *batch, const char *kernel, Fn &&fn, bool events = true) {
  kernels::Launch l;
  l.stream = batch->ctx->stream;
  if (events && batch->ctx->profiling && !batch->capturing) {
    if (hipEventCreate(&l.start) != hipSuccess || hipEventCreate(&l.stop) != hipSuccess) {
      if (l.start) hipEventDestroy(l.start);
      return fail(MI_ERR_PROFILING, "could not create profiling events");
    }
  }
  hipError_t err = fn(l);
  if (err != hipSuccess) {
    if (l.start) hipEventDestroy(l.start);
    if (l.stop) hipEventDestroy(l.stop);
    return hip_fail(MI_ERR_PIPELINE, kernel, err);
  }
  if (l.start) batch->launches.push_back({kernel, l.start, l.stop});
  return MI_OK;
}

// Tensor helpers.
bool is_contiguous(const mi_tensor &t);
uint64_t element_count(const mi_tensor &t);
mi_status require_f16(const mi_tensor *t);

}  // namespace mi

// Opaque handle types of the C ABI.
struct mi_context : mi::Context {};
struct mi_batch : mi::Batch {};
struct mi_graph {
  mi::Context *ctx = nullptr;
  mi::ScratchPool *pool = nullptr;  // the capturing batch's arena, kept busy
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
};
struct mi_kv_cache {
  mi::Context *ctx = nullptr;
  void *base = nullptr;
  uint32_t layers = 0;
  uint32_t kv_heads = 0;
  uint32_t head_dim = 0;
  uint64_t capacity = 0;
  uint64_t filled = 0;
};
