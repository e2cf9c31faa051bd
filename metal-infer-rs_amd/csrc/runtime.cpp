// Context, memory, scratch arenas, batches, profiling and the KV cache of
// the C ABI (include/mi_attn.h). Mirrors crates/metal-infer-core/src/
// context.rs and tensor.rs, and KvCache from
// crates/metal-infer-models/src/qwen3.rs:68-117.
#include "runtime.hpp"

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>

namespace mi {

namespace {
thread_local std::string g_last_error;

mi_status check_shape(const int64_t *shape, int32_t rank, uint64_t *count) {
  if (shape == nullptr || rank < 1 || rank > MI_MAX_RANK)
    return fail(MI_ERR_SHAPE, "rank and dimensions must be non-zero");
  uint64_t n = 1;
  for (int32_t i = 0; i < rank; ++i) {
    if (shape[i] <= 0)
      return fail(MI_ERR_SHAPE, "rank and dimensions must be non-zero");
    if (n > UINT64_MAX / (uint64_t)shape[i])
      return fail(MI_ERR_SHAPE, "element count overflow");
    n *= (uint64_t)shape[i];
  }
  *count = n;
  return MI_OK;
}

void fill_contiguous(mi_tensor *t, void *data, const int64_t *shape,
                     int32_t rank, int32_t dtype) {
  std::memset(t, 0, sizeof *t);
  t->data = data;
  t->dtype = dtype;
  t->rank = rank;
  int64_t stride = 1;
  for (int32_t i = rank - 1; i >= 0; --i) {
    t->shape[i] = shape[i];
    t->stride[i] = stride;
    stride *= shape[i];
  }
}

bool valid_dtype(int32_t dtype) {
  return dtype == MI_F16 || dtype == MI_F32 || dtype == MI_U32;
}

// Smallest and one-past-largest element offsets a strided view touches.
void span_of(const mi_tensor &t, int64_t *lo, int64_t *hi) {
  int64_t a = 0, b = 0;
  for (int32_t i = 0; i < t.rank; ++i) {
    const int64_t extent = (t.shape[i] - 1) * t.stride[i];
    if (extent < 0)
      a += extent;
    else
      b += extent;
  }
  *lo = a;
  *hi = b + 1;
}

// Calls fn(logical_index, element_offset) in row-major logical order.
template <typename Fn>
void for_each_element(const mi_tensor &t, Fn &&fn) {
  int64_t idx[MI_MAX_RANK] = {0, 0, 0, 0};
  const uint64_t n = element_count(t);
  for (uint64_t i = 0; i < n; ++i) {
    int64_t off = 0;
    for (int32_t d = 0; d < t.rank; ++d) off += idx[d] * t.stride[d];
    fn(i, off);
    for (int32_t d = t.rank - 1; d >= 0; --d) {
      if (++idx[d] < t.shape[d]) break;
      idx[d] = 0;
    }
  }
}

size_t align_up(size_t value, size_t alignment) {
  return (value + alignment - 1) / alignment * alignment;
}

void merge_free(std::vector<std::pair<size_t, size_t>> &free) {
  std::sort(free.begin(), free.end());
  std::vector<std::pair<size_t, size_t>> merged;
  for (const auto &r : free) {
    if (!merged.empty() && merged.back().second == r.first)
      merged.back().second = r.second;
    else
      merged.push_back(r);
  }
  free.swap(merged);
}
}  // namespace

mi_status fail(mi_status status, const std::string &message) {
  g_last_error = message;
  return status;
}

mi_status hip_fail(mi_status status, const char *what, hipError_t err) {
  return fail(status, std::string(what) + ": " + hipGetErrorString(err));
}

void clear_error() { g_last_error.clear(); }

const std::string &last_error_string() { return g_last_error; }

size_t dtype_size(int32_t dtype) {
  return dtype == MI_F16 ? 2 : (dtype == MI_F32 || dtype == MI_U32 ? 4 : 0);
}

const char *dtype_name(int32_t dtype) {
  switch (dtype) {
    case MI_F16: return "f16";
    case MI_F32: return "f32";
    case MI_U32: return "u32";
    default: return "unknown";
  }
}

bool is_contiguous(const mi_tensor &t) {
  int64_t stride = 1;
  for (int32_t i = t.rank - 1; i >= 0; --i) {
    if (t.shape[i] != 1 && t.stride[i] != stride) return false;
    stride *= t.shape[i];
  }
  return true;
}

uint64_t element_count(const mi_tensor &t) {
  uint64_t n = 1;
  for (int32_t i = 0; i < t.rank; ++i) n *= (uint64_t)t.shape[i];
  return n;
}

mi_status require_f16(const mi_tensor *t) {
  if (t->dtype != MI_F16)
    return fail(MI_ERR_DTYPE, std::string("unsupported dtype: expected f16, got ") +
                                  dtype_name(t->dtype));
  return MI_OK;
}

mi_status scratch_alloc(Batch *batch, size_t bytes, void **out) {
  Context *ctx = batch->ctx;
  ScratchPool *pool = batch->pool;
  const size_t need = align_up(std::max<size_t>(bytes, 1), kScratchAlignment);
  for (size_t c = 0; c < pool->chunks.size(); ++c) {
    auto &free = pool->chunks[c].free;
    for (size_t r = 0; r < free.size(); ++r) {
      if (free[r].second - free[r].first < need) continue;
      const size_t start = free[r].first;
      if (free[r].second - start == need)
        free.erase(free.begin() + (long)r);
      else
        free[r].first = start + need;
      void *ptr = static_cast<char *>(pool->chunks[c].base) + start;
      ctx->leases[(uintptr_t)ptr] = {pool, c, start, start + need};
      *out = ptr;
      return MI_OK;
    }
  }
  ScratchChunk chunk;
  chunk.size = std::max(need, kScratchChunkBytes);
  hipError_t err = hipMalloc(&chunk.base, chunk.size);
  if (err != hipSuccess) return hip_fail(MI_ERR_RESOURCE, "scratch buffer", err);
  ctx->allocated += chunk.size;
  if (need < chunk.size) chunk.free.push_back({need, chunk.size});
  pool->chunks.push_back(chunk);
  ctx->leases[(uintptr_t)chunk.base] = {pool, pool->chunks.size() - 1, 0, need};
  *out = chunk.base;
  return MI_OK;
}

mi_status scratch_free(Context *ctx, void *ptr) {
  auto it = ctx->leases.find((uintptr_t)ptr);
  if (it == ctx->leases.end())
    return fail(MI_ERR_INVALID_ARGUMENT, "pointer is not a live scratch lease");
  const Lease lease = it->second;
  ctx->leases.erase(it);
  auto &free = lease.pool->chunks[lease.chunk].free;
  free.push_back({lease.start, lease.end});
  merge_free(free);
  return MI_OK;
}

mi_status scratch_take(Batch *batch, const ScratchSource &src, size_t bytes, void **out) {
  if (src.fixed == nullptr) return scratch_alloc(batch, bytes, out);
  if (bytes > src.limit)
    return fail(MI_ERR_RESOURCE, "scratch of " + std::to_string(bytes) +
                                     " bytes exceeds the no-allocation buffer of " +
                                     std::to_string(src.limit) + " bytes");
  *out = src.fixed;
  return MI_OK;
}

void scratch_give(Context *ctx, const ScratchSource &src, void *ptr) {
  if (src.fixed == nullptr && ptr != nullptr) scratch_free(ctx, ptr);
}

}  // namespace mi

using namespace mi;

extern "C" {

uint32_t mi_abi_version(void) { return MI_ATTN_ABI_VERSION; }

const char *mi_status_name(int32_t status) {
  // The Display strings of CoreError (error.rs:7-31), without payloads.
  switch (status) {
    case MI_OK: return "ok";
    case MI_ERR_NO_DEVICE: return "no GPU device is available";
    case MI_ERR_RESOURCE: return "could not create GPU resource";
    case MI_ERR_SHADER: return "GPU code object could not be loaded";
    case MI_ERR_PIPELINE: return "GPU kernel launch failed";
    case MI_ERR_MISSING_KERNEL: return "GPU kernel was not found";
    case MI_ERR_COMMAND: return "GPU command failed";
    case MI_ERR_UNKNOWN_COMMAND: return "GPU command failed without an error";
    case MI_ERR_SHAPE: return "invalid tensor shape";
    case MI_ERR_DTYPE: return "unsupported dtype";
    case MI_ERR_DATA_LENGTH: return "host data length mismatch";
    case MI_ERR_PROFILING: return "GPU kernel profiling failed";
    case MI_ERR_INVALID_ARGUMENT: return "invalid argument";
    case MI_ERR_CACHE_CAPACITY: return "KV cache capacity exceeded";
    default: return "unknown status";
  }
}

mi_status mi_context_create(int32_t device, mi_context **out) {
  if (out == nullptr) return fail(MI_ERR_INVALID_ARGUMENT, "null output handle");
  *out = nullptr;
  int count = 0;
  if (hipGetDeviceCount(&count) != hipSuccess || count == 0)
    return fail(MI_ERR_NO_DEVICE, "no HIP device is available");
  if (device < 0 || device >= count)
    return fail(MI_ERR_NO_DEVICE, "HIP device index out of range");
  hipError_t err = hipSetDevice(device);
  if (err != hipSuccess) return hip_fail(MI_ERR_NO_DEVICE, "hipSetDevice", err);
  hipDeviceProp_t prop;
  err = hipGetDeviceProperties(&prop, device);
  if (err != hipSuccess) return hip_fail(MI_ERR_NO_DEVICE, "device properties", err);
  auto ctx = std::make_unique<mi_context>();
  ctx->device = device;
  ctx->name = std::string(prop.name) + " (" + prop.gcnArchName + ")";
  ctx->compute_units = (uint32_t)prop.multiProcessorCount;
  // Default priority only: streams of other priorities are not used.
  err = hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking);
  if (err != hipSuccess) return hip_fail(MI_ERR_RESOURCE, "command stream", err);
  const uint32_t counters = kernels::kSplitCounters;
  err = hipMalloc(&ctx->split_counters, counters * sizeof(uint32_t));
  if (err == hipSuccess) err = hipMemset(ctx->split_counters, 0, counters * sizeof(uint32_t));
  if (err == hipSuccess) err = hipDeviceSynchronize();
  if (err != hipSuccess) {
    if (ctx->split_counters != nullptr) hipFree(ctx->split_counters);
    hipStreamDestroy(ctx->stream);
    return hip_fail(MI_ERR_RESOURCE, "split counters", err);
  }
  ctx->split_counter_count = counters;
  ctx->allocated += counters * sizeof(uint32_t);
  // The no-allocation entry point's fixed scratch on this device.
  mi_status st = noalloc_init(device);
  if (st == MI_OK) {
    err = hipEventCreateWithFlags(&ctx->noalloc_done, hipEventDisableTiming);
    if (err != hipSuccess) st = hip_fail(MI_ERR_RESOURCE, "no-allocation event", err);
  }
  if (st != MI_OK) {
    hipFree(ctx->split_counters);
    hipStreamDestroy(ctx->stream);
    return st;
  }
  *out = ctx.release();
  return MI_OK;
}

static void release_graph(mi_graph *graph);

void mi_context_destroy(mi_context *ctx) {
  if (ctx == nullptr) return;
  hipSetDevice(ctx->device);
  hipStreamSynchronize(ctx->stream);
  for (auto &pool : ctx->pools)
    for (auto &chunk : pool->chunks) hipFree(chunk.base);
  for (auto &entry : ctx->tensors) hipFree(reinterpret_cast<void *>(entry.first));
  for (mi_graph *graph : ctx->graphs) {
    release_graph(graph);
    graph->ctx = nullptr;
  }
  for (mi_kv_cache *cache : ctx->caches) {
    hipFree(cache->base);
    cache->base = nullptr;
    cache->ctx = nullptr;
  }
  hipFree(ctx->split_counters);
  mi::release_gemm(ctx);
  mi::noalloc_forget(ctx);
  if (ctx->noalloc_done != nullptr) hipEventDestroy(ctx->noalloc_done);
  hipStreamDestroy(ctx->stream);
  delete ctx;
}

mi_status mi_context_device_name(const mi_context *ctx, char *buf, size_t len) {
  if (ctx == nullptr || buf == nullptr || len == 0)
    return fail(MI_ERR_INVALID_ARGUMENT, "null context or buffer");
  std::snprintf(buf, len, "%s", ctx->name.c_str());
  return MI_OK;
}

uint64_t mi_context_allocated_bytes(const mi_context *ctx) {
  return ctx ? ctx->allocated : 0;
}

uint32_t mi_context_compute_units(const mi_context *ctx) {
  return ctx ? ctx->compute_units : 0;
}

mi_status mi_tensor_empty(mi_context *ctx, const int64_t *shape, int32_t rank,
                          int32_t dtype, mi_tensor *out) {
  if (ctx == nullptr || out == nullptr)
    return fail(MI_ERR_INVALID_ARGUMENT, "null context or output");
  if (!valid_dtype(dtype)) return fail(MI_ERR_DTYPE, "unknown dtype");
  uint64_t count = 0;
  mi_status st = check_shape(shape, rank, &count);
  if (st != MI_OK) return st;
  const size_t bytes = count * dtype_size(dtype);
  void *data = nullptr;
  hipSetDevice(ctx->device);
  hipError_t err = hipMalloc(&data, bytes);
  if (err != hipSuccess) return hip_fail(MI_ERR_RESOURCE, "buffer", err);
  ctx->tensors[(uintptr_t)data] = bytes;
  ctx->allocated += bytes;
  fill_contiguous(out, data, shape, rank, dtype);
  return MI_OK;
}

mi_status mi_tensor_free(mi_context *ctx, mi_tensor *tensor) {
  if (ctx == nullptr || tensor == nullptr)
    return fail(MI_ERR_INVALID_ARGUMENT, "null context or tensor");
  auto it = ctx->tensors.find((uintptr_t)tensor->data);
  if (it == ctx->tensors.end()) return MI_OK;
  hipStreamSynchronize(ctx->stream);
  hipFree(tensor->data);
  ctx->allocated -= it->second;
  ctx->tensors.erase(it);
  tensor->data = nullptr;
  return MI_OK;
}

mi_status mi_tensor_upload(mi_context *ctx, const mi_tensor *tensor,
                           const void *host, size_t bytes) {
  if (ctx == nullptr || tensor == nullptr || host == nullptr || tensor->data == nullptr)
    return fail(MI_ERR_INVALID_ARGUMENT, "null context, tensor or host pointer");
  const size_t esize = dtype_size(tensor->dtype);
  const uint64_t count = element_count(*tensor);
  if (bytes != count * esize)
    return fail(MI_ERR_DATA_LENGTH, "host data has " + std::to_string(bytes / (esize ? esize : 1)) +
                                        " elements, expected " + std::to_string(count));
  hipSetDevice(ctx->device);
  hipError_t err;
  if (is_contiguous(*tensor)) {
    err = hipMemcpy(tensor->data, host, bytes, hipMemcpyHostToDevice);
  } else {
    // Read-modify-write the span the view covers.
    int64_t lo, hi;
    span_of(*tensor, &lo, &hi);
    std::vector<char> span((size_t)(hi - lo) * esize);
    char *dev = static_cast<char *>(tensor->data) + lo * (int64_t)esize;
    err = hipMemcpy(span.data(), dev, span.size(), hipMemcpyDeviceToHost);
    if (err == hipSuccess) {
      const char *src = static_cast<const char *>(host);
      for_each_element(*tensor, [&](uint64_t i, int64_t off) {
        std::memcpy(span.data() + (off - lo) * (int64_t)esize, src + i * esize, esize);
      });
      err = hipMemcpy(dev, span.data(), span.size(), hipMemcpyHostToDevice);
    }
  }
  if (err != hipSuccess) return hip_fail(MI_ERR_COMMAND, "upload", err);
  return MI_OK;
}

mi_status mi_tensor_download(mi_context *ctx, const mi_tensor *tensor,
                             void *host, size_t bytes) {
  if (ctx == nullptr || tensor == nullptr || host == nullptr || tensor->data == nullptr)
    return fail(MI_ERR_INVALID_ARGUMENT, "null context, tensor or host pointer");
  const size_t esize = dtype_size(tensor->dtype);
  const uint64_t count = element_count(*tensor);
  if (bytes != count * esize)
    return fail(MI_ERR_DATA_LENGTH, "host buffer has " + std::to_string(bytes / (esize ? esize : 1)) +
                                        " elements, expected " + std::to_string(count));
  hipSetDevice(ctx->device);
  hipError_t err;
  if (is_contiguous(*tensor)) {
    err = hipMemcpy(host, tensor->data, bytes, hipMemcpyDeviceToHost);
  } else {
    int64_t lo, hi;
    span_of(*tensor, &lo, &hi);
    std::vector<char> span((size_t)(hi - lo) * esize);
    const char *dev = static_cast<const char *>(tensor->data) + lo * (int64_t)esize;
    err = hipMemcpy(span.data(), dev, span.size(), hipMemcpyDeviceToHost);
    if (err == hipSuccess) {
      char *dst = static_cast<char *>(host);
      for_each_element(*tensor, [&](uint64_t i, int64_t off) {
        std::memcpy(dst + i * esize, span.data() + (off - lo) * (int64_t)esize, esize);
      });
    }
  }
  if (err != hipSuccess) return hip_fail(MI_ERR_COMMAND, "download", err);
  return MI_OK;
}

mi_status mi_tensor_prefix(const mi_tensor *tensor, int64_t first_dimension,
                           mi_tensor *out) {
  if (tensor == nullptr || out == nullptr)
    return fail(MI_ERR_INVALID_ARGUMENT, "null tensor or output");
  if (tensor->rank < 1) return fail(MI_ERR_SHAPE, "prefix requires rank >= 1");
  if (first_dimension <= 0 || first_dimension > tensor->shape[0])
    return fail(MI_ERR_SHAPE, "prefix " + std::to_string(first_dimension) +
                                  " is outside capacity " + std::to_string(tensor->shape[0]));
  *out = *tensor;
  out->shape[0] = first_dimension;
  return MI_OK;
}

mi_status mi_tensor_reshape(const mi_tensor *tensor, const int64_t *shape,
                            int32_t rank, mi_tensor *out) {
  if (tensor == nullptr || out == nullptr)
    return fail(MI_ERR_INVALID_ARGUMENT, "null tensor or output");
  uint64_t count = 0;
  if (check_shape(shape, rank, &count) != MI_OK || count != element_count(*tensor))
    return fail(MI_ERR_SHAPE, "cannot reshape tensor into the requested shape");
  if (!is_contiguous(*tensor))
    return fail(MI_ERR_SHAPE, "reshape requires a contiguous tensor");
  fill_contiguous(out, tensor->data, shape, rank, tensor->dtype);
  return MI_OK;
}

mi_status mi_batch_begin(mi_context *ctx, mi_batch **out) {
  if (ctx == nullptr || out == nullptr)
    return fail(MI_ERR_INVALID_ARGUMENT, "null context or output");
  *out = nullptr;
  hipSetDevice(ctx->device);
  auto batch = std::make_unique<mi_batch>();
  batch->ctx = ctx;
  for (auto &pool : ctx->pools)
    if (!pool->busy) {
      batch->pool = pool.get();
      break;
    }
  if (batch->pool == nullptr) {
    ctx->pools.push_back(std::make_unique<ScratchPool>());
    batch->pool = ctx->pools.back().get();
  }
  if (hipEventCreate(&batch->start) != hipSuccess ||
      hipEventCreate(&batch->end) != hipSuccess)
    return fail(MI_ERR_RESOURCE, "batch events");
  batch->pool->busy = true;
  hipEventRecord(batch->start, ctx->stream);
  *out = batch.release();
  return MI_OK;
}

mi_status mi_batch_empty(mi_batch *batch, const int64_t *shape, int32_t rank,
                         int32_t dtype, mi_tensor *out) {
  if (batch == nullptr || out == nullptr)
    return fail(MI_ERR_INVALID_ARGUMENT, "null batch or output");
  if (!valid_dtype(dtype)) return fail(MI_ERR_DTYPE, "unknown dtype");
  uint64_t count = 0;
  mi_status st = check_shape(shape, rank, &count);
  if (st != MI_OK) return st;
  void *data = nullptr;
  st = scratch_alloc(batch, count * dtype_size(dtype), &data);
  if (st != MI_OK) return st;
  fill_contiguous(out, data, shape, rank, dtype);
  return MI_OK;
}

mi_status mi_scratch_release(mi_context *ctx, const mi_tensor *tensor) {
  if (ctx == nullptr || tensor == nullptr)
    return fail(MI_ERR_INVALID_ARGUMENT, "null context or tensor");
  return scratch_free(ctx, tensor->data);
}

mi_status mi_batch_commit(mi_batch *batch) {
  if (batch == nullptr) return fail(MI_ERR_INVALID_ARGUMENT, "null batch");
  if (batch->committed) return fail(MI_ERR_RESOURCE, "batch was already committed");
  if (batch->capturing)
    return fail(MI_ERR_RESOURCE, "a capturing batch ends with mi_batch_end_capture");
  hipError_t err = hipEventRecord(batch->end, batch->ctx->stream);
  if (err != hipSuccess) return hip_fail(MI_ERR_COMMAND, "commit", err);
  batch->committed = true;
  batch->commit_time = std::chrono::steady_clock::now();
  return MI_OK;
}

static void release_batch(mi_batch *batch, bool keep_pool = false) {
  for (auto &rec : batch->launches) {
    hipEventDestroy(rec.start);
    hipEventDestroy(rec.end);
  }
  if (batch->start) hipEventDestroy(batch->start);
  if (batch->end) hipEventDestroy(batch->end);
  if (!keep_pool) batch->pool->busy = false;
  delete batch;
}

mi_status mi_batch_wait(mi_batch *batch, mi_dispatch_stats *stats) {
  if (batch == nullptr) return fail(MI_ERR_INVALID_ARGUMENT, "null batch");
  if (!batch->committed) {
    mi_status st = mi_batch_commit(batch);
    if (st != MI_OK) return st;
  }
  hipError_t err = hipEventSynchronize(batch->end);
  const auto wall = std::chrono::steady_clock::now() - batch->commit_time;
  if (err == hipSuccess) err = hipGetLastError();
  mi_status status = MI_OK;
  if (err != hipSuccess) {
    status = hip_fail(MI_ERR_COMMAND, "GPU command failed", err);
  } else {
    float ms = 0.0f;
    hipEventElapsedTime(&ms, batch->start, batch->end);
    if (stats != nullptr) {
      stats->gpu_ns = (uint64_t)((double)ms * 1.0e6);
      stats->wall_ns = (uint64_t)std::chrono::duration_cast<std::chrono::nanoseconds>(wall).count();
    }
    for (auto &rec : batch->launches) {
      float kms = 0.0f;
      if (hipEventElapsedTime(&kms, rec.start, rec.end) != hipSuccess) {
        status = fail(MI_ERR_PROFILING, "invalid GPU timestamps for kernel " + rec.kernel);
        break;
      }
      mi_kernel_profile prof;
      std::memset(&prof, 0, sizeof prof);
      std::snprintf(prof.kernel, sizeof prof.kernel, "%s", rec.kernel.c_str());
      prof.gpu_ns = (double)kms * 1.0e6;
      batch->ctx->profiles.push_back(prof);
    }
  }
  release_batch(batch);
  return status;
}

mi_status mi_batch_finish(mi_batch *batch, mi_dispatch_stats *stats) {
  mi_status st = mi_batch_commit(batch);
  if (st != MI_OK) {
    if (batch != nullptr) mi_batch_abandon(batch);
    return st;
  }
  return mi_batch_wait(batch, stats);
}

void mi_batch_abandon(mi_batch *batch) {
  if (batch == nullptr) return;
  if (batch->capturing) {
    // Close the capture and drop what it recorded.
    hipGraph_t graph = nullptr;
    if (hipStreamEndCapture(batch->ctx->stream, &graph) == hipSuccess && graph != nullptr)
      hipGraphDestroy(graph);
    (void)hipGetLastError();
  }
  // Kernels already handed to the stream must drain before the arena they
  // use can be claimed by another batch.
  hipStreamSynchronize(batch->ctx->stream);
  release_batch(batch);
}

mi_status mi_batch_begin_capture(mi_context *ctx, mi_batch **out) {
  mi_status st = mi_batch_begin(ctx, out);
  if (st != MI_OK) return st;
  mi_batch *batch = *out;
  // The batch's own timing events are not part of the graph.
  hipEventDestroy(batch->start);
  hipEventDestroy(batch->end);
  batch->start = batch->end = nullptr;
  hipError_t err = hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeRelaxed);
  if (err != hipSuccess) {
    release_batch(batch);
    *out = nullptr;
    return hip_fail(MI_ERR_COMMAND, "hipStreamBeginCapture", err);
  }
  batch->capturing = true;
  return MI_OK;
}

mi_status mi_batch_end_capture(mi_batch *batch, mi_graph **out) {
  if (batch == nullptr || out == nullptr)
    return fail(MI_ERR_INVALID_ARGUMENT, "null batch or output");
  *out = nullptr;
  if (!batch->capturing) return fail(MI_ERR_RESOURCE, "batch is not capturing");
  Context *ctx = batch->ctx;
  auto graph = std::make_unique<mi_graph>();
  hipError_t err = hipStreamEndCapture(ctx->stream, &graph->graph);
  batch->capturing = false;
  if (err == hipSuccess)
    err = hipGraphInstantiate(&graph->exec, graph->graph, nullptr, nullptr, 0);
  if (err != hipSuccess) {
    if (graph->graph != nullptr) hipGraphDestroy(graph->graph);
    release_batch(batch);
    return hip_fail(MI_ERR_COMMAND, "graph capture", err);
  }
  graph->ctx = ctx;
  graph->pool = batch->pool;  // stays busy: replays write into its ranges
  release_batch(batch, /*keep_pool=*/true);
  ctx->graphs.insert(graph.get());
  *out = graph.release();
  return MI_OK;
}

mi_status mi_graph_launch(mi_context *ctx, mi_graph *graph) {
  if (ctx == nullptr || graph == nullptr)
    return fail(MI_ERR_INVALID_ARGUMENT, "null context or graph");
  if (graph->ctx != ctx) return fail(MI_ERR_INVALID_ARGUMENT, "graph belongs to another context");
  hipError_t err = hipGraphLaunch(graph->exec, ctx->stream);
  if (err != hipSuccess) return hip_fail(MI_ERR_COMMAND, "hipGraphLaunch", err);
  return MI_OK;
}

static void release_graph(mi_graph *graph) {
  if (graph->exec != nullptr) hipGraphExecDestroy(graph->exec);
  if (graph->graph != nullptr) hipGraphDestroy(graph->graph);
  graph->exec = nullptr;
  graph->graph = nullptr;
}

void mi_graph_destroy(mi_graph *graph) {
  if (graph == nullptr) return;
  if (graph->ctx != nullptr) {
    hipStreamSynchronize(graph->ctx->stream);  // no replay may still use the arena
    release_graph(graph);
    graph->pool->busy = false;
    graph->ctx->graphs.erase(graph);
  }
  delete graph;
}

mi_status mi_context_synchronize(mi_context *ctx) {
  if (ctx == nullptr) return fail(MI_ERR_INVALID_ARGUMENT, "null context");
  hipError_t err = hipStreamSynchronize(ctx->stream);
  if (err != hipSuccess) return hip_fail(MI_ERR_COMMAND, "GPU command failed", err);
  return MI_OK;
}

void *mi_batch_stream(mi_batch *batch) {
  return batch ? static_cast<void *>(batch->ctx->stream) : nullptr;
}

mi_status mi_context_set_kernel_profiling(mi_context *ctx, int32_t enabled) {
  if (ctx == nullptr) return fail(MI_ERR_INVALID_ARGUMENT, "null context");
  ctx->profiling = enabled != 0;
  return MI_OK;
}

mi_status mi_context_take_kernel_profiles(mi_context *ctx, mi_kernel_profile *out,
                                          size_t capacity, size_t *count) {
  if (ctx == nullptr || count == nullptr)
    return fail(MI_ERR_INVALID_ARGUMENT, "null context or count");
  const size_t n = std::min(capacity, ctx->profiles.size());
  if (out != nullptr)
    for (size_t i = 0; i < n; ++i) out[i] = ctx->profiles[i];
  *count = out != nullptr ? n : ctx->profiles.size();
  if (out != nullptr) ctx->profiles.erase(ctx->profiles.begin(), ctx->profiles.begin() + (long)n);
  return MI_OK;
}

mi_status mi_kv_cache_create(mi_context *ctx, uint32_t layers, uint32_t kv_heads,
                             uint32_t head_dim, uint64_t capacity, mi_kv_cache **out) {
  if (ctx == nullptr || out == nullptr)
    return fail(MI_ERR_INVALID_ARGUMENT, "null context or output");
  *out = nullptr;
  if (capacity == 0) return fail(MI_ERR_SHAPE, "KV cache capacity must be non-zero");
  if (layers == 0 || kv_heads == 0 || head_dim == 0)
    return fail(MI_ERR_SHAPE, "KV cache dimensions must be non-zero");
  const uint64_t per_tensor = (uint64_t)kv_heads * capacity * head_dim;
  const uint64_t bytes = per_tensor * 2 * layers * sizeof(uint16_t);
  void *base = nullptr;
  hipSetDevice(ctx->device);
  hipError_t err = hipMalloc(&base, bytes);
  if (err != hipSuccess) return hip_fail(MI_ERR_RESOURCE, "KV cache", err);
  ctx->allocated += bytes;
  auto cache = new mi_kv_cache();
  cache->ctx = ctx;
  cache->base = base;
  cache->layers = layers;
  cache->kv_heads = kv_heads;
  cache->head_dim = head_dim;
  cache->capacity = capacity;
  ctx->caches.insert(cache);
  *out = cache;
  return MI_OK;
}

void mi_kv_cache_destroy(mi_kv_cache *cache) {
  if (cache == nullptr) return;
  Context *ctx = cache->ctx;
  if (ctx != nullptr) {  // else its context already released the storage
    hipSetDevice(ctx->device);
    hipStreamSynchronize(ctx->stream);
    hipFree(cache->base);
    ctx->allocated -= (uint64_t)cache->kv_heads * cache->capacity * cache->head_dim * 2 *
                      cache->layers * sizeof(uint16_t);
    ctx->caches.erase(cache);
  }
  delete cache;
}

uint64_t mi_kv_cache_len(const mi_kv_cache *cache) { return cache ? cache->filled : 0; }
uint64_t mi_kv_cache_capacity(const mi_kv_cache *cache) { return cache ? cache->capacity : 0; }
void mi_kv_cache_reset(mi_kv_cache *cache) {
  if (cache) cache->filled = 0;
}

mi_status mi_kv_cache_set_len(mi_kv_cache *cache, uint64_t filled) {
  if (cache == nullptr) return fail(MI_ERR_INVALID_ARGUMENT, "null cache");
  if (filled > cache->capacity)
    return fail(MI_ERR_CACHE_CAPACITY,
                "KV cache capacity " + std::to_string(cache->capacity) +
                    " is smaller than requested length " + std::to_string(filled));
  cache->filled = filled;
  return MI_OK;
}

mi_status mi_kv_cache_layer(const mi_kv_cache *cache, uint32_t layer,
                            mi_tensor *key, mi_tensor *value) {
  if (cache == nullptr || key == nullptr || value == nullptr)
    return fail(MI_ERR_INVALID_ARGUMENT, "null cache or output");
  if (layer >= cache->layers) return fail(MI_ERR_SHAPE, "missing KV cache layer");
  if (cache->ctx == nullptr) return fail(MI_ERR_RESOURCE, "KV cache outlived its context");
  const uint64_t per_tensor = (uint64_t)cache->kv_heads * cache->capacity * cache->head_dim;
  uint16_t *base = static_cast<uint16_t *>(cache->base) + per_tensor * 2 * layer;
  for (int which = 0; which < 2; ++which) {
    mi_tensor *t = which == 0 ? key : value;
    std::memset(t, 0, sizeof *t);
    t->data = base + per_tensor * which;
    t->dtype = MI_F16;
    t->rank = 3;
    t->shape[0] = (int64_t)cache->capacity;
    t->shape[1] = cache->kv_heads;
    t->shape[2] = cache->head_dim;
    t->stride[0] = cache->head_dim;  // position
    t->stride[1] = (int64_t)cache->capacity * cache->head_dim;  // head-major
    t->stride[2] = 1;
  }
  return MI_OK;
}

const char *mi_last_error(void) { return mi::last_error_string().c_str(); }

}  // extern "C"
