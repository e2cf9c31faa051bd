// Fixed scratch of the no-allocation entry point
// (mi_attention_decode_batched_noalloc): the split-K partials of a batched
// decode live in a file-scope device array instead of a batch arena lease,
// so the call itself never allocates device memory.
//
// The array exists once per GPU that loads this library's code object and
// stays allocated until the process ends. In host code its name is only a
// host-side stand-in: the device address is resolved once per device with
// hipGetSymbolAddress (with that device current, at context creation) and
// every host use (kernel arguments) goes through that address.
//
// Every context on a GPU shares its array. A call from one context while
// another context's eager call may still be running on its own stream is
// refused (MI_ERR_RESOURCE) rather than left to overwrite that call's
// partials: each eager call records an event after its launches, and the next
// call from a different context checks it. Calls recorded into a graph are
// not tracked.
#include <mutex>
#include <vector>

#include "runtime.hpp"

namespace mi {
namespace {

static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

std::mutex g_lock;
std::vector<void *> g_device_scratch;  // indexed by HIP device
// The context whose calls last used each device's array, and the event its
// stream records after each eager call (indexed by HIP device).
struct Owner {
  const Context *ctx = nullptr;
  hipEvent_t done = nullptr;
};
std::vector<Owner> g_owner;

}  // namespace

mi_status noalloc_init(int device) {
  if (device < 0) return fail(MI_ERR_NO_DEVICE, "HIP device index out of range");
  std::lock_guard<std::mutex> guard(g_lock);
  if ((size_t)device < g_device_scratch.size() && g_device_scratch[device] != nullptr)
    return MI_OK;
  void *ptr = nullptr;
  const hipError_t err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
  if (err != hipSuccess || ptr == nullptr)
    return hip_fail(MI_ERR_RESOURCE, "no-allocation scratch address", err);
  if ((size_t)device >= g_device_scratch.size()) g_device_scratch.resize(device + 1, nullptr);
  g_device_scratch[device] = ptr;
  return MI_OK;
}

void *noalloc_scratch(int device) {
  std::lock_guard<std::mutex> guard(g_lock);
  if (device < 0 || (size_t)device >= g_device_scratch.size()) return nullptr;
  return g_device_scratch[device];
}

mi_status noalloc_acquire(Context *ctx, bool capturing) {
  std::lock_guard<std::mutex> guard(g_lock);
  if ((size_t)ctx->device >= g_owner.size()) g_owner.resize(ctx->device + 1);
  Owner &owner = g_owner[ctx->device];
  if (owner.ctx != nullptr && owner.ctx != ctx && owner.done != nullptr && !capturing) {
    const hipError_t state = hipEventQuery(owner.done);
    if (state == hipErrorNotReady)
      return fail(MI_ERR_RESOURCE,
                  "the no-allocation scratch is in use by another context's unfinished call");
  }
  owner.ctx = ctx;
  owner.done = ctx->noalloc_done;
  return MI_OK;
}

void noalloc_mark(Context *ctx, bool capturing) {
  if (!capturing) (void)hipEventRecord(ctx->noalloc_done, ctx->stream);
}

void noalloc_forget(const Context *ctx) {
  std::lock_guard<std::mutex> guard(g_lock);
  for (Owner &owner : g_owner)
    if (owner.ctx == ctx) owner = Owner{};
}

}  // namespace mi
