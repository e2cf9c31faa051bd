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
#include <mutex>
#include <vector>

#include "runtime.hpp"

namespace mi {
namespace {

static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

std::mutex g_lock;
std::vector<void *> g_device_scratch;  // indexed by HIP device

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

}  // namespace mi
