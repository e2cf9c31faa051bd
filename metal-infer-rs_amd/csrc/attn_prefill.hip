// MFMA flash prefill. Until the gfx950 MFMA kernel lands, FlashPrefill is
// served by the split-K rows kernel (prefill_supported() == false).
#include "device_common.hpp"
#include "kernels.hpp"

namespace mi {
namespace kernels {

bool prefill_supported(uint32_t) { return false; }

hipError_t launch_prefill(const PrefillParams &, uint32_t, hipStream_t) {
  return hipErrorInvalidValue;
}

}  // namespace kernels
}  // namespace mi
