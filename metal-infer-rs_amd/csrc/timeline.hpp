// Per-workgroup timestamps for the timeline build of the library
// (libmi_attn_timeline.so, compiled with MI_TIMELINE; include/mi_timeline.h).
// The stream-K decode and the prefill kernels record, for each workgroup,
// the constant 100 MHz clock (s_memrealtime) at fixed points of its work and
// the hardware place it ran on (XCC_ID, HW_ID). Without MI_TIMELINE every
// call below compiles to nothing, so the product library is unchanged.
#pragma once

#include <stdint.h>

namespace mi {
namespace dev {

constexpr uint32_t kTimelineFields = 8;    // u64 words per workgroup
constexpr uint32_t kTimelineSlots = 8192;  // workgroups recorded per kernel

// One workgroup's row of stamps; only its thread 0 writes.
struct TimelineRow {
#ifdef MI_TIMELINE
  uint64_t *row = nullptr;
  __device__ void set(uint32_t field, uint64_t value) const {
    if (row != nullptr) row[field] = value;
  }
  __device__ void add(uint32_t field, uint64_t value) const {
    if (row != nullptr) row[field] += value;
  }
  __device__ void now(uint32_t field) const {
    if (row != nullptr) row[field] = __builtin_amdgcn_s_memrealtime();
  }
  __device__ uint64_t clock() const { return __builtin_amdgcn_s_memrealtime(); }
#else
  __device__ void set(uint32_t, uint64_t) const {}
  __device__ void add(uint32_t, uint64_t) const {}
  __device__ void now(uint32_t) const {}
  __device__ uint64_t clock() const { return 0; }
#endif
};

#ifdef MI_TIMELINE
// Starts workgroup `slot`'s row in `buffer` (thread 0 only): field 0 the
// start time, field 1 (HW_ID << 8) | XCC_ID, the rest zero.
__device__ __forceinline__ TimelineRow timeline_start(uint64_t *buffer, uint32_t slot,
                                                      bool writer) {
  TimelineRow r;
  if (!writer || slot >= kTimelineSlots) return r;
  r.row = buffer + (size_t)slot * kTimelineFields;
  uint32_t xcc, hw;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_HW_ID)" : "=s"(hw));
  r.row[0] = __builtin_amdgcn_s_memrealtime();
  r.row[1] = ((uint64_t)hw << 8) | (xcc & 0xffu);
  for (uint32_t f = 2; f < kTimelineFields; ++f) r.row[f] = 0;
  return r;
}
#endif

}  // namespace dev
}  // namespace mi
