// Device helpers for the CDNA4 (gfx950) kernels: f16 vectors, DPP row
// reductions, the raw exp2 instruction, MFMA operand packing and the gfx950
// direct-to-LDS and transposed LDS accesses.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mi {
namespace dev {

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef __fp16 fp16x2_t __attribute__((ext_vector_type(2)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef float float16_t __attribute__((ext_vector_type(16)));

__device__ __forceinline__ float f16_to_f32(uint16_t bits) {
  return (float)__builtin_bit_cast(_Float16, bits);
}

// Round-to-nearest-even f32 -> f16 (v_cvt_f16_f32 rounds by the mode
// register, which HIP leaves at RNE).
__device__ __forceinline__ uint16_t f32_to_f16(float value) {
  return __builtin_bit_cast(uint16_t, (_Float16)value);
}

// v_exp_f32: 2^x, exact at 0, 0 at -inf.
__device__ __forceinline__ float exp2_raw(float x) {
  return __builtin_amdgcn_exp2f(x);
}

template <int CTRL>
__device__ __forceinline__ float dpp_f32(float x) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL,
                                         0xf, 0xf, false));
}

// DPP controls: quad_perm xor-1 / xor-2, row rotate by 4 / 8 within the
// 16-lane row.
constexpr int kDppQuadXor1 = 0xB1;
constexpr int kDppQuadXor2 = 0x4E;
constexpr int kDppRowRor4 = 0x124;
constexpr int kDppRowRor8 = 0x128;

// Sum over each aligned group of N lanes (N a power of two <= 64); every
// lane of the group receives the total.
template <int N>
__device__ __forceinline__ float group_sum(float x) {
  if constexpr (N >= 2) x += dpp_f32<kDppQuadXor1>(x);
  if constexpr (N >= 4) x += dpp_f32<kDppQuadXor2>(x);
  if constexpr (N >= 8) x += __shfl_xor(x, 4, 64);
  if constexpr (N >= 16) x += __shfl_xor(x, 8, 64);
  if constexpr (N >= 32) x += __shfl_xor(x, 16, 64);
  if constexpr (N >= 64) x += __shfl_xor(x, 32, 64);
  return x;
}

// 16-lane row sum using only DPP (rotations make every lane hold the
// total, as for group_sum<16>).
__device__ __forceinline__ float row16_sum(float x) {
  x += dpp_f32<kDppQuadXor1>(x);
  x += dpp_f32<kDppQuadXor2>(x);
  x += dpp_f32<kDppRowRor4>(x);
  x += dpp_f32<kDppRowRor8>(x);
  return x;
}

template <int N>
__device__ __forceinline__ float lane_group_sum(float x) {
  if constexpr (N == 16) {
    return row16_sum(x);
  } else if constexpr (N == 32) {
    x = row16_sum(x);
    return x + __shfl_xor(x, 16, 64);
  } else {
    return group_sum<N>(x);
  }
}

// f16x2 dot product accumulated in f32 (v_dot2_f32_f16).
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(fp16x2_t, a),
                                __builtin_bit_cast(fp16x2_t, b), c, false);
}

// Eight f16 values of one MFMA operand register quad.
typedef __fp16 h8_t __attribute__((ext_vector_type(8)));
__device__ __forceinline__ h8_t as_h8(uint4 v) { return __builtin_bit_cast(h8_t, v); }

// v_cvt_pk_f16_f32: two f32 -> packed f16, round to nearest even.
__device__ __forceinline__ uint32_t pack_f16x2(float lo, float hi) {
  typedef float f2_t __attribute__((ext_vector_type(2)));
  const f2_t v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, half2_t));
}

// gfx950 direct global->LDS load of 16 bytes per lane: lane L's bytes land
// at lds + 16 L (lds is wave-uniform).
__device__ __forceinline__ void load_lds16(const uint16_t *global, uint16_t *lds) {
  __builtin_amdgcn_global_load_lds(global, lds, 16, 0, 0);
}
// The same with the non-temporal hint (cache policy 2: the `nt` bit), for
// data read once, as a decode's cache rows are.
__device__ __forceinline__ void load_lds16_nt(const uint16_t *global, uint16_t *lds) {
  __builtin_amdgcn_global_load_lds(global, lds, 16, 0, 2);
}

// gfx950 ds_read_b64_tr_b16: within each 16-lane group, output lane 4a + b,
// element j receives half b of the 8 bytes addressed by lane a + 4j.
__device__ __forceinline__ uint2 read_tr16(const uint16_t *lds) {
  typedef short v4s_t __attribute__((ext_vector_type(4)));
  const v4s_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (v4s_t __attribute__((address_space(3))) *)(lds));
  return __builtin_bit_cast(uint2, v);
}

__device__ __forceinline__ float lo_f16(uint32_t packed) {
  return (float)__builtin_bit_cast(half2_t, packed).x;
}
__device__ __forceinline__ float hi_f16(uint32_t packed) {
  return (float)__builtin_bit_cast(half2_t, packed).y;
}

// Device-scope (agent) relaxed accesses: stores write through to the
// device-coherent level and loads read from it, so partial results pass
// between workgroups on different XCDs of one launch without a cache-wide
// fence. A writer waits for its stores (kWaitVmcnt0) before signalling.
__device__ __forceinline__ void store_coherent(float *ptr, float v) {
  __hip_atomic_store(ptr, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_coherent2(float *ptr, float a, float b) {
  const uint64_t bits = (uint64_t)__float_as_uint(a) | ((uint64_t)__float_as_uint(b) << 32);
  __hip_atomic_store(reinterpret_cast<uint64_t *>(ptr), bits, __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float2 load_coherent2(const float *ptr) {
  const uint64_t bits =
      __hip_atomic_load(reinterpret_cast<uint64_t *>(const_cast<float *>(ptr)),
                        __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return make_float2(__uint_as_float((uint32_t)bits), __uint_as_float((uint32_t)(bits >> 32)));
}
// s_waitcnt vmcnt(0) (expcnt and lgkmcnt left at their maxima): every
// vector-memory access of this wave, stores included, has completed.
constexpr int kWaitVmcnt0 = 0x0F70;

// Split partials passed between workgroups of one launch ("the last split
// to arrive merges"):
//  - every thread stores its part of the partial with agent-scope atomic
//    stores (store_partial*), waits for them to complete (s_waitcnt
//    vmcnt(0)), and the workgroup meets at a barrier;
//  - one thread counts the arrival with an agent-scope read-modify-write on
//    the unit's counter (arrive);
//  - the thread that sees itself last issues an agent-scope ACQUIRE fence
//    (acquire_partials), then the workgroup meets at a barrier and reads the
//    other splits' partials with agent-scope atomic loads (load_partial*).
// The arrival carries no release fence. On gfx950 (the HIP memory model as
// LLVM implements it for gfx942 and later) an agent-scope release is an L2
// writeback (buffer_wbl2 sc1) followed by s_waitcnt vmcnt(0). The writeback
// is there for plain stores, which may sit dirty in the writer's XCD L2;
// everything published here is written with agent-scope atomic stores
// (sc1: written through to the device-coherent level), and the writer has
// already waited for their completion before it arrives, so the writeback
// would only flush unrelated lines. Measured on MI355X (same box, c3
// prefill with 3 key splits): 42.2-42.6 us per call with the release, 39.3-
// 40.0 us without it and with the acquire kept, 39.0-39.5 us with neither.
// The merger's acquire (an L2 invalidate) is cheap and is kept.
__device__ __forceinline__ void store_partial(float *ptr, float v) { store_coherent(ptr, v); }
__device__ __forceinline__ void store_partial2(float *ptr, float a, float b) {
  store_coherent2(ptr, a, b);
}
__device__ __forceinline__ float load_partial(const float *ptr) {
  return __hip_atomic_load(const_cast<float *>(ptr), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float2 load_partial2(const float *ptr) { return load_coherent2(ptr); }
// Two packed words (f16 pairs) of a partial, bits unchanged.
__device__ __forceinline__ void store_partial_words(float *ptr, uint32_t a, uint32_t b) {
  store_coherent2(ptr, __uint_as_float(a), __uint_as_float(b));
}
__device__ __forceinline__ uint2 load_partial_words(const float *ptr) {
  const float2 v = load_coherent2(ptr);
  return make_uint2(__float_as_uint(v.x), __float_as_uint(v.y));
}
// Returns the counter's previous value. Call after the workgroup's partial
// stores have completed (s_waitcnt vmcnt(0)) and it has met at a barrier.
__device__ __forceinline__ uint32_t arrive(uint32_t *counter) {
  return __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void acquire_partials() {
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
}

}  // namespace dev
}  // namespace mi
