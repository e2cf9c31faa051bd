// Calibration kernels (include/mi_probe.h): the launch floor of a grid, the
// streaming read rate of a byte count, and the single-sequence decode's
// loads and split-K exchange without its arithmetic. The benchmark times
// them beside the attention kernels; nothing on the attention path calls
// them.
#include "device_common.hpp"
#include "mi_probe.h"

namespace {

using namespace mi::dev;

typedef unsigned u4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint32_t fold(const u4_t &v) { return v.x ^ v.y ^ v.z ^ v.w; }

__device__ __forceinline__ u4_t load_stream(const uint16_t *ptr) {
  return __builtin_nontemporal_load(reinterpret_cast<const u4_t *>(ptr));
}

__device__ __forceinline__ uint32_t wave_fold(uint32_t x) {
#pragma unroll
  for (int mask = 1; mask < 64; mask <<= 1) x ^= __shfl_xor(x, mask, 64);
  return x;
}

__global__ void probe_empty_kernel() {}

constexpr int kReadThreads = 256;
constexpr int kReadUnroll = 8;

__global__ __launch_bounds__(kReadThreads) void probe_read_kernel(const u4_t *src, uint64_t words,
                                                                   uint32_t *sink) {
  const u4_t *base = src + (uint64_t)blockIdx.x * words;
  uint32_t x = 0;
  for (uint64_t i = threadIdx.x; i < words; i += kReadThreads * kReadUnroll) {
    u4_t v[kReadUnroll];
#pragma unroll
    for (int u = 0; u < kReadUnroll; ++u) {
      const uint64_t idx = i + (uint64_t)u * kReadThreads;
      v[u] = idx < words ? __builtin_nontemporal_load(base + idx) : u4_t{0, 0, 0, 0};
    }
#pragma unroll
    for (int u = 0; u < kReadUnroll; ++u) x ^= fold(v[u]);
  }
  x = wave_fold(x);
  if ((threadIdx.x & 63) == 0) sink[blockIdx.x * (kReadThreads / 64) + threadIdx.x / 64] = x;
}

// The attention rows kernel's geometry at head_dim 128: eight waves, a key
// row over 16 lanes (16 bytes each), four rows per wave and four batches of
// 32 rows per load round.
constexpr int kD = 128;
constexpr int kWaves = 8;
constexpr int kThreads = kWaves * 64;
constexpr int kRowsPerRound = kWaves * 4;
constexpr int kBatches = 4;
constexpr int kMergeChunk = 16;
// Words between two KV heads' arrival counters: one 128-byte line each, as
// the attention kernels keep theirs (arrivals on one line queue behind each
// other).
constexpr uint32_t kProbeCounterStride = 32;

struct SplitArgs {
  const uint16_t *k, *v;
  uint64_t head_stride;
  uint32_t group, keys, block_keys;
  float *partial;
  uint32_t *counters;
  uint32_t *out_words;
  uint16_t *out_f16;
};

template <bool PUBLISH>
__global__ __launch_bounds__(kThreads) void probe_split_decode_kernel(const SplitArgs a) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int col = lane & 15, row = wave * 4 + (lane >> 4);
  const uint32_t split = blockIdx.x, splits = gridDim.x, unit = blockIdx.y;
  const uint32_t k0 = split * a.block_keys;
  const uint32_t k1 = min(a.keys, k0 + a.block_keys);  // k0 < keys: the grid is exact
  const uint16_t *kb = a.k + (uint64_t)unit * a.head_stride + col * 8;
  const uint16_t *vb = a.v + (uint64_t)unit * a.head_stride + col * 8;
  uint32_t x = 0;
  for (uint32_t key = k0 + row; key < k1; key += kRowsPerRound * kBatches) {
    u4_t kv[kBatches], vv[kBatches];
#pragma unroll
    for (int u = 0; u < kBatches; ++u) {
      const uint32_t kk = min(key + (uint32_t)(u * kRowsPerRound), k1 - 1);
      kv[u] = load_stream(kb + (uint64_t)kk * kD);
      vv[u] = load_stream(vb + (uint64_t)kk * kD);
    }
#pragma unroll
    for (int u = 0; u < kBatches; ++u) x ^= fold(kv[u]) ^ fold(vv[u]);
  }
  __shared__ uint32_t s_x[kWaves];
  x = wave_fold(x);
  if (lane == 0) s_x[wave] = x;
  __syncthreads();
  uint32_t total = 0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) total ^= s_x[w];
  if constexpr (!PUBLISH) {
    if (tid == 0) a.out_words[unit * splits + split] = total;
    return;
  } else {
    // (max, sum, acc[128]) per query head of the group, finite by construction.
    constexpr int ROW = kD + 2;
    float *part = a.partial + ((size_t)unit * splits + split) * a.group * ROW;
    for (uint32_t idx = tid; idx < a.group * kD; idx += kThreads) {
      const uint32_t g = idx / kD, d = idx % kD;
      store_partial(part + g * ROW + 2 + d, (float)((total >> (d & 15)) & 0xffu));
      if (d == 0) {
        store_partial(part + g * ROW, (float)(total & 7u));
        store_partial(part + g * ROW + 1, 1.0f + (float)(total & 3u));
      }
    }
    __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
    __shared__ uint32_t s_last;
    __syncthreads();
    if (tid == 0) {
      const bool last = arrive(a.counters + (size_t)unit * kProbeCounterStride) == splits - 1;
      if (last) {
        acquire_partials();
        __hip_atomic_store(a.counters + (size_t)unit * kProbeCounterStride, 0u, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
      }
      s_last = last;
    }
    __syncthreads();
    if (s_last == 0) return;
    const float *base = a.partial + (size_t)unit * splits * a.group * ROW;
    for (uint32_t idx = tid; idx < a.group * kD; idx += kThreads) {
      const uint32_t g = idx / kD, d = idx % kD;
      float M = -INFINITY, Ls = 0.0f, As = 0.0f;
      for (uint32_t s0 = 0; s0 < splits; s0 += kMergeChunk) {
        float m[kMergeChunk], l[kMergeChunk], v[kMergeChunk];
#pragma unroll
        for (int i = 0; i < kMergeChunk; ++i) {
          const float *ps = base + (size_t)(min(s0 + i, splits - 1) * a.group + g) * ROW;
          m[i] = load_partial(ps);
          l[i] = load_partial(ps + 1);
          v[i] = load_partial(ps + 2 + d);
          if (s0 + i >= splits) m[i] = -INFINITY;
        }
        float cm = M;
#pragma unroll
        for (int i = 0; i < kMergeChunk; ++i) cm = fmaxf(cm, m[i]);
        const float r = M == -INFINITY ? 0.0f : exp2_raw(M - cm);
        Ls *= r;
        As *= r;
#pragma unroll
        for (int i = 0; i < kMergeChunk; ++i) {
          const float f = m[i] == -INFINITY ? 0.0f : exp2_raw(m[i] - cm);
          Ls = fmaf(l[i], f, Ls);
          As = fmaf(v[i], f, As);
        }
        M = cm;
      }
      a.out_f16[((size_t)unit * a.group + g) * kD + d] = f32_to_f16(As / Ls);
    }
  }
}

}  // namespace

extern "C" {

int32_t mi_probe_empty(void *stream, uint32_t grid_x, uint32_t grid_y, uint32_t threads) {
  if (grid_x == 0 || grid_y == 0 || threads == 0 || threads > 1024) return hipErrorInvalidValue;
  hipLaunchKernelGGL(probe_empty_kernel, dim3(grid_x, grid_y), dim3(threads), 0,
                     static_cast<hipStream_t>(stream));
  return hipGetLastError();
}

int32_t mi_probe_read(void *stream, const void *src, uint64_t bytes_per_workgroup,
                      uint32_t workgroups, uint32_t *sink) {
  if (src == nullptr || sink == nullptr || workgroups == 0 || bytes_per_workgroup == 0 ||
      bytes_per_workgroup % 16 != 0 || reinterpret_cast<uintptr_t>(src) % 16 != 0)
    return hipErrorInvalidValue;
  hipLaunchKernelGGL(probe_read_kernel, dim3(workgroups), dim3(kReadThreads), 0,
                     static_cast<hipStream_t>(stream), static_cast<const u4_t *>(src),
                     bytes_per_workgroup / 16, sink);
  return hipGetLastError();
}

int32_t mi_probe_split_decode(void *stream, const uint16_t *k, const uint16_t *v,
                              uint64_t head_stride, uint32_t kv_heads, uint32_t group,
                              uint32_t keys, uint32_t block_keys, int32_t publish,
                              float *partial, uint32_t *counters, uint32_t *out_words,
                              uint16_t *out_f16) {
  if (k == nullptr || v == nullptr || kv_heads == 0 || kv_heads > 65535 || group == 0 ||
      group > 8 || keys == 0 || block_keys == 0 || head_stride < (uint64_t)keys * kD ||
      reinterpret_cast<uintptr_t>(k) % 16 != 0 || reinterpret_cast<uintptr_t>(v) % 16 != 0)
    return hipErrorInvalidValue;
  if (publish != 0 ? (partial == nullptr || counters == nullptr || out_f16 == nullptr)
                   : out_words == nullptr)
    return hipErrorInvalidValue;
  const uint32_t splits = (keys + block_keys - 1) / block_keys;
  const SplitArgs args{k, v, head_stride, group, keys, block_keys, partial, counters, out_words,
                       out_f16};
  const dim3 grid(splits, kv_heads);
  if (publish != 0)
    hipLaunchKernelGGL(probe_split_decode_kernel<true>, grid, dim3(kThreads), 0,
                       static_cast<hipStream_t>(stream), args);
  else
    hipLaunchKernelGGL(probe_split_decode_kernel<false>, grid, dim3(kThreads), 0,
                       static_cast<hipStream_t>(stream), args);
  return hipGetLastError();
}

}  // extern "C"
