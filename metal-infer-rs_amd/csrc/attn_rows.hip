// Split-K ("flash-decoding") attention over KV rows, for any GQA ratio and
// any power-of-two head_dim <= 256.
//
// Replaces the reference's row-wise kernels: attention_tiled_f16
// (transformer.metal:1614-1665), attention_decode_f16 (:1824-1909), the
// FlashDecode partial kernels (:1911-2249) and their reduce kernels
// (:2251-2316). Semantics are the reference's online softmax; the work
// decomposition is MI355X-first:
//  - one workgroup per (sequence*token, KV head, head chunk, key split), so
//    each K/V row is fetched once for all query heads of its GQA group;
//  - a key row of D halves is spread over D/8 lanes, each issuing one
//    128-bit load, so a wave reads 64 * 16 B contiguous bytes per load;
//  - per-row dot products reduce with DPP inside a 16-lane row;
//  - scores and the softmax stay in f32 (v_exp_f32 on log2-scaled scores);
//  - the split-K merge is fused: the last workgroup of a (row, KV head) to
//    finish merges every split's (max, sum, acc[D]) partial, so a decode is
//    one launch. Arrival counters are reset by that workgroup, so they are
//    zero between launches without any memset.
#include "device_common.hpp"
#include "kernels.hpp"

namespace mi {
namespace kernels {
namespace {

using namespace mi::dev;

template <int VEC>
struct Vec {
  uint32_t w[VEC >= 2 ? VEC / 2 : 1];
};

template <int VEC>
__device__ __forceinline__ Vec<VEC> load_vec(const uint16_t *ptr) {
  Vec<VEC> r;
  if constexpr (VEC == 8) {
    uint4 x = *reinterpret_cast<const uint4 *>(ptr);
    r.w[0] = x.x, r.w[1] = x.y, r.w[2] = x.z, r.w[3] = x.w;
  } else if constexpr (VEC == 4) {
    uint2 x = *reinterpret_cast<const uint2 *>(ptr);
    r.w[0] = x.x, r.w[1] = x.y;
  } else if constexpr (VEC == 2) {
    r.w[0] = *reinterpret_cast<const uint32_t *>(ptr);
  } else {
    r.w[0] = *ptr;
  }
  return r;
}

template <int VEC>
__device__ __forceinline__ Vec<VEC> zero_vec() {
  Vec<VEC> r;
#pragma unroll
  for (int i = 0; i < (VEC >= 2 ? VEC / 2 : 1); ++i) r.w[i] = 0;
  return r;
}

template <int VEC>
__device__ __forceinline__ float elem(const Vec<VEC> &v, int i) {
  return (i & 1) ? hi_f16(v.w[i >> 1]) : lo_f16(v.w[i >> 1]);
}

template <int VEC>
__device__ __forceinline__ float dot(const Vec<VEC> &a, const Vec<VEC> &b) {
  if constexpr (VEC == 1) {
    return lo_f16(a.w[0]) * lo_f16(b.w[0]);
  } else {
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < VEC / 2; ++i) s = dot2(a.w[i], b.w[i], s);
    return s;
  }
}

template <int D, int WAVES, int GC>
__global__ __launch_bounds__(WAVES * 64) void attn_rows_kernel(
    const RowsParams p) {
  constexpr int VEC = D >= 8 ? 8 : D;  // halves per lane per key row
  constexpr int LPR = D / VEC;         // lanes per key row
  constexpr int RPW = 64 / LPR;        // key rows per wave per step
  constexpr int R = WAVES * RPW;       // key rows per workgroup per step
  constexpr int U = D >= 64 ? 4 : (D >= 16 ? 2 : 1);  // steps per iteration
  constexpr int THREADS = WAVES * 64;

  __shared__ float s_m[WAVES][GC];
  __shared__ float s_l[WAVES][GC];
  __shared__ float s_acc[WAVES][GC][D];
  __shared__ int s_last;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int col = lane % LPR;
  const int rloc = lane / LPR;
  const int row = wave * RPW + rloc;

  const uint32_t split = blockIdx.x;
  const uint32_t kvh = blockIdx.y / p.head_chunks;
  const uint32_t hc = blockIdx.y % p.head_chunks;
  const uint32_t b = blockIdx.z / p.tokens;
  const uint32_t t = blockIdx.z % p.tokens;
  const uint32_t unit = blockIdx.z * gridDim.y + blockIdx.y;

  uint32_t len = p.kv_length;
  uint32_t off = p.query_offset;
  if (p.lengths != nullptr) {
    len = min(p.lengths[b], p.kv_length);
    off = len >= p.tokens ? len - p.tokens : 0u;
  }
  // transformer.metal:1589-1590 (causal window of query token t).
  const uint64_t window = (uint64_t)off + t + 1;
  const uint32_t available =
      p.causal != 0 ? (uint32_t)min((uint64_t)len, window) : len;
  const uint32_t nsplits = (available + p.block_keys - 1) / p.block_keys;
  const uint32_t h0 = kvh * p.group + hc * GC;
  uint16_t *out = p.out + (int64_t)b * p.o_seq + (int64_t)t * p.o_tok +
                  (int64_t)h0 * p.o_head;

  if (available == 0) {
    // No visible key: the reference divides 0 by 0.
    if (split == 0)
      for (int idx = tid; idx < GC * D; idx += THREADS)
        out[(idx / D) * p.o_head + idx % D] = 0x7e00;
    return;
  }
  if (split >= nsplits) return;

  const uint32_t k0 = split * p.block_keys;
  const uint32_t k1 = min(available, k0 + p.block_keys);

  Vec<VEC> qv[GC];
  {
    const uint16_t *qb = p.q + (int64_t)b * p.q_seq + (int64_t)t * p.q_tok +
                         (int64_t)h0 * p.q_head + col * VEC;
#pragma unroll
    for (int g = 0; g < GC; ++g) qv[g] = load_vec<VEC>(qb + g * p.q_head);
  }
  const uint16_t *kb =
      p.k + (int64_t)b * p.k_seq + (int64_t)kvh * p.k_head + col * VEC;
  const uint16_t *vb =
      p.v + (int64_t)b * p.v_seq + (int64_t)kvh * p.v_head + col * VEC;

  float m[GC], l[GC], acc[GC][VEC];
#pragma unroll
  for (int g = 0; g < GC; ++g) {
    m[g] = -INFINITY;
    l[g] = 0.0f;
#pragma unroll
    for (int i = 0; i < VEC; ++i) acc[g][i] = 0.0f;
  }

  // Every lane of a key row shares `row`, so the DPP reductions below only
  // ever combine lanes with identical trip counts.
  for (uint32_t key = k0 + row; key < k1; key += R * U) {
    Vec<VEC> kv[U], vv[U];
    bool valid[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t kk = key + u * R;
      valid[u] = kk < k1;
      if (valid[u]) {
        kv[u] = load_vec<VEC>(kb + (int64_t)kk * p.k_pos);
        vv[u] = load_vec<VEC>(vb + (int64_t)kk * p.v_pos);
      } else {
        kv[u] = zero_vec<VEC>();
        vv[u] = zero_vec<VEC>();
      }
    }
#pragma unroll
    for (int g = 0; g < GC; ++g) {
      float s[U];
      float mx = m[g];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        s[u] = lane_group_sum<LPR>(dot<VEC>(qv[g], kv[u])) * p.scale_log2;
        s[u] = valid[u] ? s[u] : -INFINITY;
        mx = fmaxf(mx, s[u]);
      }
      // u = 0 is always valid here, so mx is finite.
      const float alpha = exp2_raw(m[g] - mx);
      float pu[U];
      float ps = 0.0f;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        pu[u] = exp2_raw(s[u] - mx);
        ps += pu[u];
      }
      l[g] = l[g] * alpha + ps;
#pragma unroll
      for (int i = 0; i < VEC; ++i) {
        float a = acc[g][i] * alpha;
#pragma unroll
        for (int u = 0; u < U; ++u) a = fmaf(pu[u], elem<VEC>(vv[u], i), a);
        acc[g][i] = a;
      }
      m[g] = mx;
    }
  }

  // Merge the key rows of this wave (lanes that differ in their row bits).
#pragma unroll
  for (int g = 0; g < GC; ++g) {
    float M = m[g];
#pragma unroll
    for (int mask = LPR; mask < 64; mask <<= 1)
      M = fmaxf(M, __shfl_xor(M, mask, 64));
    const float f = m[g] == -INFINITY ? 0.0f : exp2_raw(m[g] - M);
    float lw = l[g] * f;
#pragma unroll
    for (int mask = LPR; mask < 64; mask <<= 1) lw += __shfl_xor(lw, mask, 64);
#pragma unroll
    for (int i = 0; i < VEC; ++i) {
      float a = acc[g][i] * f;
#pragma unroll
      for (int mask = LPR; mask < 64; mask <<= 1) a += __shfl_xor(a, mask, 64);
      acc[g][i] = a;
    }
    m[g] = M;
    l[g] = lw;
  }
  if (rloc == 0) {
#pragma unroll
    for (int g = 0; g < GC; ++g) {
      if (col == 0) {
        s_m[wave][g] = m[g];
        s_l[wave][g] = l[g];
      }
#pragma unroll
      for (int i = 0; i < VEC; ++i) s_acc[wave][g][col * VEC + i] = acc[g][i];
    }
  }
  __syncthreads();

  // Merge the waves; write the output (one split) or this split's partial.
  const bool direct = nsplits == 1;
  float *part =
      p.partial + ((size_t)unit * p.max_splits + split) * GC * (D + 2);
  for (int idx = tid; idx < GC * D; idx += THREADS) {
    const int g = idx / D, d = idx % D;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < WAVES; ++w) M = fmaxf(M, s_m[w][g]);
    float L = 0.0f, A = 0.0f;
#pragma unroll
    for (int w = 0; w < WAVES; ++w) {
      const float f = s_m[w][g] == -INFINITY ? 0.0f : exp2_raw(s_m[w][g] - M);
      L += s_l[w][g] * f;
      A += s_acc[w][g][d] * f;
    }
    if (direct) {
      out[g * p.o_head + d] = f32_to_f16(A / L);
    } else {
      part[g * (D + 2) + 2 + d] = A;
      if (d == 0) {
        part[g * (D + 2)] = M;
        part[g * (D + 2) + 1] = L;
      }
    }
  }
  if (direct) return;

  // Publish the partial, count arrivals; the last split merges.
  __threadfence();
  __syncthreads();
  if (tid == 0) {
    const unsigned prev = atomicAdd(&p.counters[unit], 1u);
    s_last = prev == nsplits - 1;
  }
  __syncthreads();
  if (!s_last) return;
  __threadfence();
  const float *base = p.partial + (size_t)unit * p.max_splits * GC * (D + 2);
  for (int idx = tid; idx < GC * D; idx += THREADS) {
    const int g = idx / D, d = idx % D;
    float M = -INFINITY;
    for (uint32_t s = 0; s < nsplits; ++s)
      M = fmaxf(M, base[(s * GC + g) * (D + 2)]);
    float L = 0.0f, A = 0.0f;
    for (uint32_t s = 0; s < nsplits; ++s) {
      const float *ps = base + (s * GC + g) * (D + 2);
      const float f = exp2_raw(ps[0] - M);
      L += ps[1] * f;
      A += ps[2 + d] * f;
    }
    out[g * p.o_head + d] = f32_to_f16(A / L);
  }
  if (tid == 0) atomicExch(&p.counters[unit], 0u);
}

template <int D, int WAVES>
hipError_t launch_rows_dw(const RowsParams &p, uint32_t chunk,
                          hipStream_t stream) {
  const dim3 grid(p.max_splits, p.kv_heads * p.head_chunks,
                  p.batch * p.tokens);
  const dim3 block(WAVES * 64);
  switch (chunk) {
    case 8:
      attn_rows_kernel<D, WAVES, 8><<<grid, block, 0, stream>>>(p);
      break;
    case 4:
      attn_rows_kernel<D, WAVES, 4><<<grid, block, 0, stream>>>(p);
      break;
    case 2:
      attn_rows_kernel<D, WAVES, 2><<<grid, block, 0, stream>>>(p);
      break;
    case 1:
      attn_rows_kernel<D, WAVES, 1><<<grid, block, 0, stream>>>(p);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <int D>
hipError_t launch_rows_d(const RowsParams &p, uint32_t waves, uint32_t chunk,
                         hipStream_t stream) {
  if (waves == 4) return launch_rows_dw<D, 4>(p, chunk, stream);
  if (waves == 2) return launch_rows_dw<D, 2>(p, chunk, stream);
  return hipErrorInvalidValue;
}

}  // namespace

uint32_t rows_chunk(uint32_t group) {
  for (uint32_t c : {8u, 4u, 2u}) if (group % c == 0) return c;
  return 1;
}

hipError_t launch_rows(const RowsParams &p, uint32_t head_dim, uint32_t waves,
                       uint32_t chunk, hipStream_t stream) {
  switch (head_dim) {
    case 1: return launch_rows_d<1>(p, waves, chunk, stream);
    case 2: return launch_rows_d<2>(p, waves, chunk, stream);
    case 4: return launch_rows_d<4>(p, waves, chunk, stream);
    case 8: return launch_rows_d<8>(p, waves, chunk, stream);
    case 16: return launch_rows_d<16>(p, waves, chunk, stream);
    case 32: return launch_rows_d<32>(p, waves, chunk, stream);
    case 64: return launch_rows_d<64>(p, waves, chunk, stream);
    case 128: return launch_rows_d<128>(p, waves, chunk, stream);
    case 256: return launch_rows_d<256>(p, waves, chunk, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace kernels
}  // namespace mi
