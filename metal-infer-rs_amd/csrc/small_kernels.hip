// The exact Reference attention, the KV-cache append and the fused
// QK-RMSNorm + RoPE + K-append kernels.
#include "device_common.hpp"
#include "kernels.hpp"

namespace mi {
namespace kernels {
namespace {

using namespace mi::dev;

// AttentionKind::Reference: the exact two-pass softmax of
// attention_reference_f16 (transformer.metal:1579-1612), one workgroup per
// (query token, query head). Each key's score is summed over x in
// ascending order (one thread per key), pass 2 runs one thread per output
// dimension over keys in ascending order, and contraction is off, so every
// f32 operation is the one the reference's source spells out.
__global__ __launch_bounds__(256) void attn_naive_kernel(NaiveParams p,
                                                         uint32_t row_begin) {
#pragma clang fp contract(off)
  extern __shared__ float s_scores[];
  __shared__ float s_red[256];
  const uint32_t row = row_begin + blockIdx.x;
  const uint32_t qi = row / p.q_heads;
  const uint32_t h = row % p.q_heads;
  const uint32_t kvh = h / (p.q_heads / p.kv_heads);
  const uint64_t window = (uint64_t)p.query_offset + qi + 1;
  const uint32_t available =
      p.causal != 0 ? (uint32_t)min((uint64_t)p.kv_length, window)
                    : p.kv_length;
  float *scores = p.kv_length <= kNaiveLdsKeys
                      ? s_scores
                      : p.scores + (size_t)blockIdx.x * p.kv_length;
  const uint16_t *q = p.q + (int64_t)qi * p.q_tok + (int64_t)h * p.q_head;
  const uint16_t *k = p.k + (int64_t)kvh * p.k_head;
  const uint16_t *v = p.v + (int64_t)kvh * p.v_head;

  for (uint32_t j = threadIdx.x; j < available; j += blockDim.x) {
    const uint16_t *kr = k + (int64_t)j * p.k_pos;
    float score = 0.0f;
    for (uint32_t x = 0; x < p.head_dim; ++x)
      score += f16_to_f32(q[x]) * f16_to_f32(kr[x]);
    scores[j] = score;
  }
  __syncthreads();
  float local = -INFINITY;
  for (uint32_t j = threadIdx.x; j < available; j += blockDim.x)
    local = fmaxf(local, scores[j] * p.scale);
  s_red[threadIdx.x] = local;
  __syncthreads();
  for (uint32_t stride = blockDim.x / 2; stride > 0; stride >>= 1) {
    if (threadIdx.x < stride)
      s_red[threadIdx.x] =
          fmaxf(s_red[threadIdx.x], s_red[threadIdx.x + stride]);
    __syncthreads();
  }
  const float maximum = s_red[0];
  for (uint32_t d = threadIdx.x; d < p.head_dim; d += blockDim.x) {
    float denominator = 0.0f, numerator = 0.0f;
    for (uint32_t j = 0; j < available; ++j) {
      const float probability = expf(scores[j] * p.scale - maximum);
      denominator += probability;
      numerator += probability * f16_to_f32(v[(int64_t)j * p.v_pos + d]);
    }
    p.out[(int64_t)qi * p.o_tok + (int64_t)h * p.o_head + d] =
        f32_to_f16(numerator / denominator);
  }
}

// KV append (copy_kv_f16, transformer.metal:2318-2325) into any cache
// layout: each thread moves 8 halves (16 B) when rows allow it.
template <int VEC>
__global__ __launch_bounds__(256) void copy_kv_kernel(CopyKvParams p) {
  const uint32_t per_row = p.head_dim / VEC;
  const uint64_t total = (uint64_t)p.tokens * p.heads * per_row;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
       i < total; i += (uint64_t)gridDim.x * blockDim.x) {
    const uint32_t c = (uint32_t)(i % per_row);
    const uint64_t r = i / per_row;
    const uint32_t h = (uint32_t)(r % p.heads);
    const uint32_t t = (uint32_t)(r / p.heads);
    const uint16_t *src =
        p.src + (int64_t)t * p.s_tok + (int64_t)h * p.s_head + c * VEC;
    uint16_t *dst = p.dst + (int64_t)(p.offset + t) * p.d_pos +
                    (int64_t)h * p.d_head + c * VEC;
    if constexpr (VEC == 8) {
      *reinterpret_cast<uint4 *>(dst) = *reinterpret_cast<const uint4 *>(src);
    } else {
      *dst = *src;
    }
  }
}

// qk_norm_rope_cache_f16 (transformer.metal:1533-1577): one wave per
// (token, head) row; query rows first, then key rows, which are written
// straight into the cache at position offset + token. With p.v set, a last
// group of rows copies the value rows into their cache (copy_kv_f16,
// transformer.metal:2318-2325) in the same launch.
__global__ __launch_bounds__(64) void qk_norm_rope_kernel(QkNormRopeParams p) {
#pragma clang fp contract(off)
  const uint32_t group = blockIdx.x;
  const uint32_t qk_rows = p.tokens * (p.q_heads + p.kv_heads);
  if (group >= qk_rows) {
    const uint32_t row = group - qk_rows;
    const uint32_t token = row / p.kv_heads, head = row % p.kv_heads;
    const uint16_t *src = p.v + (int64_t)token * p.v_tok + (int64_t)head * p.v_head;
    uint16_t *dst = p.v_cache + (int64_t)(p.offset + token) * p.vc_pos + (int64_t)head * p.vc_head;
    for (uint32_t i = threadIdx.x; i < p.head_dim; i += 64) dst[i] = src[i];
    return;
  }
  const uint32_t query_rows = p.tokens * p.q_heads;
  const bool is_query = group < query_rows;
  const uint32_t row = is_query ? group : group - query_rows;
  const uint32_t heads = is_query ? p.q_heads : p.kv_heads;
  const uint32_t token = row / heads;
  const uint32_t head = row % heads;
  const uint16_t *input =
      is_query ? p.q + (int64_t)token * p.q_tok + (int64_t)head * p.q_head
               : p.k + (int64_t)token * p.k_tok + (int64_t)head * p.k_head;
  const uint16_t *weight = is_query ? p.q_weight : p.k_weight;
  uint16_t *output =
      is_query
          ? p.q_out + (int64_t)token * p.qo_tok + (int64_t)head * p.qo_head
          : p.cache + (int64_t)(p.offset + token) * p.c_pos +
                (int64_t)head * p.c_head;
  const uint32_t lane = threadIdx.x;
  float sum = 0.0f;
  for (uint32_t i = lane; i < p.head_dim; i += 64) {
    const float value = f16_to_f32(input[i]);
    sum += value * value;
  }
  for (int mask = 32; mask > 0; mask >>= 1) sum += __shfl_xor(sum, mask, 64);
  const float scale = 1.0f / sqrtf(sum / (float)p.head_dim + p.epsilon);
  const uint32_t half = p.head_dim / 2;
  for (uint32_t pair = lane; pair < half; pair += 64) {
    const uint32_t second = pair + half;
    const float x = f16_to_f32(input[pair]) * scale * f16_to_f32(weight[pair]);
    const float y =
        f16_to_f32(input[second]) * scale * f16_to_f32(weight[second]);
    const float frequency =
        powf(p.theta, -(float)(pair * 2) / (float)p.head_dim);
    const float angle = (float)(token + p.offset) * frequency;
    const float c = cosf(angle), s = sinf(angle);
    output[pair] = f32_to_f16(x * c - y * s);
    output[second] = f32_to_f16(x * s + y * c);
  }
}

// The same operations for head_dim HD in {128, 256} with 16-byte aligned
// rows, HPW head rows of one token per wave. A row is spread over 16 lanes:
// lane l of the row's 16-lane group holds elements EPL l .. EPL l + EPL - 1
// (EPL = HD / 16, one or two 16-byte accesses), so lanes 0-7 hold the first
// half and lanes 8-15 the matching second half. A pair's partner is then lane
// l ^ 8 (a DPP rotate by 8 within the group), the row sum is four DPP
// rotate-and-add steps (each lane adds the same values in the same order, so
// all 16 agree), and each wave step covers four rows, one per group. The
// angles depend on (token, pair) only: the wave computes each once (pair
// lane + 64 a) and shares them through LDS. All of a wave's rows are loaded
// before any is written. Per element the f32 steps are the generic kernel's:
// x c - y s as x c + y (-s) and x s + y c as y c + x s, both exact
// rewrites. The row sum adds the squares in another order.
// DPP rotate right by K within each 16-lane row (row_ror:K).
template <int K>
__device__ __forceinline__ float row_ror(float x) {
  return __uint_as_float(__builtin_amdgcn_update_dpp(0u, __float_as_uint(x), 0x120 + K, 0xf, 0xf, false));
}

template <int HD, int HPW>
__global__ __launch_bounds__(64) void qk_norm_rope_rows_kernel(QkNormRopeParams p) {
#pragma clang fp contract(off)
  constexpr int EPL = HD / 16, HALF = HD / 2, PIECES = EPL / 8, STEPS = HPW / 4;
  static_assert(HPW % 4 == 0, "four rows per step");
  __shared__ __attribute__((aligned(16))) float s_cos[HALF], s_sin[HALF];
  const uint32_t lane = threadIdx.x;
  const uint32_t q_chunks = (p.q_heads + HPW - 1) / HPW;
  const uint32_t k_chunks = (p.kv_heads + HPW - 1) / HPW;
  const uint32_t qk_groups = p.tokens * (q_chunks + k_chunks);
  const uint32_t group = blockIdx.x;
  if (group >= qk_groups) {
    // Value rows, four per wave (one per 16-lane group), one or two 16-byte
    // pieces per lane.
    const uint32_t row = 4 * (group - qk_groups) + (lane >> 4);
    if (row >= p.tokens * p.kv_heads) return;
    const uint32_t token = row / p.kv_heads, head = row % p.kv_heads;
    const uint16_t *src = p.v + (int64_t)token * p.v_tok + (int64_t)head * p.v_head + EPL * (lane & 15);
    uint16_t *dst = p.v_cache + (int64_t)(p.offset + token) * p.vc_pos + (int64_t)head * p.vc_head +
                    EPL * (lane & 15);
#pragma unroll
    for (int k = 0; k < PIECES; ++k)
      *reinterpret_cast<uint4 *>(dst + 8 * k) = *reinterpret_cast<const uint4 *>(src + 8 * k);
    return;
  }
  const uint32_t q_groups = p.tokens * q_chunks;
  const bool is_query = group < q_groups;
  const uint32_t chunk_row = is_query ? group : group - q_groups;
  const uint32_t chunks = is_query ? q_chunks : k_chunks;
  const uint32_t heads = is_query ? p.q_heads : p.kv_heads;
  const uint32_t token = chunk_row / chunks;
  const uint32_t h0 = (chunk_row % chunks) * HPW;
  const uint16_t *weight = is_query ? p.q_weight : p.k_weight;
  const uint32_t g = lane >> 4, l = lane & 15;
  const bool first = l < 8;
  const uint32_t e0 = EPL * l;             // this lane's first element of a row
  const uint32_t pair0 = EPL * (l & 7);    // ... and its first pair
  auto row_ptr = [&](uint32_t head) -> const uint16_t * {
    return is_query ? p.q + (int64_t)token * p.q_tok + (int64_t)head * p.q_head
                    : p.k + (int64_t)token * p.k_tok + (int64_t)head * p.k_head;
  };
  // Every row load is issued first, the norm weights with them.
  uint4 wv[PIECES];
#pragma unroll
  for (int k = 0; k < PIECES; ++k) wv[k] = *reinterpret_cast<const uint4 *>(weight + e0 + 8 * k);
  uint4 v[STEPS][PIECES];
#pragma unroll
  for (int i = 0; i < STEPS; ++i) {
    const uint32_t head = h0 + 4 * i + g;
#pragma unroll
    for (int k = 0; k < PIECES; ++k)
      v[i][k] = head < heads ? *reinterpret_cast<const uint4 *>(row_ptr(head) + e0 + 8 * k)
                             : make_uint4(0, 0, 0, 0);
  }
  // Each angle once per wave.
#pragma unroll
  for (int a = 0; a < HALF / 64; ++a) {
    const uint32_t pair = lane + 64 * a;
    const float frequency = powf(p.theta, -(float)(pair * 2) / (float)HD);
    const float angle = (float)(token + p.offset) * frequency;
    s_cos[pair] = cosf(angle);
    s_sin[pair] = sinf(angle);
  }
  __syncthreads();
  float c[EPL], sn[EPL], w[EPL];
#pragma unroll
  for (int e = 0; e < EPL; e += 4) {
    const float4 cv = *reinterpret_cast<const float4 *>(s_cos + pair0 + e);
    const float4 sv = *reinterpret_cast<const float4 *>(s_sin + pair0 + e);
    c[e] = cv.x, c[e + 1] = cv.y, c[e + 2] = cv.z, c[e + 3] = cv.w;
    // First halves take -sin (x c + y (-s)), second halves +sin.
    sn[e] = first ? -sv.x : sv.x, sn[e + 1] = first ? -sv.y : sv.y;
    sn[e + 2] = first ? -sv.z : sv.z, sn[e + 3] = first ? -sv.w : sv.w;
  }
#pragma unroll
  for (int k = 0; k < PIECES; ++k) {
    const uint32_t ww[4] = {wv[k].x, wv[k].y, wv[k].z, wv[k].w};
#pragma unroll
    for (int t = 0; t < 8; ++t) w[8 * k + t] = (t & 1) ? hi_f16(ww[t >> 1]) : lo_f16(ww[t >> 1]);
  }
#pragma unroll
  for (int i = 0; i < STEPS; ++i) {
    if (h0 + 4 * i >= heads) break;  // no row of this step exists
    const uint32_t head = h0 + 4 * i + g;
    float x[EPL];
    float sum = 0.0f;
#pragma unroll
    for (int k = 0; k < PIECES; ++k) {
      const uint32_t ww[4] = {v[i][k].x, v[i][k].y, v[i][k].z, v[i][k].w};
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        x[8 * k + t] = (t & 1) ? hi_f16(ww[t >> 1]) : lo_f16(ww[t >> 1]);
        sum += x[8 * k + t] * x[8 * k + t];
      }
    }
    // Row sum over the row's 16 lanes.
    sum += row_ror<8>(sum);
    sum += row_ror<4>(sum);
    sum += row_ror<2>(sum);
    sum += row_ror<1>(sum);
    const float scale = 1.0f / sqrtf(sum / (float)HD + p.epsilon);
    float out[EPL];
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
      const float n = x[e] * scale * w[e];
      const float m = row_ror<8>(n);  // the partner's normalised element
      out[e] = n * c[e] + m * sn[e];
    }
    if (head < heads) {
      uint16_t *dst =
          (is_query ? p.q_out + (int64_t)token * p.qo_tok + (int64_t)head * p.qo_head
                    : p.cache + (int64_t)(p.offset + token) * p.c_pos + (int64_t)head * p.c_head) +
          e0;
#pragma unroll
      for (int k = 0; k < PIECES; ++k)
        *reinterpret_cast<uint4 *>(dst + 8 * k) =
            make_uint4(pack_f16x2(out[8 * k], out[8 * k + 1]), pack_f16x2(out[8 * k + 2], out[8 * k + 3]),
                       pack_f16x2(out[8 * k + 4], out[8 * k + 5]), pack_f16x2(out[8 * k + 6], out[8 * k + 7]));
    }
  }
}

}  // namespace

hipError_t launch_naive(const NaiveParams &p, uint32_t row_begin,
                        uint32_t row_count, const Launch &l) {
  if (row_count == 0) return no_dispatch(l);
  const uint32_t lds =
      p.kv_length <= kNaiveLdsKeys ? p.kv_length * (uint32_t)sizeof(float) : 0;
  return dispatch(attn_naive_kernel, dim3(row_count), dim3(256), lds, l, p, row_begin);
}

hipError_t launch_copy_kv(const CopyKvParams &p, const Launch &l) {
  const bool vec8 =
      p.head_dim % 8 == 0 && p.s_tok % 8 == 0 && p.s_head % 8 == 0 &&
      p.d_pos % 8 == 0 && p.d_head % 8 == 0 &&
      reinterpret_cast<uintptr_t>(p.src) % 16 == 0 &&
      reinterpret_cast<uintptr_t>(p.dst) % 16 == 0;
  const uint64_t items =
      (uint64_t)p.tokens * p.heads * (vec8 ? p.head_dim / 8 : p.head_dim);
  if (items == 0) return no_dispatch(l);
  const uint64_t blocks64 = (items + 255) / 256;
  const uint32_t blocks = (uint32_t)(blocks64 < 65536 ? blocks64 : 65536);
  if (vec8) return dispatch(copy_kv_kernel<8>, dim3(blocks), dim3(256), 0, l, p);
  return dispatch(copy_kv_kernel<1>, dim3(blocks), dim3(256), 0, l, p);
}

namespace {
template <int HD, int HPW>
hipError_t launch_qk_rows(const QkNormRopeParams &p, const Launch &l) {
  const uint32_t chunks = (p.q_heads + HPW - 1) / HPW + (p.kv_heads + HPW - 1) / HPW;
  const uint32_t groups = p.tokens * chunks + (p.v != nullptr ? (p.tokens * p.kv_heads + 3) / 4 : 0u);
  if (groups == 0) return no_dispatch(l);
  return dispatch(qk_norm_rope_rows_kernel<HD, HPW>, dim3(groups), dim3(64), 0, l, p);
}
}  // namespace

hipError_t launch_qk_norm_rope(const QkNormRopeParams &p, const Launch &l) {
  // Many tokens (prefill): 32 head rows per wave at head_dim 128, 16 at 256,
  // share the angles (c5's chunk, Q [4096, 64, 128] + K [4096, 8, 128]: 16
  // rows 29.9-30.2 us, 32 rows 29.0-29.1, 64 rows 29.4-29.5; at head_dim 256
  // 16 rows measured best). Few tokens (decode): four rows per wave (one per
  // 16-lane group), for the most waves in flight. Needs 16-byte aligned rows
  // and weights (value rows included when the value is appended).
  const bool many = p.tokens >= 16;
  constexpr uint32_t vec = 8;  // halves per 16-byte access
  auto al = [](const void *ptr) { return reinterpret_cast<uintptr_t>(ptr) % 16 == 0; };
  const bool aligned = (p.head_dim == 128 || p.head_dim == 256) && p.q_tok % vec == 0 &&
                       p.q_head % vec == 0 && p.k_tok % vec == 0 && p.k_head % vec == 0 &&
                       p.qo_tok % vec == 0 && p.qo_head % vec == 0 && p.c_pos % vec == 0 &&
                       p.c_head % vec == 0 && al(p.q) && al(p.k) && al(p.q_out) && al(p.cache) &&
                       al(p.q_weight) && al(p.k_weight) &&
                       (p.v == nullptr || (p.v_tok % vec == 0 && p.v_head % vec == 0 &&
                                           p.vc_pos % vec == 0 && p.vc_head % vec == 0 &&
                                           al(p.v) && al(p.v_cache)));
  if (aligned && p.head_dim == 128)
    return many ? launch_qk_rows<128, 32>(p, l) : launch_qk_rows<128, 4>(p, l);
  if (aligned && p.head_dim == 256)
    return many ? launch_qk_rows<256, 16>(p, l) : launch_qk_rows<256, 4>(p, l);
  const uint32_t groups =
      p.tokens * (p.q_heads + p.kv_heads) + (p.v != nullptr ? p.tokens * p.kv_heads : 0u);
  if (groups == 0) return no_dispatch(l);
  return dispatch(qk_norm_rope_kernel, dim3(groups), dim3(64), 0, l, p);
}

}  // namespace kernels
}  // namespace mi
