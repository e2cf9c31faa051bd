// The attention block's neighbours in the Qwen3 layer: RMSNorm and RoPE of
// the unfused Q/K path, and the few-row matmul of the decode o_proj.
#include <type_traits>

#include "device_common.hpp"
#include "kernels.hpp"

namespace mi {
namespace kernels {
namespace {

using namespace mi::dev;

__device__ __forceinline__ int64_t row_offset(const RowIndex &ri, uint32_t row) {
  const uint32_t i2 = row % ri.n2;
  const uint32_t t = row / ri.n2;
  return (int64_t)(t / ri.n1) * ri.s0 + (int64_t)(t % ri.n1) * ri.s1 + (int64_t)i2 * ri.s2;
}

__device__ __forceinline__ uint4 load16(const uint16_t *ptr) {
  return *reinterpret_cast<const uint4 *>(ptr);
}

// Weights are streamed (each byte read once per call): non-temporal loads.
__device__ __forceinline__ uint4 load16_stream(const uint16_t *ptr) {
  typedef unsigned u4_t __attribute__((ext_vector_type(4)));
  const u4_t x = __builtin_nontemporal_load(reinterpret_cast<const u4_t *>(ptr));
  return make_uint4(x.x, x.y, x.z, x.w);
}

// Eight f16 products of two 16-byte pieces, accumulated in f32.
__device__ __forceinline__ float dot8(uint4 a, uint4 b, float acc) {
  acc = dot2(a.x, b.x, acc);
  acc = dot2(a.y, b.y, acc);
  acc = dot2(a.z, b.z, acc);
  return dot2(a.w, b.w, acc);
}

// rms_norm_f16 (transformer.metal:1318-1340): one wave per row, four rows per
// workgroup. Pass 1 sums squares (16-byte loads when rows allow), pass 2
// writes f16(x * scale * w). Rows of up to kRmsCached 16-byte pieces per
// lane (8192 halves) are loaded once, all pieces in flight together, and kept
// in registers for pass 2; wider rows re-read (an L1/L2 hit). EARLY_W (grids
// smaller than the CUs, a decode token) loads the weights with the row, one
// round trip before the reduction instead of a second one after it (measured
// on MI355X, [1, 5120]: 3.5 against 4.0 us per call); large grids keep the
// later load, whose lower register count holds more waves per CU ([4096,
// 5120]: 16.6 against 17.7 us).
constexpr int kRmsCached = 16;

template <bool VEC, bool EARLY_W>
__global__ __launch_bounds__(256) void rms_norm_kernel(RmsNormParams p) {
  const uint32_t row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= p.rows) return;
  const uint32_t lane = threadIdx.x & 63;
  const uint16_t *x = p.x + row_offset(p.x_rows, row);
  uint16_t *out = p.out + row_offset(p.o_rows, row);
  float sum = 0.0f;
  if constexpr (VEC) {
    if (p.width <= 512u * kRmsCached) {
      uint4 v[kRmsCached], wt[EARLY_W ? kRmsCached : 1];
#pragma unroll
      for (int j = 0; j < kRmsCached; ++j) {
        const uint32_t i = lane * 8 + 512 * j;
        v[j] = i < p.width ? load16(x + i) : make_uint4(0, 0, 0, 0);
        if constexpr (EARLY_W) wt[j] = i < p.width ? load16(p.weight + i) : make_uint4(0, 0, 0, 0);
      }
      // Same order as the streaming loop below (zero pieces add exactly 0).
#pragma unroll
      for (int j = 0; j < kRmsCached; ++j) sum = dot8(v[j], v[j], sum);
      sum = group_sum<64>(sum);
      const float scale = 1.0f / sqrtf(sum / (float)p.width + p.epsilon);
#pragma unroll
      for (int j = 0; j < kRmsCached; ++j) {
        const uint32_t i = lane * 8 + 512 * j;
        if (i < p.width) {
          uint4 w;
          if constexpr (EARLY_W) w = wt[j];
          else w = load16(p.weight + i);
          const uint32_t vin[4] = {v[j].x, v[j].y, v[j].z, v[j].w}, win[4] = {w.x, w.y, w.z, w.w};
          uint32_t o[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const uint16_t lo = f32_to_f16(lo_f16(vin[e]) * scale * lo_f16(win[e]));
            const uint16_t hi = f32_to_f16(hi_f16(vin[e]) * scale * hi_f16(win[e]));
            o[e] = (uint32_t)lo | ((uint32_t)hi << 16);
          }
          *reinterpret_cast<uint4 *>(out + i) = make_uint4(o[0], o[1], o[2], o[3]);
        }
      }
      return;
    }
  }
  if constexpr (VEC) {
    for (uint32_t i = lane * 8; i < p.width; i += 512) {
      const uint4 v = load16(x + i);
      sum = dot8(v, v, sum);
    }
  } else {
    for (uint32_t i = lane; i < p.width; i += 64) {
      const float v = f16_to_f32(x[i]);
      sum += v * v;
    }
  }
  sum = group_sum<64>(sum);
  const float scale = 1.0f / sqrtf(sum / (float)p.width + p.epsilon);
  if constexpr (VEC) {
    for (uint32_t i = lane * 8; i < p.width; i += 512) {
      const uint4 v = load16(x + i), w = load16(p.weight + i);
      const uint32_t vin[4] = {v.x, v.y, v.z, v.w}, win[4] = {w.x, w.y, w.z, w.w};
      uint32_t o[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint16_t lo = f32_to_f16(lo_f16(vin[j]) * scale * lo_f16(win[j]));
        const uint16_t hi = f32_to_f16(hi_f16(vin[j]) * scale * hi_f16(win[j]));
        o[j] = (uint32_t)lo | ((uint32_t)hi << 16);
      }
      *reinterpret_cast<uint4 *>(out + i) = make_uint4(o[0], o[1], o[2], o[3]);
    }
  } else {
    for (uint32_t i = lane; i < p.width; i += 64)
      out[i] = f32_to_f16(f16_to_f32(x[i]) * scale * f16_to_f32(p.weight[i]));
  }
}

// rope_f16 (transformer.metal:1514-1531): pairs (i, i + D/2) rotated by
// (token + offset) * theta^(-2i/D). The same f32 operations, uncontracted,
// as the fused Q/K kernel's RoPE step.
constexpr uint32_t kRopeHeads = 8;  // heads per thread

// One thread per (token, chunk of kRopeHeads heads, PAIRS consecutive
// pairs): the angles' cosines and sines depend on (token, pair) only, so
// they are computed once for the chunk's heads. A wave covers consecutive
// pairs of one row, so each head's two halves load and store as contiguous
// runs (PAIRS = 2: 4-byte accesses, 256 bytes per wave).
template <int PAIRS>
__global__ __launch_bounds__(256) void rope_kernel(RopeParams p) {
#pragma clang fp contract(off)
  const uint32_t half = p.head_dim / 2;
  const uint32_t groups = half / PAIRS;
  const uint32_t chunks = (p.heads + kRopeHeads - 1) / kRopeHeads;
  const uint64_t total = (uint64_t)p.tokens * chunks * groups;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (uint64_t)gridDim.x * blockDim.x) {
    const uint32_t pair = (uint32_t)(i % groups) * PAIRS;
    const uint64_t r = i / groups;
    const uint32_t chunk = (uint32_t)(r % chunks);
    const uint32_t token = (uint32_t)(r / chunks);
    float c[PAIRS], s[PAIRS];
#pragma unroll
    for (int e = 0; e < PAIRS; ++e) {
      const float frequency = powf(p.theta, -(float)((pair + e) * 2) / (float)p.head_dim);
      const float angle = (float)(token + p.offset) * frequency;
      c[e] = cosf(angle);
      s[e] = sinf(angle);
    }
    const uint16_t *x = p.x + (int64_t)token * p.x_tok + pair;
    uint16_t *out = p.out + (int64_t)token * p.o_tok + pair;
#pragma unroll
    for (uint32_t j = 0; j < kRopeHeads; ++j) {
      const uint32_t head = chunk * kRopeHeads + j;
      if (head < p.heads) {
        const uint16_t *xa = x + (int64_t)head * p.x_head;
        uint16_t *oa = out + (int64_t)head * p.o_head;
        if constexpr (PAIRS == 2) {
          const uint32_t wa = *reinterpret_cast<const uint32_t *>(xa);
          const uint32_t wb = *reinterpret_cast<const uint32_t *>(xa + half);
          float a[2] = {lo_f16(wa), hi_f16(wa)}, bb[2] = {lo_f16(wb), hi_f16(wb)};
          uint32_t lo = 0, hi = 0;
#pragma unroll
          for (int e = 0; e < 2; ++e) {
            lo |= (uint32_t)f32_to_f16(a[e] * c[e] - bb[e] * s[e]) << (16 * e);
            hi |= (uint32_t)f32_to_f16(a[e] * s[e] + bb[e] * c[e]) << (16 * e);
          }
          *reinterpret_cast<uint32_t *>(oa) = lo;
          *reinterpret_cast<uint32_t *>(oa + half) = hi;
        } else {
          const float a = f16_to_f32(xa[0]), bb = f16_to_f32(xa[half]);
          oa[0] = f32_to_f16(a * c[0] - bb * s[0]);
          oa[half] = f32_to_f16(a * s[0] + bb * c[0]);
        }
      }
    }
  }
}

// The same rotation for 16-byte aligned rows with head_dim a multiple of 16
// (up to 512): one workgroup per token. Its angles depend on (token, pair)
// only, so the workgroup computes each once (one pair per thread) into LDS.
// Then each thread rotates 8 consecutive pairs of one head: a 16-byte load of
// the first-half elements and one of the matching second-half elements,
// every load of the thread issued before it computes. The f32 steps per
// element are the ones above, so the output is bit-identical.
constexpr uint32_t kRopeRowItems = 2;  // (head, 8-pair) items per thread and round
__global__ __launch_bounds__(256) void rope_rows_kernel(RopeParams p) {
#pragma clang fp contract(off)
  __shared__ __attribute__((aligned(16))) float s_cos[256], s_sin[256];
  const uint32_t token = blockIdx.x, tid = threadIdx.x;
  const uint32_t half = p.head_dim / 2;
  const uint32_t per_head = half / 8;
  const uint32_t items = p.heads * per_head;
  const uint16_t *xt = p.x + (int64_t)token * p.x_tok;
  uint16_t *ot = p.out + (int64_t)token * p.o_tok;
  uint4 a[kRopeRowItems], b[kRopeRowItems];
  auto load = [&](uint32_t base) __attribute__((always_inline)) {
#pragma unroll
    for (uint32_t k = 0; k < kRopeRowItems; ++k) {
      const uint32_t it = base + tid + 256 * k;
      if (it < items) {
        const uint16_t *row = xt + (int64_t)(it / per_head) * p.x_head + 8 * (it % per_head);
        a[k] = *reinterpret_cast<const uint4 *>(row);
        b[k] = *reinterpret_cast<const uint4 *>(row + half);
      }
    }
  };
  // The first rows are in flight while the angles are computed (a decode
  // token's rows are all of them).
  load(0);
  for (uint32_t pair = tid; pair < half; pair += 256) {
    const float frequency = powf(p.theta, -(float)(pair * 2) / (float)p.head_dim);
    const float angle = (float)(token + p.offset) * frequency;
    s_cos[pair] = cosf(angle);
    s_sin[pair] = sinf(angle);
  }
  __syncthreads();
  for (uint32_t base = 0; base < items; base += 256 * kRopeRowItems) {
    if (base != 0) load(base);
#pragma unroll
    for (uint32_t k = 0; k < kRopeRowItems; ++k) {
      const uint32_t it = base + tid + 256 * k;
      if (it >= items) continue;
      const uint32_t pair0 = 8 * (it % per_head);
      const uint32_t wa[4] = {a[k].x, a[k].y, a[k].z, a[k].w};
      const uint32_t wb[4] = {b[k].x, b[k].y, b[k].z, b[k].w};
      uint32_t lo[4], hi[4];
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const float2 c = *reinterpret_cast<const float2 *>(s_cos + pair0 + 2 * w);
        const float2 sn = *reinterpret_cast<const float2 *>(s_sin + pair0 + 2 * w);
        const float a0 = lo_f16(wa[w]), a1 = hi_f16(wa[w]);
        const float b0 = lo_f16(wb[w]), b1 = hi_f16(wb[w]);
        lo[w] = pack_f16x2(a0 * c.x - b0 * sn.x, a1 * c.y - b1 * sn.y);
        hi[w] = pack_f16x2(a0 * sn.x + b0 * c.x, a1 * sn.y + b1 * c.y);
      }
      uint16_t *orow = ot + (int64_t)(it / per_head) * p.o_head + pair0;
      *reinterpret_cast<uint4 *>(orow) = make_uint4(lo[0], lo[1], lo[2], lo[3]);
      *reinterpret_cast<uint4 *>(orow + half) = make_uint4(hi[0], hi[1], hi[2], hi[3]);
    }
  }
}

// Skinny GEMM for 8 < m <= 32 rows of x (the batched-decode o_proj,
// qwen3.rs:751-752 over B sequences): out[m, n] = x[m, k] . w[n, k]^T with
// f32 accumulation, bound by streaming the weight once.
//
// One workgroup per 16 output features (weight rows), so n / 16 workgroups
// spread over the CUs; its four waves take a quarter of k each, and the x
// rows are the A operand of v_mfma_f32_16x16x32_f16, the weight rows the B
// operand. Loads are coalesced: eight lanes read 128 contiguous bytes of one
// row, a 1 KB load covering eight rows of one 64-key step. Each wave moves
// its loads through a private LDS tile of rows of 64 keys (16-byte chunk c
// of row r at c ^ ((r >> 1) & 7), so both the row-wise writes and the
// MFMA-layout reads, 16 rows x one chunk, hit all 64 banks once) into MFMA
// layout; a wave's LDS accesses execute in order, so the tile needs no
// barrier. Chunks of CS steps alternate between two register sets: two
// chunks of loads are in flight while one is multiplied. The four waves'
// sums meet in LDS and add in wave order. Rows of x at or past m re-read
// row m - 1 and are never stored.
//
// Measured on MI355X (graph replays, weights rotated through 512 MB): the
// split-k alternatives (64 features per workgroup, k split over workgroups)
// lost their gain in the cross-workgroup merge (agent-scope release per
// workgroup, or a second launch); rotating each workgroup's chunk order and
// masking the loads of x rows past m were slower too.
template <int MB>
__global__ __launch_bounds__(256) void skinny_gemm_kernel(MatvecParams p) {
  using namespace dev;
  constexpr int CS = kSkinnyChunkSteps;
  constexpr int ROWS = 16 + 16 * MB;  // weight rows, then x rows
  constexpr int LOADS = ROWS / 8;     // 1 KB loads per 64-key step
  typedef float sf4 __attribute__((ext_vector_type(4)));
  typedef unsigned u4_t __attribute__((ext_vector_type(4)));
  __shared__ __attribute__((aligned(16))) uint16_t s_tile[4][CS][ROWS][64];
  __shared__ float s_acc[4][MB][64][4];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const uint32_t n0 = blockIdx.x * 16;
  const uint32_t quarter = p.k / 4, k0 = wave * quarter;
  // Load i of a step: tile row 8 i + lane / 8, chunk lane % 8.
  const int lrow = lane >> 3, lchunk = lane & 7;
  const uint16_t *src[LOADS];
  int dst[LOADS];
#pragma unroll
  for (int i = 0; i < LOADS; ++i) {
    const int row = 8 * i + lrow;
    src[i] = row < 16 ? p.w + (int64_t)(n0 + row) * p.w_row + k0 + 8 * lchunk
                      : p.x + (int64_t)min((uint32_t)(row - 16), p.m - 1) * p.x_row + k0 + 8 * lchunk;
    dst[i] = row * 64 + ((lchunk ^ ((row >> 1) & 7)) * 8);
  }
  // MFMA operands: lane (r, kg) takes chunks kg (h = 0) and kg + 4 (h = 1)
  // of row r, keys 8 kg .. 8 kg + 7 and 32 + 8 kg .. 32 + 8 kg + 7, for the
  // weight and the x rows alike.
  const int r = lane & 15, kg = lane >> 4;
  int wread[2], xread[MB][2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    wread[h] = r * 64 + (((kg + 4 * h) ^ ((r >> 1) & 7)) * 8);
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      const int xr = 16 + 16 * mb + r;
      xread[mb][h] = xr * 64 + (((kg + 4 * h) ^ ((xr >> 1) & 7)) * 8);
    }
  }
  u4_t regs[2][CS][LOADS];
  auto load = [&](uint32_t chunk, auto set_tag) __attribute__((always_inline)) {
    constexpr int S = decltype(set_tag)::value;
    const uint32_t off = chunk * CS * 64;
#pragma unroll
    for (int s = 0; s < CS; ++s)
#pragma unroll
      for (int i = 0; i < LOADS; ++i)
        regs[S][s][i] = *reinterpret_cast<const u4_t *>(src[i] + off + 64 * s);
  };
  auto store = [&](auto set_tag) __attribute__((always_inline)) {
    constexpr int S = decltype(set_tag)::value;
#pragma unroll
    for (int s = 0; s < CS; ++s)
#pragma unroll
      for (int i = 0; i < LOADS; ++i)
        *reinterpret_cast<u4_t *>(&s_tile[wave][s][0][0] + dst[i]) = regs[S][s][i];
  };
  sf4 acc[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) acc[mb] = sf4{0.0f, 0.0f, 0.0f, 0.0f};
  auto compute = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int s = 0; s < CS; ++s)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const h8_t b = as_h8(*reinterpret_cast<const uint4 *>(&s_tile[wave][s][0][0] + wread[h]));
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
          acc[mb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
              as_h8(*reinterpret_cast<const uint4 *>(&s_tile[wave][s][0][0] + xread[mb][h])), b,
              acc[mb], 0, 0, 0);
      }
  };
  using Set0 = std::integral_constant<int, 0>;
  using Set1 = std::integral_constant<int, 1>;
  // The quarter is a whole number of chunk pairs; the last pair issues no
  // further loads. The scheduling barriers keep each chunk's loads issued
  // ahead of the multiplies.
  const uint32_t pairs = quarter / (2 * CS * 64);
  load(0, Set0{});
  load(1, Set1{});
  for (uint32_t pi = 0; pi + 1 < pairs; ++pi) {
    store(Set0{});
    load(2 * pi + 2, Set0{});
    __builtin_amdgcn_sched_barrier(0);
    compute();
    __builtin_amdgcn_sched_barrier(0);
    store(Set1{});
    load(2 * pi + 3, Set1{});
    __builtin_amdgcn_sched_barrier(0);
    compute();
    __builtin_amdgcn_sched_barrier(0);
  }
  store(Set0{});
  compute();
  store(Set1{});
  compute();
  // Lane (j, g) of block mb holds rows 16 mb + 4 g .. + 3 of feature n0 + j.
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int e = 0; e < 4; ++e) s_acc[wave][mb][lane][e] = acc[mb][e];
  __syncthreads();
  if (tid < 64 * MB) {
    const int mb = tid >> 6, ln = tid & 63;
    const uint32_t col = n0 + (ln & 15);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float v = ((s_acc[0][mb][ln][e] + s_acc[1][mb][ln][e]) + s_acc[2][mb][ln][e]) +
                      s_acc[3][mb][ln][e];
      const uint32_t row = 16 * mb + 4 * (ln >> 4) + e;
      if (row < p.m) p.out[(int64_t)row * p.o_row + col] = f32_to_f16(v);
    }
  }
}

// Few-row matmul (the decode o_proj, matvec_f16 family of
// transformer.metal:274-400): one wave per weight row (= output column),
// four per workgroup. Lanes stream the row in 16-byte pieces (64 lanes cover
// 512 halves), kPieces pieces in flight per lane, and multiply each piece with
// the same piece of up to ROWS rows of x, which stay cache-resident across the
// waves. The weight is read from HBM once per ROWS rows of x. Grid
// (ceil(n / 4), ceil(m / ROWS)).
template <int ROWS, bool VEC>
__global__ __launch_bounds__(256) void matvec_kernel(MatvecParams p) {
  constexpr uint32_t kPieces = 4;
  const uint32_t lane = threadIdx.x & 63;
  const uint32_t col = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (col >= p.n) return;
  const uint32_t r0 = blockIdx.y * ROWS;
  const uint32_t rows = min((uint32_t)ROWS, p.m - r0);
  const uint16_t *w = p.w + (int64_t)col * p.w_row;
  const uint16_t *x = p.x + (int64_t)r0 * p.x_row;
  float acc[ROWS];
#pragma unroll
  for (int r = 0; r < ROWS; ++r) acc[r] = 0.0f;
  if constexpr (VEC) {
    const uint32_t pieces = p.k / 8;
    for (uint32_t base = lane; base < pieces; base += 64 * kPieces) {
      uint4 wv[kPieces];
#pragma unroll
      for (uint32_t u = 0; u < kPieces; ++u) {
        const uint32_t idx = base + 64 * u;
        wv[u] = idx < pieces ? load16_stream(w + (size_t)idx * 8) : make_uint4(0, 0, 0, 0);
      }
#pragma unroll
      for (uint32_t u = 0; u < kPieces; ++u) {
        const uint32_t idx = base + 64 * u;
        if (idx < pieces) {
#pragma unroll
          for (int r = 0; r < ROWS; ++r)
            if (r < (int)rows)
              acc[r] = dot8(wv[u], load16(x + (int64_t)r * p.x_row + (size_t)idx * 8), acc[r]);
        }
      }
    }
  } else {
    for (uint32_t i = lane; i < p.k; i += 64) {
      const float wv = f16_to_f32(w[i]);
#pragma unroll
      for (int r = 0; r < ROWS; ++r)
        if (r < (int)rows) acc[r] += wv * f16_to_f32(x[(int64_t)r * p.x_row + i]);
    }
  }
#pragma unroll
  for (int r = 0; r < ROWS; ++r) {
    const float total = group_sum<64>(acc[r]);
    if (lane == (uint32_t)r && r < (int)rows)
      p.out[(int64_t)(r0 + r) * p.o_row + col] = f32_to_f16(total);
  }
}

bool aligned16(const void *ptr) { return reinterpret_cast<uintptr_t>(ptr) % 16 == 0; }

bool rows_vector_friendly(const RowIndex &ri) {
  return ri.s0 % 8 == 0 && ri.s1 % 8 == 0 && ri.s2 % 8 == 0;
}

template <int ROWS>
hipError_t dispatch_matvec(const MatvecParams &p, bool vec, dim3 grid, const Launch &l) {
  if (vec) return dispatch(matvec_kernel<ROWS, true>, grid, dim3(256), 0, l, p);
  return dispatch(matvec_kernel<ROWS, false>, grid, dim3(256), 0, l, p);
}

}  // namespace

hipError_t launch_rms_norm(const RmsNormParams &p, uint32_t compute_units, const Launch &l) {
  if (p.rows == 0 || p.width == 0) return no_dispatch(l);
  const bool vec = p.width % 8 == 0 && rows_vector_friendly(p.x_rows) &&
                   rows_vector_friendly(p.o_rows) && aligned16(p.x) && aligned16(p.out) &&
                   aligned16(p.weight);
  const dim3 grid((p.rows + 3) / 4);
  // Grids smaller than the CUs load the weights with the row (one round
  // trip less); larger ones keep the later load, which holds more waves.
  if (vec && grid.x < compute_units)
    return dispatch(rms_norm_kernel<true, true>, grid, dim3(256), 0, l, p);
  if (vec) return dispatch(rms_norm_kernel<true, false>, grid, dim3(256), 0, l, p);
  return dispatch(rms_norm_kernel<false, false>, grid, dim3(256), 0, l, p);
}

hipError_t launch_rope(const RopeParams &p, const Launch &l) {
  // 16-byte rows: one workgroup per token (c5's Q [4096, 64, 128]: 30.3-31.1
  // us with the per-thread kernel below).
  auto al16 = [](const void *ptr) { return reinterpret_cast<uintptr_t>(ptr) % 16 == 0; };
  if (p.head_dim % 16 == 0 && p.head_dim <= 512 && p.x_tok % 8 == 0 && p.x_head % 8 == 0 &&
      p.o_tok % 8 == 0 && p.o_head % 8 == 0 && al16(p.x) && al16(p.out)) {
    if (p.tokens == 0 || p.heads == 0) return no_dispatch(l);
    return dispatch(rope_rows_kernel, dim3(p.tokens), dim3(256), 0, l, p);
  }
  // 4-byte accesses when every row start and both halves are 4-byte aligned.
  const bool two = p.head_dim % 4 == 0 && p.x_tok % 2 == 0 && p.x_head % 2 == 0 &&
                   p.o_tok % 2 == 0 && p.o_head % 2 == 0 &&
                   reinterpret_cast<uintptr_t>(p.x) % 4 == 0 &&
                   reinterpret_cast<uintptr_t>(p.out) % 4 == 0;
  const uint64_t items = (uint64_t)p.tokens * ((p.heads + kRopeHeads - 1) / kRopeHeads) *
                         (p.head_dim / 2 / (two ? 2 : 1));
  if (items == 0) return no_dispatch(l);
  const uint64_t blocks64 = (items + 255) / 256;
  const uint32_t blocks = (uint32_t)(blocks64 < 65536 ? blocks64 : 65536);
  if (two) return dispatch(rope_kernel<2>, dim3(blocks), dim3(256), 0, l, p);
  return dispatch(rope_kernel<1>, dim3(blocks), dim3(256), 0, l, p);
}

bool skinny_gemm_supported(const MatvecParams &p, uint32_t compute_units) {
  auto al16 = [](const void *ptr) { return reinterpret_cast<uintptr_t>(ptr) % 16 == 0; };
  return p.m > kMatvecRows && p.m <= kSkinnyMaxRows && p.n > 0 && p.k > 0 && p.n % 16 == 0 &&
         p.n / 16 <= compute_units &&
         p.k % (4 * 2 * kSkinnyChunkSteps * 64) == 0 && p.x_row % 8 == 0 && p.w_row % 8 == 0 &&
         al16(p.x) && al16(p.w);
}

hipError_t launch_skinny_gemm(const MatvecParams &p, uint32_t compute_units, const Launch &l) {
  if (!skinny_gemm_supported(p, compute_units)) return hipErrorInvalidValue;
  if (p.m <= 16) return dispatch(skinny_gemm_kernel<1>, dim3(p.n / 16), dim3(256), 0, l, p);
  return dispatch(skinny_gemm_kernel<2>, dim3(p.n / 16), dim3(256), 0, l, p);
}

hipError_t launch_matvec(const MatvecParams &p, const Launch &l) {
  if (p.m == 0 || p.n == 0) return no_dispatch(l);
  const bool vec = p.k % 8 == 0 && p.x_row % 8 == 0 && p.w_row % 8 == 0 && aligned16(p.x) &&
                   aligned16(p.w);
  const uint32_t rows = p.m <= 1 ? 1 : p.m <= 2 ? 2 : p.m <= 4 ? 4 : kMatvecRows;
  const dim3 grid((p.n + 3) / 4, (p.m + rows - 1) / rows);
  switch (rows) {
    case 1: return dispatch_matvec<1>(p, vec, grid, l);
    case 2: return dispatch_matvec<2>(p, vec, grid, l);
    case 4: return dispatch_matvec<4>(p, vec, grid, l);
    default: return dispatch_matvec<kMatvecRows>(p, vec, grid, l);
  }
}

}  // namespace kernels
}  // namespace mi
