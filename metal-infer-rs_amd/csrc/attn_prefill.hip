// MFMA flash prefill for gfx950 (AttentionKind::FlashPrefill at D = 64, 128).
//
// Replaces attention_flash_prefill_f16 (transformer.metal:1667-1822) with a
// CDNA4 design:
//  - GQA packing: a workgroup owns 128 rows of the packed (token, head in
//    group) dimension of ONE KV head, so each K/V tile is staged into LDS once
//    for all G query heads that share it;
//  - S^T = K Q^T on v_mfma_f32_32x32x16_f16, K read from LDS as the A
//    operand and Q^T kept in registers as the B operand. Each lane then holds
//    one query row's scores, so the f32 online softmax is lane-local plus a
//    single exchange with the partner half-wave;
//  - O^T += V^T P^T on the same MFMA: P^T is the S^T accumulator converted to
//    f16 in place (no shuffles), because V is transposed into LDS with its
//    keys permuted (bits 2 and 3 of the key index swapped) to match the order
//    in which the S^T accumulator holds them;
//  - the next tile's K/V global loads are in flight while the current tile
//    is computed; causally heavy row tiles are dispatched first.
#include <type_traits>

#include "device_common.hpp"
#include "kernels.hpp"

namespace mi {
namespace kernels {
namespace {

using namespace mi::dev;

constexpr int BM = kPrefillBlockM;  // packed rows per workgroup
constexpr int BN = 64;              // keys per KV tile
constexpr int THREADS = 256;        // 4 waves x 32 rows

typedef __fp16 h8_t __attribute__((ext_vector_type(8)));

// Column of key `key` (0..63 within a tile) in the transposed V tile: bits
// 2 and 3 swapped, which is the key order of the P operand (see above).
__device__ __forceinline__ int vt_col(int key) {
  return (key & ~12) | ((key & 4) << 1) | ((key & 8) >> 1);
}

__device__ __forceinline__ uint4 load16(const uint16_t *p) {
  return *reinterpret_cast<const uint4 *>(p);
}

__device__ __forceinline__ h8_t as_h8(uint4 v) {
  return __builtin_bit_cast(h8_t, v);
}

// Packs the f16 halves of words a and b: lo -> (a.lo, b.lo), hi -> (a.hi, b.hi).
__device__ __forceinline__ uint32_t pack_lo(uint32_t a, uint32_t b) {
  return __builtin_amdgcn_perm(b, a, 0x05040100u);
}
__device__ __forceinline__ uint32_t pack_hi(uint32_t a, uint32_t b) {
  return __builtin_amdgcn_perm(b, a, 0x07060302u);
}

// v_cvt_pk_f16_f32: two f32 -> packed f16, round to nearest even.
__device__ __forceinline__ uint32_t pack_f16x2(float lo, float hi) {
  typedef float f2_t __attribute__((ext_vector_type(2)));
  const f2_t v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, half2_t));
}

// O and l are rescaled only when a row's max grows past its reference by
// more than 2^8. The reference may then lag the true max, which keeps
// P = 2^(s - m_ref) <= 256 (well inside f16) and changes nothing in O / l,
// since both use the same reference.
constexpr float kRescaleLog2 = 8.0f;

// sched_group_barrier instruction classes (LLVM AMDGPU): MFMA, LDS read.
constexpr int kSchedMfma = 0x008;
constexpr int kSchedDsRead = 0x100;
constexpr int kReadAhead = 4;

template <int D>
__global__ __launch_bounds__(THREADS, 2) void attn_prefill_kernel(
    const PrefillParams p) {
  constexpr int DC = D / 16;          // 16-wide d chunks of Q K^T
  constexpr int DT = D / 32;          // 32-row d tiles of O^T
  constexpr int KS = D + 8;           // K tile row stride (halves)
  constexpr int VS = BN + 8;          // V^T tile row stride (halves)
  constexpr int K_CHUNKS = BN * D / 8 / THREADS;           // 16-B pieces
  constexpr int V_JOBS = (BN / 4) * (D / 8);                // 4 keys x 8 d
  constexpr int V_PER = (V_JOBS + THREADS - 1) / THREADS;
  // Two LDS stages: tile i is read from one while tile i+1 is written into
  // the other, so one barrier per tile suffices.
  __shared__ __attribute__((aligned(16))) uint16_t k_lds2[2][BN * KS];
  __shared__ __attribute__((aligned(16))) uint16_t v_lds2[2][D * VS];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int n = lane & 31, h = lane >> 5;
  const uint32_t G = p.group;
  // XCD-aware order: workgroups are dispatched round-robin over the 8 XCDs
  // by linear id, so id % 8 selects the XCD. When the KV heads split evenly
  // over the XCDs, each XCD gets whole heads (their K/V stay in its L2);
  // within an XCD the heaviest row tiles go first.
  uint32_t tile, kvh;
  {
    const uint32_t id = blockIdx.x + gridDim.x * blockIdx.y;
    const uint32_t H = gridDim.y;
    if (H % 8 == 0) {
      const uint32_t xcd = id % 8, k = id / 8, per = H / 8;
      kvh = xcd * per + k % per;
      tile = p.row_tiles - 1 - k / per;
    } else {
      tile = p.row_tiles - 1 - blockIdx.x;
      kvh = blockIdx.y;
    }
  }
  const uint32_t row0 = tile * BM;
  const uint32_t my_row = row0 + wave * 32 + n;
  const uint32_t my_t = my_row / G, my_g = my_row % G;
  const bool row_ok = my_t < p.tokens;
  const uint32_t t_first = row0 / G;
  const uint32_t t_last = min(p.tokens - 1, (row0 + BM - 1) / G);
  const uint64_t L = p.kv_length;
  const uint64_t off = p.query_offset;
  const uint32_t kmax =
      p.causal != 0 ? (uint32_t)min(L, off + t_last + 1) : (uint32_t)L;
  const uint32_t n_tiles = (kmax + BN - 1) / BN;
  // Last visible key of this lane's row, and of the tile's first row (below
  // which no key needs a mask).
  const uint64_t lim =
      p.causal != 0 ? min(L - 1, off + min(my_t, p.tokens - 1)) : L - 1;
  const uint64_t full_lim = p.causal != 0 ? min(L - 1, off + t_first) : L - 1;

  // Q^T as the B operand: lane (h, n) holds Q[row n][16c + 8h .. +8].
  h8_t qop[DC];
  {
    const uint16_t *qrow = p.q + (int64_t)min(my_t, p.tokens - 1) * p.q_tok +
                           (int64_t)(kvh * G + my_g) * p.q_head;
#pragma unroll
    for (int c = 0; c < DC; ++c)
      qop[c] = row_ok ? as_h8(load16(qrow + 16 * c + 8 * h))
                      : as_h8(make_uint4(0, 0, 0, 0));
  }
  const uint16_t *kbase = p.k + (int64_t)kvh * p.k_head;
  const uint16_t *vbase = p.v + (int64_t)kvh * p.v_head;

  // Tile staging registers: K as 16-B row pieces, V as 4-key x 8-d blocks.
  uint4 kreg[K_CHUNKS];
  uint4 vreg[V_PER][4];
  auto load_tile = [&](uint32_t j0) {
    // Uniform tile base + 32-bit per-lane offsets (scalar-base addressing).
    const uint16_t *kt = kbase + (int64_t)j0 * p.k_pos;
    const uint16_t *vt = vbase + (int64_t)j0 * p.v_pos;
    const int last = j0 + BN > kmax ? (int)(kmax - 1 - j0) : BN - 1;
#pragma unroll
    for (int i = 0; i < K_CHUNKS; ++i) {
      const int c = tid + i * THREADS;
      const int key = min(c / (D / 8), last);
      kreg[i] = load16(kt + (uint32_t)(key * p.k_pos + (c % (D / 8)) * 8));
    }
#pragma unroll
    for (int i = 0; i < V_PER; ++i) {
      const int job = tid + i * THREADS;
      if (job < V_JOBS) {
        const int quad = job % (BN / 4), dg = job / (BN / 4);
#pragma unroll
        for (int e = 0; e < 4; ++e)
          vreg[i][e] = load16(vt + (uint32_t)(min(4 * quad + e, last) * p.v_pos + dg * 8));
      }
    }
  };
  auto store_tile = [&](int stage) {
    uint16_t *k_lds = k_lds2[stage];
    uint16_t *v_lds = v_lds2[stage];
#pragma unroll
    for (int i = 0; i < K_CHUNKS; ++i) {
      const int c = tid + i * THREADS;
      const int key = c / (D / 8), piece = c % (D / 8);
      *reinterpret_cast<uint4 *>(k_lds + key * KS + piece * 8) = kreg[i];
    }
#pragma unroll
    for (int i = 0; i < V_PER; ++i) {
      const int job = tid + i * THREADS;
      if (job < V_JOBS) {
        const int quad = job % (BN / 4), dg = job / (BN / 4);
        const int col = vt_col(4 * quad);
        const uint32_t *w0 = reinterpret_cast<const uint32_t *>(&vreg[i][0]);
        const uint32_t *w1 = reinterpret_cast<const uint32_t *>(&vreg[i][1]);
        const uint32_t *w2 = reinterpret_cast<const uint32_t *>(&vreg[i][2]);
        const uint32_t *w3 = reinterpret_cast<const uint32_t *>(&vreg[i][3]);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int w = e >> 1;
          uint2 pair;
          pair.x = (e & 1) ? pack_hi(w0[w], w1[w]) : pack_lo(w0[w], w1[w]);
          pair.y = (e & 1) ? pack_hi(w2[w], w3[w]) : pack_lo(w2[w], w3[w]);
          *reinterpret_cast<uint2 *>(v_lds + (dg * 8 + e) * VS + col) = pair;
        }
      }
    }
  };

  float16_t o[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[dt][r] = 0.0f;
  float m_run = -INFINITY;  // raw-score running max of this row
  float l_run = 0.0f;       // this half-wave's share of the row sum
  const float c2 = p.scale_log2;

  auto step = [&](uint32_t it, auto mask_tag) {
    constexpr bool MASK = decltype(mask_tag)::value;
    const uint32_t j0 = it * BN;
    const uint16_t *k_lds = k_lds2[it & 1];
    const uint16_t *v_lds = v_lds2[it & 1];

    // S^T[key][row] for the 64 keys of the tile: two 32-key M tiles. MFMA
    // phases run at raised wave priority, so while one wave of a SIMD feeds
    // the matrix core the other's softmax VALU fills the issue gaps.
    __builtin_amdgcn_s_setprio(1);
    float16_t s[2];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
#pragma unroll
      for (int r = 0; r < 16; ++r) s[mt][r] = 0.0f;
#pragma unroll
      for (int c = 0; c < DC; ++c) {
        const h8_t a = as_h8(*reinterpret_cast<const uint4 *>(
            k_lds + (32 * mt + n) * KS + 16 * c + 8 * h));
        s[mt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, qop[c], s[mt], 0, 0, 0);
      }
    }
    // Schedule: kReadAhead operand reads stay in flight ahead of the MFMAs
    // (one wave streams at most one 1 KB LDS operand per MFMA duration).
    __builtin_amdgcn_sched_group_barrier(kSchedDsRead, kReadAhead, 0);
#pragma unroll
    for (int k = 0; k < 2 * DC - kReadAhead; ++k) {
      __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
      __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(kSchedMfma, kReadAhead, 0);
    __builtin_amdgcn_s_setprio(0);
    // Online softmax of row n over this lane's 32 keys (MASK: causal and
    // length mask, needed only past the first row's window).
    int lim_rel = BN;
    if constexpr (MASK)
      lim_rel = (int)max(min((int64_t)lim - (int64_t)j0, (int64_t)BN), (int64_t)-1);
    float mx = -INFINITY;
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        if constexpr (MASK) {
          const int key_rel = 32 * mt + 8 * (r >> 2) + 4 * h + (r & 3);
          s[mt][r] = key_rel > lim_rel ? -INFINITY : s[mt][r];
        }
        mx = fmaxf(mx, s[mt][r]);
      }
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    // m_run is the reference max; it only moves when some row of the wave
    // outgrows it by 2^kRescaleLog2 (always on the first tile, as key 0 is
    // visible to every row).
    if (__any((mx - m_run) * c2 > kRescaleLog2)) {
      const float m_new = fmaxf(m_run, mx);
      const float alpha = exp2_raw((m_run - m_new) * c2);
      l_run *= alpha;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[dt][r] *= alpha;
      m_run = m_new;
    }
    const float mc = m_run * c2;
    uint32_t pw[2][8];  // P as packed f16 pairs, in accumulator order
    float psum = 0.0f;
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int r = 0; r < 16; r += 2) {
        const float p0 = exp2_raw(fmaf(s[mt][r], c2, -mc));
        const float p1 = exp2_raw(fmaf(s[mt][r + 1], c2, -mc));
        const uint32_t w = pack_f16x2(p0, p1);
        pw[mt][r >> 1] = w;
        // The row sum uses the same f16-rounded weights as P V.
        psum = dot2(w, 0x3c003c00u, psum);
      }
    l_run += psum;

    // O^T[d][row] += V^T[d][keys] P^T[keys][row], four 16-key chunks.
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int mt = c >> 1, base = (c & 1) * 4;
      const h8_t b = as_h8(make_uint4(pw[mt][base], pw[mt][base + 1],
                                      pw[mt][base + 2], pw[mt][base + 3]));
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const h8_t a = as_h8(*reinterpret_cast<const uint4 *>(
            v_lds + (32 * dt + n) * VS + 16 * c + 8 * h));
        o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, o[dt], 0, 0, 0);
      }
    }
    __builtin_amdgcn_sched_group_barrier(kSchedDsRead, kReadAhead, 1);
#pragma unroll
    for (int k = 0; k < 4 * DT - kReadAhead; ++k) {
      __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 1);
      __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 1, 1);
    }
    __builtin_amdgcn_sched_group_barrier(kSchedMfma, kReadAhead, 1);
    __builtin_amdgcn_s_setprio(0);
    // Tile it+1 (loaded during the previous tile) goes to the other stage,
    // whose last readers finished before the previous barrier; then the
    // loads for tile it+2 are issued to overlap the next tile's compute.
    if (it + 1 < n_tiles) store_tile((it + 1) & 1);
    __syncthreads();
    if (it + 2 < n_tiles) load_tile(j0 + 2 * BN);
  };

  // Tiles wholly inside the first row's window need no mask.
  const uint32_t n_full = (uint32_t)min((uint64_t)n_tiles, (full_lim + 1) / BN);
  load_tile(0);
  store_tile(0);
  if (n_tiles > 1) load_tile(BN);
  __syncthreads();
  uint32_t it = 0;
  for (; it < n_full; ++it) step(it, std::false_type{});
  for (; it < n_tiles; ++it) step(it, std::true_type{});

  // Normalise and store: lane (h, n) holds d = 32dt + 8q + 4h + 0..3.
  const float l_total = l_run + __shfl_xor(l_run, 32, 64);
  if (!row_ok) return;
  const float inv = 1.0f / l_total;
  uint16_t *orow =
      p.out + (int64_t)my_t * p.o_tok + (int64_t)(kvh * G + my_g) * p.o_head;
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      uint2 v;
      v.x = pack_f16x2(o[dt][4 * q] * inv, o[dt][4 * q + 1] * inv);
      v.y = pack_f16x2(o[dt][4 * q + 2] * inv, o[dt][4 * q + 3] * inv);
      *reinterpret_cast<uint2 *>(orow + 32 * dt + 8 * q + 4 * h) = v;
    }
}

}  // namespace

bool prefill_supported(uint32_t head_dim) {
  return head_dim == 64 || head_dim == 128;
}

hipError_t launch_prefill(const PrefillParams &p, uint32_t head_dim, const Launch &l) {
  const dim3 grid(p.row_tiles, p.kv_heads);
  switch (head_dim) {
    case 64: return dispatch(attn_prefill_kernel<64>, grid, dim3(THREADS), 0, l, p);
    case 128: return dispatch(attn_prefill_kernel<128>, grid, dim3(THREADS), 0, l, p);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace kernels
}  // namespace mi
