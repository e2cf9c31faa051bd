// MFMA flash prefill for gfx950 (AttentionKind::FlashPrefill at D = 32, 64, 128,
// 256).
//
// Replaces attention_flash_prefill_f16 (transformer.metal:1667-1822) with a
// CDNA4 design:
//  - GQA packing: a workgroup owns 128 rows of the packed (token, head in
//    group) dimension of ONE KV head, so each K/V tile is staged into LDS once
//    for all G query heads that share it;
//  - S^T = K Q^T on v_mfma_f32_32x32x16_f16, K read from LDS as the A
//    operand and Q^T kept in registers as the B operand. Each lane then holds
//    one query row's scores, so the f32 online softmax is lane-local (plus an
//    exchange with the partner half-wave when the row's reference max moves);
//  - O^T += V^T P^T on the same MFMA: P^T is the S^T accumulator converted to
//    f16 in place (no shuffles), because V is transposed into LDS with its
//    keys permuted (bits 2 and 3 of the key index swapped) to match the order
//    in which the S^T accumulator holds them;
//  - the next tile's K/V global loads are in flight while the current tile
//    is computed; causally heavy row tiles are dispatched first (split plans:
//    longest piece first, each CU's long piece paired with a short one).
#include <type_traits>

#include "device_common.hpp"
#include "kernels.hpp"
#include "timeline.hpp"

namespace mi {
namespace kernels {
namespace {

using namespace mi::dev;

constexpr int BN = kPrefillBlockN;  // keys per KV tile

#ifdef MI_TIMELINE
__device__ uint64_t prefill_timeline[kTimelineSlots * kTimelineFields];
#endif

// Column of key `key` (0..63 within a tile) in the transposed V tile: bits
// 2 and 3 swapped, which is the key order of the P operand (see above).
__device__ __forceinline__ int vt_col(int key) {
  return (key & ~12) | ((key & 4) << 1) | ((key & 8) >> 1);
}

// Direct-load tile layout (D = 64, 128): a tile row of D halves is 2D bytes
// in 16-byte chunks, the chunks of row r XOR-swizzled so that the K operand
// reads (16 rows, one chunk each) and the V^T transpose reads (four rows,
// eight bytes per lane) of 16 / 32 lanes fall on distinct banks. D = 128
// (256-byte rows span the 64 banks): K chunk ^ (r & 15), V chunk ^ 4 (r & 3).
// D = 64 (128-byte rows, two per bank row): rows 2m and 2m + 1 already sit
// in opposite bank halves, so K uses chunk ^ ((r >> 1) & 7) and V
// chunk ^ 4 ((r >> 1) & 1).
template <int D>
__device__ __forceinline__ int k_swizzle(int r) {
  return D == 128 ? (r & 15) : ((r >> 1) & 7);
}
template <int D>
__device__ __forceinline__ int v_swizzle(int r) {
  return D == 128 ? ((r & 3) << 2) : (((r >> 1) & 1) << 2);
}

// Output staging (the rows of one wave as f16 in LDS): 16-byte chunk c of
// row r sits at chunk c ^ out_swizzle(r), so that the writes (one chunk of
// 32 rows per instruction) and the reads (whole rows) spread over the banks.
template <int D>
__device__ __forceinline__ int out_swizzle(int r) {
  constexpr int CPR = D / 8, RB = D >= 128 ? 1 : 128 / D;  // rows per 256 bytes
  return (r / RB) & (CPR - 1);
}

__device__ __forceinline__ uint4 load16(const uint16_t *p) {
  return *reinterpret_cast<const uint4 *>(p);
}

// Packs the f16 halves of words a and b: lo -> (a.lo, b.lo), hi -> (a.hi, b.hi).
__device__ __forceinline__ uint32_t pack_lo(uint32_t a, uint32_t b) {
  return __builtin_amdgcn_perm(b, a, 0x05040100u);
}
__device__ __forceinline__ uint32_t pack_hi(uint32_t a, uint32_t b) {
  return __builtin_amdgcn_perm(b, a, 0x07060302u);
}

// sched_group_barrier instruction classes (LLVM AMDGPU): MFMA, LDS read.
constexpr int kSchedMfma = 0x008;
constexpr int kSchedDsRead = 0x100;
constexpr int kReadAhead = 4;

// BMT packed rows per workgroup, 32 per wave: 128 (4 waves, two workgroups
// per CU) or, for D = 128 grids of at least four workgroups per CU, 256 (8
// waves sharing each K/V tile, one workgroup per CU). D = 256 runs one
// 4-wave workgroup per CU: its Q operand and O accumulators (64 + 128
// registers per lane) leave room for one wave per SIMD, and its two LDS
// stages take 141 KB. ORDERED: a split plan whose pieces run in the host's
// order (PrefillParams::order); a separate instantiation, so that the other
// launches do not wait on the order entry's load.
template <int D, int BMT, bool ORDERED>
__global__ __launch_bounds__(BMT * 2, (BMT == 128 && D <= 128) ? 2 : 1) void attn_prefill_kernel(
    const PrefillParams p) {
  constexpr int BM = BMT;
  constexpr int THREADS = BMT * 2;
  constexpr int WAVES = THREADS / 64;
  constexpr int BPW = BN * D * 2 / 1024 / WAVES;  // 1 KB blocks per wave of each K / V tile
  constexpr int CPR = D / 8;          // 16-byte chunks per tile row
  constexpr int RPB = 1024 / (2 * D); // tile rows per 1 KB block
  static_assert(BM == 128 || (BM == 256 && D == 128), "row tile");
  static_assert(D == 32 || D == 64 || D == 128 || D == 256, "head_dim");
  constexpr int DC = D / 16;          // 16-wide d chunks of Q K^T
  constexpr int DT = D / 32;          // 32-row d tiles of O^T
  constexpr int KS = D + 8;           // K tile row stride (halves)
  constexpr int VS = BN + 8;          // V^T tile row stride (halves)
  constexpr int K_CHUNKS = BN * D / 8 / THREADS;           // 16-B pieces
  constexpr int V_JOBS = (BN / 4) * (D / 8);                // 4 keys x 8 d
  constexpr int V_PER = (V_JOBS + THREADS - 1) / THREADS;
  // Two LDS stages: tile i is read from one while tile i+1 is written into
  // the other, so one barrier per tile suffices.
  // D = 64, 128: K and V tiles arrive by direct global->LDS loads as rows
  // of 16-byte chunks, XOR-swizzled (k_swizzle, v_swizzle) so that the K
  // operand reads and the V^T transpose reads are free of bank conflicts.
  // D = 32, 256: register staging, K padded, V stored transposed (at D = 32
  // a K row is 64 bytes, two S MFMAs deep, and O^T one 32-row d tile).
  constexpr bool DIRECT = D == 64 || D == 128;
  constexpr int K_ELEMS = DIRECT ? BN * D : BN * KS;
  constexpr int V_ELEMS = DIRECT ? BN * D : D * VS;
  // One array per stage (and the stage a compile-time choice in the loop),
  // so alias analysis can tell the direct loads into one stage from the
  // reads of the other and no wait for in-flight loads is inserted before
  // every LDS read.
  __shared__ __attribute__((aligned(16))) uint16_t k_lds_a[K_ELEMS], k_lds_b[K_ELEMS];
  __shared__ __attribute__((aligned(16))) uint16_t v_lds_a[V_ELEMS], v_lds_b[V_ELEMS];
  auto k_stage = [&](int st) __attribute__((always_inline)) -> uint16_t * { return st ? k_lds_b : k_lds_a; };
  auto v_stage = [&](int st) __attribute__((always_inline)) -> uint16_t * { return st ? v_lds_b : v_lds_a; };

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int n = lane & 31, h = lane >> 5;
  const uint32_t G = p.group;
#ifdef MI_TIMELINE
  const TimelineRow tl = timeline_start(
      prefill_timeline, blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z), tid == 0);
#else
  const TimelineRow tl;
#endif
  // Dispatch order: workgroups are handed out in linear-id order, and
  // round-robin over the 8 XCDs, so id % 8 selects the XCD. When the KV
  // heads split evenly over the XCDs, each XCD gets whole heads (their K/V
  // stay in its L2). Within a head, an ordered split plan runs its pieces in
  // the host's order (p.order); otherwise row tiles go heaviest first and
  // the gridDim.z key splits of one row tile go together, a split past the
  // row tile's last key tile returning at once.
  uint32_t tile, kvh, split;
  {
    const uint32_t id = blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z);
    const uint32_t H = p.kv_heads, S = gridDim.z;
    uint32_t rest;
    if (H % 8 == 0) {
      const uint32_t xcd = id % 8, k = id / 8, per = H / 8;
      kvh = xcd * per + k % per;
      rest = k / per;
    } else {
      kvh = id % H;
      rest = id / H;
    }
    if constexpr (ORDERED) {
      const uint32_t piece = p.order[rest];
      tile = piece >> 4;
      split = piece & 15;
    } else {
      tile = p.row_tiles - 1 - rest / S;
      split = rest % S;
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
  // This split's key tiles [t_begin, t_end), and whether the row tile has
  // other splits.
  const uint32_t per_split = p.split_tiles != 0 ? p.split_tiles : n_tiles;
  uint32_t t_begin, t_end;
  bool partial_out;
  tl.set(7, (uint64_t)tile | (uint64_t)split << 16);
  if constexpr (ORDERED) {
    const uint32_t nsplit = (n_tiles + per_split - 1) / per_split;
    if (split >= nsplit) {  // not in a plan the host made
      tl.now(2);
      return;
    }
    t_begin = split * n_tiles / nsplit;
    t_end = (split + 1) * n_tiles / nsplit;
    partial_out = nsplit > 1;
  } else {
    t_begin = split * per_split;
    if (t_begin >= n_tiles) {  // the row tile needs fewer splits
      tl.now(2);
      return;
    }
    t_end = min(n_tiles, t_begin + per_split);
    partial_out = n_tiles > per_split;
  }
  tl.set(7, (uint64_t)tile | (uint64_t)split << 16 | (uint64_t)t_begin << 20 |
                (uint64_t)t_end << 40);
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
    uint16_t *k_lds = k_stage(stage);
    uint16_t *v_lds = v_stage(stage);
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

  // Direct loads of tile `ti` into LDS stage `stage`: each wave fills BPW
  // 1 KB blocks (RPB tile rows each), lane L writing bytes 16L..16L+15 of a
  // block, so the lane fetches the global 16 bytes that belong at that
  // swizzled position.
  // Full tiles: loop-invariant per-lane byte offsets from a wave-uniform
  // tile base (scalar base + 32-bit vector offset per load).
  uint32_t k_off[BPW], v_off[BPW];
#pragma unroll
  for (int i = 0; i < BPW; ++i) {
    const int row = (wave * BPW + i) * RPB + lane / CPR, pc = lane % CPR;
    k_off[i] = (uint32_t)(row * p.k_pos + ((pc ^ k_swizzle<D>(row)) * 8)) * 2u;
    v_off[i] = (uint32_t)(row * p.v_pos + ((pc ^ v_swizzle<D>(row)) * 8)) * 2u;
  }
  auto issue_tile = [&](uint32_t ti, int stage) {
    const uint32_t j0 = ti * BN;
    const uint16_t *kt = kbase + (int64_t)j0 * p.k_pos;
    const uint16_t *vt = vbase + (int64_t)j0 * p.v_pos;
    if (j0 + BN <= kmax) {
#pragma unroll
      for (int i = 0; i < BPW; ++i) {
        const int blk = wave * BPW + i;
        load_lds16(reinterpret_cast<const uint16_t *>(reinterpret_cast<const char *>(kt) + k_off[i]),
                   k_stage(stage) + blk * 512);
        load_lds16(reinterpret_cast<const uint16_t *>(reinterpret_cast<const char *>(vt) + v_off[i]),
                   v_stage(stage) + blk * 512);
      }
      return;
    }
    // Partial last tile: rows past the last key re-read that key.
    const int last = (int)(kmax - 1 - j0);
#pragma unroll
    for (int i = 0; i < BPW; ++i) {
      const int blk = wave * BPW + i;
      const int row = blk * RPB + lane / CPR;
      const int pc = lane % CPR;
      const int rr = min(row, last);
      load_lds16(kt + (uint32_t)(rr * p.k_pos + ((pc ^ k_swizzle<D>(row)) * 8)),
                 k_stage(stage) + blk * 512);
      load_lds16(vt + (uint32_t)(rr * p.v_pos + ((pc ^ v_swizzle<D>(row)) * 8)),
                 v_stage(stage) + blk * 512);
    }
  };
  // Lane roles in the V^T transpose reads (ds_read_b64_tr_b16): within each
  // 16-lane group g, output lane 4a + b, element j receives element b of the
  // 8 bytes addressed by lane a + 4j. Lane (a4, jj) of group g therefore
  // addresses key 4 (g / 2) + jj (+ 8 for the second read) at d offset
  // 16 (g % 2) + 4 a4, so output lane (h, n) gets 4 keys of column n.
  const int tr_g = lane >> 4, tr_a = lane & 3, tr_j = (lane >> 2) & 3;
  const int tr_key = 4 * (tr_g >> 1) + tr_j;
  const int tr_off = tr_key * D + 4 * (tr_a & 1);
  const int tr_chunk = 2 * (tr_g & 1) + (tr_a >> 1);

  auto step = [&](uint32_t it, auto mask_tag, auto stage_tag) {
    constexpr bool MASK = decltype(mask_tag)::value;
    constexpr int ST = decltype(stage_tag)::value;  // LDS stage of tile it
    const uint32_t j0 = it * BN;
    const uint16_t *k_lds = ST ? k_lds_b : k_lds_a;
    const uint16_t *v_lds = ST ? v_lds_b : v_lds_a;

    // S^T[key][row] for the 64 keys of the tile: two 32-key M tiles. MFMA
    // phases run at raised wave priority (measured on MI355X, 256-row tiles:
    // c5 2.27 ms with it, 2.33-2.35 ms without).
    __builtin_amdgcn_s_setprio(1);
    float16_t s[2];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
#pragma unroll
      for (int r = 0; r < 16; ++r) s[mt][r] = 0.0f;
#pragma unroll
      for (int c = 0; c < DC; ++c) {
        const uint16_t *kp;
        if constexpr (DIRECT)
          kp = k_lds + (32 * mt + n) * D + (((2 * c + h) ^ k_swizzle<D>(n)) * 8);
        else
          kp = k_lds + (32 * mt + n) * KS + 16 * c + 8 * h;
        const h8_t a = as_h8(*reinterpret_cast<const uint4 *>(kp));
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
    if constexpr (MASK) {
      // Key 32 mt + 8 (r >> 2) + 4 h + (r & 3) of the tile is visible when
      // it is at most lim_rel. The lane's 4 h moves to the limit, so each
      // compare is against a constant (no per-key lane values to keep).
      const int lim_rel = (int)max(min((int64_t)lim - (int64_t)j0, (int64_t)BN), (int64_t)-1);
      const int lim_lane = lim_rel - 4 * h;
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key_c = 32 * mt + 8 * (r >> 2) + (r & 3);
          s[mt][r] = key_c > lim_lane ? -INFINITY : s[mt][r];
        }
    }
    // P = 2^(s c2 - m_ref c2) against the row's reference max m_run, as f16
    // pairs in accumulator order; the row sum uses the same f16-rounded
    // weights as P V (two partial sums, to halve the dependent chain).
    uint32_t pw[2][8];
    float psum;
    auto weights = [&](float mc) __attribute__((always_inline)) {
      float ps0 = 0.0f, ps1 = 0.0f;
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int r = 0; r < 16; r += 2) {
          const float p0 = exp2_raw(fmaf(s[mt][r], c2, -mc));
          const float p1 = exp2_raw(fmaf(s[mt][r + 1], c2, -mc));
          const uint32_t w = pack_f16x2(p0, p1);
          pw[mt][r >> 1] = w;
          if (r & 2)
            ps1 = dot2(w, 0x3c003c00u, ps1);
          else
            ps0 = dot2(w, 0x3c003c00u, ps0);
        }
      psum = ps0 + ps1;
    };
    // The reference max moves only when a weight leaves f16's range: the
    // row sum is then +inf (a weight rounded to f16 infinity) or NaN. A row
    // without a reference yet (m_run = -inf, so -mc = +inf) always lands
    // there. Until then every weight is at most 65504 (f16's largest finite
    // value), and O and l share the reference, so no max pass is needed.
    weights(m_run * c2);
    if (__any(!(psum <= __FLT_MAX__))) {
      float mx = -INFINITY;
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[mt][r]);
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      const float m_new = fmaxf(m_run, mx);
      // A row that has seen no visible key yet (only possible in a later
      // key split) keeps m = -inf and nothing to rescale.
      const float alpha = m_new == -INFINITY ? 1.0f : exp2_raw((m_run - m_new) * c2);
      l_run *= alpha;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[dt][r] *= alpha;
      m_run = m_new;
      weights(m_run == -INFINITY ? 0.0f : m_run * c2);
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
        h8_t a;
        if constexpr (DIRECT) {
          const int sw = ((4 * dt + tr_chunk) ^ v_swizzle<D>(tr_key)) * 8;
          const uint16_t *v0 = v_lds + 16 * c * D + tr_off + sw;
          const uint2 l2 = read_tr16(v0), h2 = read_tr16(v0 + 8 * D);
          a = as_h8(make_uint4(l2.x, l2.y, h2.x, h2.y));
        } else {
          a = as_h8(*reinterpret_cast<const uint4 *>(v_lds + (32 * dt + n) * VS + 16 * c + 8 * h));
        }
        o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, o[dt], 0, 0, 0);
      }
    }
    constexpr int PV_READS = DIRECT ? 2 : 1;  // LDS reads per PV MFMA
    __builtin_amdgcn_sched_group_barrier(kSchedDsRead, PV_READS * kReadAhead, 1);
#pragma unroll
    for (int k = 0; k < 4 * DT - kReadAhead; ++k) {
      __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 1);
      __builtin_amdgcn_sched_group_barrier(kSchedDsRead, PV_READS, 1);
    }
    __builtin_amdgcn_sched_group_barrier(kSchedMfma, kReadAhead, 1);
    __builtin_amdgcn_s_setprio(0);
    // Tile it+1 (loaded during the previous tile) goes to the other stage,
    // whose last readers finished before the previous barrier; then the
    // loads for tile it+2 are issued to overlap the next tile's compute.
    if constexpr (DIRECT) {
      // Tile it+1 (issued a tile ago) has landed in every wave's part of
      // the other stage; after the barrier nobody reads this stage, which
      // then receives tile it+2.
      __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
      __syncthreads();
      if (it + 2 < t_end) issue_tile(it + 2, ST);
    } else {
      if (it + 1 < t_end) store_tile(ST ^ 1);
      __syncthreads();
      if (it + 2 < t_end) load_tile(j0 + 2 * BN);
    }
  };

  // Tiles wholly inside the first row's window need no mask.
  const uint32_t n_full = (uint32_t)min((uint64_t)t_end, (full_lim + 1) / BN);
  // Tile t_begin + k lives in stage k & 1.
  if constexpr (DIRECT) {
    // The first tile is computed once it (and the Q rows, loaded earlier)
    // has landed; the second stays in flight. Loads complete in issue order,
    // so vmcnt(2 BPW) leaves only the second tile's 2 BPW loads pending.
    // The barrier is a bare s_barrier (no fence: a workgroup-scope fence
    // would wait for every load, the second tile's too); each wave has
    // waited for its own part of the first tile, and the memory clobber
    // keeps the compiler from moving LDS reads above it.
    issue_tile(t_begin, 0);
    if (t_begin + 1 < t_end) {
      issue_tile(t_begin + 1, 1);
      static_assert(2 * BPW < 16, "vmcnt immediate");
      __builtin_amdgcn_s_waitcnt(kWaitVmcnt0 | (2 * BPW));
    } else {
      __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
    }
    asm volatile("s_barrier" ::: "memory");
  } else {
    load_tile(t_begin * BN);
    store_tile(0);
    if (t_begin + 1 < t_end) load_tile((t_begin + 1) * BN);
    __syncthreads();
  }
  tl.now(3);
  using S0 = std::integral_constant<int, 0>;
  using S1 = std::integral_constant<int, 1>;
  uint32_t it = t_begin;
  for (; it + 1 < n_full; it += 2) {
    step(it, std::false_type{}, S0{});
    step(it + 1, std::false_type{}, S1{});
  }
  if (it < n_full) {
    step(it, std::false_type{}, S0{});
    ++it;
  }
  // The masked tail continues the stage alternation.
  if (((it - t_begin) & 1) != 0 && it < t_end) {
    step(it, std::true_type{}, S1{});
    ++it;
  }
  for (; it + 1 < t_end; it += 2) {
    step(it, std::true_type{}, S0{});
    step(it + 1, std::true_type{}, S1{});
  }
  if (it < t_end) step(it, std::true_type{}, S0{});

  const float l_total = l_run + __shfl_xor(l_run, 32, 64);
  tl.now(4);
  if (partial_out) {
    // Publish this split's rows with device-scope stores, wait until they
    // have completed, then count the arrival. The last split of the row tile
    // merges; the others are done. Each row goes out as (m, l) in f32 and O
    // normalised by its own l in f16 (half the bytes of f32 O: the merger
    // reads every other split's partial, and the publication and that read
    // are bound by bytes, not round trips; measured on MI355X, c3: f32 O
    // ~33.5 us per call against ~31.5 us with half as many bytes). The
    // merger uses the same rounded values for its own split, so the result
    // does not depend on which split arrives last. Layout per wave, in the
    // accumulator's own order so every store and load moves 512 contiguous
    // bytes: 8-byte slot 0 = (m, l), slot 1 + 4dt + q = O values 4q .. 4q + 3
    // of d tile dt, each slot 64 lanes wide.
    constexpr uint32_t SLOTS = kPrefillPartialSlots(D);
    const size_t split_stride = (size_t)p.row_tiles * p.kv_heads * WAVES * SLOTS * 64 * 2;
    float *wave_base =
        p.partial + ((((size_t)tile * p.kv_heads + kvh) * WAVES + wave) * SLOTS * 64 + lane) * 2;
    // A row without a visible key in this split (l = 0) publishes O = 0.
    const float inv_own = l_total > 0.0f ? 1.0f / l_total : 0.0f;
    uint32_t own[DT][8];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        own[dt][2 * q] = pack_f16x2(o[dt][4 * q] * inv_own, o[dt][4 * q + 1] * inv_own);
        own[dt][2 * q + 1] = pack_f16x2(o[dt][4 * q + 2] * inv_own, o[dt][4 * q + 3] * inv_own);
      }
    {
      float *mine = wave_base + split * split_stride;
      store_partial2(mine, m_run, l_total);
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          store_partial_words(mine + (1 + 4 * dt + q) * 128, own[dt][2 * q], own[dt][2 * q + 1]);
    }
    __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
    __shared__ uint32_t s_last;
    __syncthreads();
    tl.now(5);
    // Both plans cut a row tile into ceil(n_tiles / split_tiles) splits.
    const uint32_t nsplit = (n_tiles + per_split - 1) / per_split;
    if (tid == 0) {
      uint32_t *counter = p.counters + (size_t)(tile * p.kv_heads + kvh) * p.counter_stride;
      const uint32_t arrived = arrive(counter);
      const bool last = arrived == nsplit - 1;
      if (last) {
        acquire_partials();
        __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      s_last = last;
      if (last) tl.add(7, 1ull << 63);
    }
    __syncthreads();
    tl.now(6);
    if (s_last == 0) {
      tl.now(2);
      return;
    }
    // Log-sum-exp merge in split order (deterministic whichever split
    // arrives last): O = sum_s O_s l_s 2^(m_s - M) / sum_s l_s 2^(m_s - M).
    // Split 0 holds key 0, so M is finite; a split in which a row saw no key
    // has m = -inf and weight 0.
    const float c2 = p.scale_log2;
    float ms[kMaxPrefillSplits], ls[kMaxPrefillSplits];
    float M = -INFINITY;
#pragma unroll
    for (int s = 0; s < (int)kMaxPrefillSplits; ++s) {
      if (s >= (int)nsplit) break;
      float2 ml = make_float2(m_run, l_total);
      if (s != (int)split) ml = load_partial2(wave_base + s * split_stride);
      ms[s] = ml.x;
      ls[s] = ml.y;
      M = fmaxf(M, ml.x);
    }
    float lsum = 0.0f;
    float16_t acc[DT];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[dt][r] = 0.0f;
#pragma unroll
    for (int s = 0; s < (int)kMaxPrefillSplits; ++s) {
      if (s >= (int)nsplit) break;
      const float w = exp2_raw((ms[s] - M) * c2);
      lsum = fmaf(ls[s], w, lsum);
      const float lw = ls[s] * w;
      // The split's O words: this split's from registers, another's loaded
      // (all of them in one round).
      uint32_t words[DT][8];
      if (s == (int)split) {
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
          for (int i = 0; i < 8; ++i) words[dt][i] = own[dt][i];
      } else {
        const float *src = wave_base + s * split_stride;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const uint2 v = load_partial_words(src + (1 + 4 * dt + q) * 128);
            words[dt][2 * q] = v.x;
            words[dt][2 * q + 1] = v.y;
          }
      }
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          acc[dt][2 * i] = fmaf(f16_to_f32((uint16_t)words[dt][i]), lw, acc[dt][2 * i]);
          acc[dt][2 * i + 1] = fmaf(f16_to_f32((uint16_t)(words[dt][i] >> 16)), lw, acc[dt][2 * i + 1]);
        }
    }
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[dt][r] = acc[dt][r];
    l_run = lsum;  // the normalisation below divides by the merged sum
  }

  // Normalise, then store through LDS: lane (h, n) holds d = 32dt + 8q +
  // 4h + 0..3 of row n, so stored directly every instruction would write
  // 8-byte pieces of 32 rows. Each wave instead writes its 32 rows as f16
  // into a region of the (now idle) K/V stages, chunks XOR-swizzled per row
  // (out_swizzle), and stores them back as whole 16-byte chunks, D / 8
  // consecutive lanes per row. Rows past the last token are not stored.
  const float inv = 1.0f / (partial_out ? l_run : l_total);
  constexpr int CPR_OUT = D / 8;           // 16-byte chunks per output row
  constexpr int RPI = 64 / CPR_OUT;        // rows per store instruction
  static_assert(2 * 32 * D <= K_ELEMS && 2 * 32 * D <= V_ELEMS, "output staging");
  __syncthreads();  // every wave is past its last LDS operand read
  uint16_t *rows_lds =
      (wave < 2 ? k_lds_a : wave < 4 ? k_lds_b : wave < 6 ? v_lds_a : v_lds_b) + (wave & 1) * 32 * D;
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      uint2 v;
      v.x = pack_f16x2(o[dt][4 * q] * inv, o[dt][4 * q + 1] * inv);
      v.y = pack_f16x2(o[dt][4 * q + 2] * inv, o[dt][4 * q + 3] * inv);
      const int chunk = (4 * dt + q) ^ out_swizzle<D>(n);
      *reinterpret_cast<uint2 *>(rows_lds + n * D + chunk * 8 + 4 * h) = v;
    }
  __syncthreads();
  // The lane index and the wave's first packed row are derived afresh (lane
  // from mbcnt, the row from scalars) rather than taken from the prologue,
  // whose values the compiler would otherwise keep, or spill, across the loop.
  const int lane_o = (int)__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
  const int c_out = lane_o % CPR_OUT;
  const uint32_t wave_row0 = row0 + (uint32_t)__builtin_amdgcn_readfirstlane(wave) * 32;
#pragma unroll
  for (int i = 0; i < 32 / RPI; ++i) {
    const int r = i * RPI + lane_o / CPR_OUT;
    const uint4 v = *reinterpret_cast<const uint4 *>(rows_lds + r * D +
                                                     (c_out ^ out_swizzle<D>(r)) * 8);
    const uint32_t prow = wave_row0 + r;
    const uint32_t t = prow / G, g = prow % G;
    if (t < p.tokens)
      *reinterpret_cast<uint4 *>(p.out + (int64_t)t * p.o_tok + (int64_t)(kvh * G + g) * p.o_head +
                                 c_out * 8) = v;
  }
  tl.now(2);
}

}  // namespace

bool prefill_supported(uint32_t head_dim) {
  return head_dim == 32 || head_dim == 64 || head_dim == 128 || head_dim == 256;
}

hipError_t launch_prefill(const PrefillParams &p, uint32_t head_dim, const Launch &l) {
  // One workgroup per piece of an ordered split plan, else per (row tile, KV
  // head, key split).
  const dim3 grid = p.pieces_per_head != 0
                        ? dim3(p.pieces_per_head, p.kv_heads, 1)
                        : dim3(p.row_tiles, p.kv_heads, p.splits > 1 ? p.splits : 1);
  const bool ordered = p.pieces_per_head != 0;
  if (ordered && (p.pieces_per_head > kPrefillOrderMax || p.block_m != 128 || head_dim > 128))
    return hipErrorInvalidValue;
  switch (head_dim) {
    case 32:
      if (p.block_m != 128) return hipErrorInvalidValue;
      return ordered ? dispatch(attn_prefill_kernel<32, 128, true>, grid, dim3(256), 0, l, p)
                     : dispatch(attn_prefill_kernel<32, 128, false>, grid, dim3(256), 0, l, p);
    case 64:
      if (p.block_m != 128) return hipErrorInvalidValue;
      return ordered ? dispatch(attn_prefill_kernel<64, 128, true>, grid, dim3(256), 0, l, p)
                     : dispatch(attn_prefill_kernel<64, 128, false>, grid, dim3(256), 0, l, p);
    case 128:
      if (p.block_m == 256)
        return dispatch(attn_prefill_kernel<128, 256, false>, grid, dim3(512), 0, l, p);
      if (p.block_m != 128) return hipErrorInvalidValue;
      return ordered ? dispatch(attn_prefill_kernel<128, 128, true>, grid, dim3(256), 0, l, p)
                     : dispatch(attn_prefill_kernel<128, 128, false>, grid, dim3(256), 0, l, p);
    case 256:
      if (p.block_m != 128) return hipErrorInvalidValue;
      return dispatch(attn_prefill_kernel<256, 128, false>, grid, dim3(256), 0, l, p);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace kernels
}  // namespace mi

#ifdef MI_TIMELINE
extern "C" int32_t mi_timeline_read_prefill(void *dst, uint64_t bytes) {
  const uint64_t cap = sizeof(uint64_t) * mi::dev::kTimelineSlots * mi::dev::kTimelineFields;
  if (dst == nullptr || bytes > cap) return hipErrorInvalidValue;
  return hipMemcpyFromSymbol(dst, HIP_SYMBOL(mi::kernels::prefill_timeline), bytes, 0,
                             hipMemcpyDeviceToHost);
}
#endif
