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
//  - with more than one split, each split writes a (max, sum, acc[D])
//    partial. Either the unit's last split merges them in the same launch
//    (device-scope partial stores, a wait for their completion, then an
//    arrival counter: no cache-wide release fence, which on a multi-XCD part
//    writes back the XCD's whole L2 and measured slower than a second
//    launch), or attn_merge_kernel does in a second launch.
// The batched decode at head_dim 128 has its own kernel further down
// (attn_decode_stream_kernel: MFMA tiles, stream-K split).
#include <type_traits>

#include "device_common.hpp"
#include "kernels.hpp"
#include "timeline.hpp"

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

// K/V rows are streamed: a decode reads each cache byte once, so the loads
// carry the non-temporal hint and do not displace reusable lines (measured
// on MI355X: +6-9% on the 32-sequence batched decode).
template <int VEC>
__device__ __forceinline__ Vec<VEC> load_vec_stream(const uint16_t *ptr) {
  Vec<VEC> r;
  if constexpr (VEC == 8) {
    typedef unsigned u4_t __attribute__((ext_vector_type(4)));
    const u4_t x = __builtin_nontemporal_load(reinterpret_cast<const u4_t *>(ptr));
    r.w[0] = x.x, r.w[1] = x.y, r.w[2] = x.z, r.w[3] = x.w;
  } else if constexpr (VEC == 4) {
    typedef unsigned u2_t __attribute__((ext_vector_type(2)));
    const u2_t x = __builtin_nontemporal_load(reinterpret_cast<const u2_t *>(ptr));
    r.w[0] = x.x, r.w[1] = x.y;
  } else if constexpr (VEC == 2) {
    r.w[0] = __builtin_nontemporal_load(reinterpret_cast<const uint32_t *>(ptr));
  } else {
    r.w[0] = __builtin_nontemporal_load(ptr);
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

// Log-sum-exp combine of split partials, the reference's reduce kernels
// (transformer.metal:2251-2316). `base` holds nsplits consecutive partials
// of GC heads, (max, sum, acc[D]) each; the result goes to
// out[g * o_head + d]. Each output element loads every split's (max, sum,
// acc[d]) at once, kMergeChunk splits per pass, so a merge costs one memory
// round trip per pass (measured on MI355X at c2, 16 splits: 7.9 us per call
// against 8.5 us when the partials were staged through LDS first). COHERENT:
// the partials come from other workgroups of this launch (device-scope
// loads after the acquire that follows the last arrival).
constexpr int kMergeChunk = 16;

// CHUNK: splits per pass (a merge of fewer splits still loads a whole pass,
// re-reading the last split with weight 0).
template <int D, int GC, int THREADS, bool COHERENT, int CHUNK = kMergeChunk>
__device__ __forceinline__ void merge_direct(const float *base, uint32_t nsplits, uint16_t *out,
                                             int64_t o_head) {
  constexpr int ROW = D + 2;
  auto load = [](const float *ptr) __attribute__((always_inline)) {
    if constexpr (COHERENT) return load_partial(ptr);
    else return *ptr;
  };
  for (int idx = threadIdx.x; idx < GC * D; idx += THREADS) {
    const int g = idx / D, d = idx % D;
    float M = -INFINITY, Ls = 0.0f, As = 0.0f;
    for (uint32_t s0 = 0; s0 < nsplits; s0 += CHUNK) {
      float m[CHUNK], l[CHUNK], a[CHUNK];
#pragma unroll
      for (int i = 0; i < CHUNK; ++i) {
        // Past the last split a lane re-reads it (in bounds) with weight 0.
        const float *ps = base + (size_t)(min(s0 + i, nsplits - 1) * GC + g) * ROW;
        m[i] = load(ps);
        l[i] = load(ps + 1);
        a[i] = load(ps + 2 + d);
        if (s0 + i >= nsplits) m[i] = -INFINITY;
      }
      float cm = M;
#pragma unroll
      for (int i = 0; i < CHUNK; ++i) cm = fmaxf(cm, m[i]);
      // A split (or a whole pass) with no visible key has max -inf, weight 0.
      const float r = M == -INFINITY ? 0.0f : exp2_raw(M - cm);
      Ls *= r;
      As *= r;
#pragma unroll
      for (int i = 0; i < CHUNK; ++i) {
        const float f = m[i] == -INFINITY ? 0.0f : exp2_raw(m[i] - cm);
        Ls = fmaf(l[i], f, Ls);
        As = fmaf(a[i], f, As);
      }
      M = cm;
    }
    out[g * o_head + d] = f32_to_f16(As / Ls);
  }
}

template <int D, int GC, int THREADS, bool COHERENT>
__device__ __forceinline__ void merge_splits(const RowsParams &p, uint32_t unit,
                                             uint32_t nsplits, uint16_t *out) {
  merge_direct<D, GC, THREADS, COHERENT>(p.partial + (size_t)unit * p.max_splits * GC * (D + 2),
                                         nsplits, out, p.o_head);
}

// qk_norm_rope_cache's per-head transform (ops.rs:917-977,
// transformer.metal:1533-1577) of one D = 128 row held as the rows kernel
// holds it: 16 lanes, lane `col` with elements 8 col .. 8 col + 7 (and the
// same elements of the weight). The RoPE partner of element d < 64 is d + 64,
// held by lane col ^ 8 (first: col < 8); cs / sn are the cosines and sines of
// this lane's 8 pairs. Per element the f32 steps are
// those of qk_norm_rope_kernel; the row sum adds the squares in another order.
__device__ __forceinline__ Vec<8> norm_rope_row(const Vec<8> &raw, const Vec<8> &weight,
                                                const float *cs, const float *sn, float eps,
                                                bool first) {
#pragma clang fp contract(off)
  float x[8], n[8];
  float sum = 0.0f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    x[e] = elem<8>(raw, e);
    sum += x[e] * x[e];
  }
  sum = lane_group_sum<16>(sum);
  const float scale = 1.0f / sqrtf(sum / 128.0f + eps);
#pragma unroll
  for (int e = 0; e < 8; ++e) n[e] = x[e] * scale * elem<8>(weight, e);
  Vec<8> r;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    uint32_t h[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int e = 2 * w + t;
      const float m = dpp_f32<kDppRowRor8>(n[e]);  // lane col ^ 8 of the 16
      // First halves x c - y s, second halves y s + x c (y, x: partner's),
      // both as n c + (-+ m s) without a branch.
      const float ms = m * sn[e];
      h[t] = f32_to_f16(n[e] * cs[e] + (first ? -ms : ms));
    }
    r.w[w] = h[0] | (h[1] << 16);
  }
  return r;
}

// FUSED: with more than one split, each split publishes its partial with
// device-scope stores and counts its arrival on the unit's counter; the last
// split to arrive merges all of them in split order (no second launch).
// STEP: the decode step (RowsParams::step_k), D = 128 and one token only.
#ifdef MI_TIMELINE
__device__ uint64_t rows_timeline[kTimelineSlots * kTimelineFields];
#endif

template <int D, int WAVES, int GC, bool FUSED, bool STEP = false>
__global__ __launch_bounds__(WAVES * 64) void attn_rows_kernel(
    const RowsParams p) {
  constexpr int VEC = D >= 8 ? 8 : D;  // halves per lane per key row
  constexpr int LPR = D / VEC;         // lanes per key row
  constexpr int RPW = 64 / LPR;        // key rows per wave per step
  constexpr int R = WAVES * RPW;       // key rows per workgroup per step
  constexpr int U = D >= 64 ? 4 : (D >= 16 ? 2 : 1);  // steps per iteration
  constexpr int THREADS = WAVES * 64;

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
#ifdef MI_TIMELINE
  const TimelineRow tl = timeline_start(
      rows_timeline, blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z), tid == 0);
#else
  const TimelineRow tl;
#endif

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
  if (split >= nsplits) {
    tl.now(2);
    return;
  }
  tl.set(7, (uint64_t)split | (uint64_t)nsplits << 16);

  const uint32_t k0 = split * p.block_keys;
  const uint32_t k1 = min(available, k0 + p.block_keys);

  Vec<VEC> qv[GC];
  {
    const uint16_t *qb = p.q + (int64_t)b * p.q_seq + (int64_t)t * p.q_tok +
                         (int64_t)h0 * p.q_head + col * VEC;
#pragma unroll
    for (int g = 0; g < GC; ++g) qv[g] = load_vec<VEC>(qb + g * p.q_head);
  }
  // STEP: the new key (raw, then transformed) and value rows of head kvh,
  // loaded ahead of the cache rows so their wait leaves those in flight.
  Vec<VEC> kr, vr, wq, wk;
  if constexpr (STEP) {
    static_assert(D == 128 && VEC == 8, "decode step: head_dim 128");
    kr = load_vec<VEC>(p.step_k + (int64_t)kvh * p.step_k_head + col * VEC);
    vr = load_vec<VEC>(p.step_v + (int64_t)kvh * p.step_v_head + col * VEC);
    wq = load_vec<VEC>(p.step_qw + col * VEC);
    wk = load_vec<VEC>(p.step_kw + col * VEC);
    // Issued before the cache rows' loads, which the transforms below must
    // not wait for (loads complete in issue order).
    __builtin_amdgcn_sched_barrier(0);
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

  // Loads are unconditional: past the split's end a lane re-reads the last
  // key row (always in bounds) and its score is masked to -inf, so every
  // batch of 2*U loads issues back to back. The next batch is in flight
  // while the current one is consumed.
  auto load_batch = [&](uint32_t first, Vec<VEC> *kd, Vec<VEC> *vd) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t kk = min(first + (uint32_t)(u * R), k1 - 1);
      kd[u] = load_vec_stream<VEC>(kb + (int64_t)kk * p.k_pos);
      vd[u] = load_vec_stream<VEC>(vb + (int64_t)kk * p.v_pos);
    }
  };
  // One batch of U key rows per lane: scores, online softmax, V accumulate.
  // PARTIAL: the batch runs past the split's end, so its missing rows (which
  // re-read row k1 - 1) get score -inf and a zero V. A batch is full or
  // partial for a whole 16-lane key row, so every DPP reduction below only
  // combines lanes on the same path.
  auto consume = [&](const Vec<VEC> *kv, Vec<VEC> *vv, uint32_t key,
                     auto partial_tag) __attribute__((always_inline)) {
    constexpr bool PARTIAL = decltype(partial_tag)::value;
    bool valid[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      valid[u] = !PARTIAL || key + (uint32_t)(u * R) < k1;
      if (PARTIAL && !valid[u]) vv[u] = zero_vec<VEC>();
    }
#pragma unroll
    for (int g = 0; g < GC; ++g) {
      float s[U];
      float mx = m[g];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        s[u] = lane_group_sum<LPR>(dot<VEC>(qv[g], kv[u])) * p.scale_log2;
        if (PARTIAL) s[u] = valid[u] ? s[u] : -INFINITY;
        mx = fmaxf(mx, s[u]);
      }
      // u = 0 is always valid, so mx is finite.
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
  };
  auto consume_any = [&](const Vec<VEC> *kv, Vec<VEC> *vv, uint32_t key)
                         __attribute__((always_inline)) {
    if (key + (uint32_t)((U - 1) * R) < k1)
      consume(kv, vv, key, std::false_type{});
    else
      consume(kv, vv, key, std::true_type{});
  };
  // Two register buffers alternate (loop unrolled by two), so the batch in
  // flight never has to be copied into the one being consumed.
  Vec<VEC> ka[U], va[U], kb2[U], vb2[U];
  uint32_t key = k0 + row;
  // (STEP: unconditional, as the clamped rows stay in bounds, so that the
  // waits below count only loads issued on every path.)
  if (STEP || key < k1) load_batch(key, ka, va);
  if constexpr (STEP) {
    // While the cache rows are in flight: one RoPE angle per lane (pair =
    // lane, position query_offset, as qk_norm_rope_kernel computes it),
    // gathered by the lanes whose elements use it; then the query rows and
    // the key row are transformed. The key's last split writes the key and
    // value rows into the caches; it reads them from registers below.
    // (Sharing the angles through LDS, 16 per wave, measured no faster.)
    float ca, sa;
    {
#pragma clang fp contract(off)
      const float frequency = powf(p.step_theta, -(float)(lane * 2) / (float)D);
      const float angle = (float)p.query_offset * frequency;
      ca = cosf(angle);
      sa = sinf(angle);
    }
    float cs[8], sn[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      cs[e] = __shfl(ca, 8 * (col & 7) + e, 64);
      sn[e] = __shfl(sa, 8 * (col & 7) + e, 64);
    }
    // The GC query rows and the key row, one per 16-lane group (four per
    // pass), then gathered by every group.
    constexpr int PASSES = (GC + 1 + 3) / 4;
    Vec<VEC> t[PASSES];
#pragma unroll
    for (int ps = 0; ps < PASSES; ++ps) {
      const int i = 4 * ps + rloc;  // this group's row: query head i < GC, else the key
      Vec<VEC> raw = kr, w = wk;
#pragma unroll
      for (int g = 0; g < GC; ++g)
#pragma unroll
        for (int k = 0; k < VEC / 2; ++k) {
          raw.w[k] = i == g ? qv[g].w[k] : raw.w[k];
          w.w[k] = i == g ? wq.w[k] : w.w[k];
        }
      t[ps] = norm_rope_row(raw, w, cs, sn, p.step_eps, col < 8);
    }
#pragma unroll
    for (int k = 0; k < VEC / 2; ++k) {
#pragma unroll
      for (int g = 0; g < GC; ++g) qv[g].w[k] = __shfl(t[g / 4].w[k], (g % 4) * LPR + col, 64);
      kr.w[k] = __shfl(t[GC / 4].w[k], (GC % 4) * LPR + col, 64);
    }
    if (split == nsplits - 1 && hc == 0 && wave == 0 && rloc == 0) {
      const int64_t pos = p.query_offset;
      *reinterpret_cast<uint4 *>(p.step_kc + (int64_t)kvh * p.k_head + pos * p.k_pos + col * VEC) =
          make_uint4(kr.w[0], kr.w[1], kr.w[2], kr.w[3]);
      *reinterpret_cast<uint4 *>(p.step_vc + (int64_t)kvh * p.v_head + pos * p.v_pos + col * VEC) =
          make_uint4(vr.w[0], vr.w[1], vr.w[2], vr.w[3]);
    }
  }
  // STEP: the cache row at query_offset is read before (or while) it is
  // written, so its lanes take the new rows from registers instead.
  auto patch = [&](Vec<VEC> *kd, Vec<VEC> *vd, uint32_t first) __attribute__((always_inline)) {
    if constexpr (STEP) {
#pragma unroll
      for (int u = 0; u < U; ++u)
        if (first + (uint32_t)(u * R) == p.query_offset) {
          kd[u] = kr;
          vd[u] = vr;
        }
    }
  };
#ifdef MI_TIMELINE
  // Timeline build only: wait for the first batch (and the query rows), so
  // that word 3 marks the data's arrival apart from the arithmetic.
  __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
  tl.now(3);
#endif
  while (key < k1) {
    uint32_t next = key + R * U;
    if (next < k1) load_batch(next, kb2, vb2);
    patch(ka, va, key);
    consume_any(ka, va, key);
    key = next;
    if (key >= k1) break;
    next = key + R * U;
    if (next < k1) load_batch(next, ka, va);
    patch(kb2, vb2, key);
    consume_any(kb2, vb2, key);
    key = next;
  }

  tl.now(4);
  const bool direct = nsplits == 1;
  float *part =
      p.partial + ((size_t)unit * p.max_splits + split) * GC * (D + 2);
  // This workgroup's (M, L, A) for output element (g, d): the output itself
  // (one split) or this split's partial.
  auto emit = [&](int g, int d, float M, float L, float A) __attribute__((always_inline)) {
    if (direct) {
      out[g * p.o_head + d] = f32_to_f16(A / L);
    } else if constexpr (FUSED) {
      store_partial(part + g * (D + 2) + 2 + d, A);
      if (d == 0) {
        store_partial(part + g * (D + 2), M);
        store_partial(part + g * (D + 2) + 1, L);
      }
    } else {
      part[g * (D + 2) + 2 + d] = A;
      if (d == 0) {
        part[g * (D + 2)] = M;
        part[g * (D + 2) + 1] = L;
      }
    }
  };
  constexpr int RR = WAVES * RPW;  // key rows of the workgroup
  if constexpr (D == 128 && GC <= 2 && RR == 32 && !STEP) {
    // Every key row's (m, l, acc) goes to LDS as it is (32 KB); one wave
    // turns the rows' maxima into weights 2^(m - M) and the merged sum; each
    // output element then adds its RR rows in row order. This replaces the
    // in-wave shuffle merge and per-thread exponentials of the general path
    // below (measured on MI355X, c2: 7.16-7.25 against 7.27-7.33 us per
    // call, three interleaved rounds on one box; the one-launch decode step
    // measured 7.74 against 7.67 us with it, so it keeps the general path).
    __shared__ float s_rm[RR][GC], s_rl[RR][GC], s_f[RR][GC], s_ml[2][GC];
    __shared__ __attribute__((aligned(16))) float s_racc[RR][GC][D];
#pragma unroll
    for (int g = 0; g < GC; ++g) {
      if (col == 0) {
        s_rm[row][g] = m[g];
        s_rl[row][g] = l[g];
      }
      float4 *dst = reinterpret_cast<float4 *>(&s_racc[row][g][col * VEC]);
      dst[0] = make_float4(acc[g][0], acc[g][1], acc[g][2], acc[g][3]);
      dst[1] = make_float4(acc[g][4], acc[g][5], acc[g][6], acc[g][7]);
    }
    __syncthreads();
    if (wave == 0) {
      const int r = lane % RR, g = lane / RR;
      const float mr = g < GC ? s_rm[r][g] : -INFINITY;
      float M = mr;
#pragma unroll
      for (int mask = 1; mask < RR; mask <<= 1) M = fmaxf(M, __shfl_xor(M, mask, 64));
      const float f = mr == -INFINITY ? 0.0f : exp2_raw(mr - M);
      float lw = (g < GC ? s_rl[r][g] : 0.0f) * f;
#pragma unroll
      for (int mask = 1; mask < RR; mask <<= 1) lw += __shfl_xor(lw, mask, 64);
      if (g < GC) {
        s_f[r][g] = f;
        if (r == 0) {
          s_ml[0][g] = M;
          s_ml[1][g] = lw;
        }
      }
    }
    __syncthreads();
    for (int idx = tid; idx < GC * D; idx += THREADS) {
      const int g = idx / D, d = idx % D;
      float A = 0.0f;
#pragma unroll
      for (int r = 0; r < RR; ++r) A = fmaf(s_racc[r][g][d], s_f[r][g], A);
      emit(g, d, s_ml[0][g], s_ml[1][g], A);
    }
  } else {
    __shared__ float s_m[WAVES][GC];
    __shared__ float s_l[WAVES][GC];
    __shared__ float s_acc[WAVES][GC][D];
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
      emit(g, d, M, L, A);
    }
  }
  if constexpr (FUSED) {
    if (direct) {
      tl.now(2);
      return;
    }
    // Every store of this workgroup has completed before the arrival counts.
    __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
    __shared__ uint32_t s_last;
    __syncthreads();
    tl.now(5);
    if (tid == 0) {
      uint32_t *counter = p.counters + (size_t)unit * p.counter_stride;
      const uint32_t arrived = arrive(counter);
      const bool last = arrived == nsplits - 1;
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
    merge_splits<D, GC, THREADS, true>(p, unit, nsplits, out);
  }
  tl.now(2);
}


// ---------------------------------------------------------------------------
// Batched decode on MFMA with a stream-K split (one query token per sequence,
// D = 128). Measured on MI355X at 32 sequences, L ~ U[1024, 8192], GQA 4:
// 110 us against 126 us for the rows kernel with 768-key splits.
//  - Work split: the launch's workgroups divide the flattened (unit, key)
//    space of all sequences (unit = sequence, KV head, head chunk) into equal
//    segments, so each workgroup streams the same number of bytes whatever
//    the lengths. A segment is the tail of one unit, whole units and the head
//    of another; each such piece ends in one partial, at slot
//    (workgroup + unit) (unique, and a unit's pieces are consecutive slots).
//    attn_stream_merge_kernel, launched next on the same stream, merges the
//    pieces of every split unit (stream order makes the partials visible).
//    In-launch merges measured slower on MI355X at 32 sequences: 27% with a
//    release per piece (an L2 writeback while the other workgroups stream),
//    3% with every workgroup's arrivals counted at its segment's end (the
//    last arrivers are the slow second workgroups of their CUs).
//  - Per 32-key tile and wave: S^T[key][head] = K Q^T on
//    v_mfma_f32_16x16x32_f16, K rows loaded straight into the A operand
//    (lane (g, c) holds key c, d 8 g + 32 j) and Q^T as the B operand (head
//    c of the chunk, zero past it). Each lane then holds 8 keys of one head,
//    so the f32 online softmax is lane-local plus a max over the four
//    16-lane groups. O^T[d][head] += V^T P^T on the same MFMA: V rows land in
//    the wave's LDS stage by direct loads, in a key order that matches the S
//    accumulator, and are read transposed (ds_read_b64_tr_b16), so P is used
//    in place.
//  - The 4 waves take interleaved tiles, each with two register / LDS stages
//    (the next tile is in flight while one is computed).
constexpr int kStreamWaves = 4;
constexpr int kStreamTile = 32;

#ifdef MI_TIMELINE
__device__ uint64_t stream_timeline[kTimelineSlots * kTimelineFields];
#endif

typedef float sf4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint4 load16_stream(const uint16_t *ptr) {
  typedef unsigned u4_t __attribute__((ext_vector_type(4)));
  const u4_t x = __builtin_nontemporal_load(reinterpret_cast<const u4_t *>(ptr));
  return make_uint4(x.x, x.y, x.z, x.w);
}
// Key of LDS row r of a V tile: k-slot 8 g + i of the PV operand holds key
// 16 (i / 4) + 4 g + i % 4, the keys lane group g holds in the S accumulator.
__device__ __forceinline__ int stream_slot_key(int r) {
  return (((r >> 2) & 1) << 4) | (((r >> 3) & 3) << 2) | (r & 3);
}
// XOR applied to the 32-byte column pair of V row r: the 16 rows of one
// transposed read then fall on 8 distinct bank groups.
__device__ __forceinline__ int stream_swizzle(int r) { return (r & 3) | (((r >> 3) & 1) << 2); }

template <int GC>
__global__ __launch_bounds__(kStreamWaves * 64, 2) void attn_decode_stream_kernel(
    const RowsParams p) {
  constexpr int D = 128, WAVES = kStreamWaves, KT = kStreamTile, DC = D / 32, DB = D / 16;
  constexpr int THREADS = WAVES * 64;
  constexpr int STAGE = KT * D;  // halves of V per wave and stage
  static_assert(WAVES * GC * D * 4 <= WAVES * STAGE * 2, "wave merge must fit a stage");
  // Two V stages, one array each, so the compiler can tell the direct loads
  // into one from the reads of the other. After a piece's tile loop stage a
  // holds the wave merge.
  __shared__ __attribute__((aligned(16))) uint16_t v_lds_a[WAVES * STAGE];
  __shared__ __attribute__((aligned(16))) uint16_t v_lds_b[WAVES * STAGE];
  __shared__ float s_m[WAVES][GC];
  __shared__ float s_l[WAVES][GC];
  __shared__ uint64_t s_pre[kStreamMaxBatch + 1];  // keys of all units before sequence b
  __shared__ uint32_t s_len[kStreamMaxBatch];      // visible keys of sequence b

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int col = lane & 15, grp = lane >> 4;
#ifdef MI_TIMELINE
  const TimelineRow tl = timeline_start(stream_timeline, blockIdx.x, tid == 0);
#else
  const TimelineRow tl;
#endif
  const uint32_t upb = p.kv_heads * p.head_chunks;  // units per sequence
  const float c2 = p.scale_log2;
  // Visible keys of sequence b: its cached length (one query at the end).
  auto visible = [&](uint32_t b) -> uint32_t {
    return p.lengths != nullptr ? min(p.lengths[b], p.kv_length) : p.kv_length;
  };
  // Prefix sums of the per-sequence key counts: all lengths load at once,
  // then wave 0 scans them 64 at a time.
  for (uint32_t b = tid; b < p.batch; b += THREADS) {
    const uint32_t n = visible(b);
    s_len[b] = n;
    s_pre[b + 1] = (uint64_t)n * upb;
  }
  __syncthreads();
  if (wave == 0) {
    uint64_t carry = 0;
    for (uint32_t c0 = 0; c0 < p.batch; c0 += 64) {
      const uint32_t b = c0 + lane;
      uint64_t x = b < p.batch ? s_pre[b + 1] : 0;
#pragma unroll
      for (int d = 1; d < 64; d <<= 1) {
        const uint64_t y = __shfl_up(x, d, 64);
        if (lane >= d) x += y;
      }
      if (b < p.batch) s_pre[b + 1] = carry + x;
      carry += __shfl(x, 63, 64);
    }
    if (lane == 0) s_pre[0] = 0;
  }
  __syncthreads();
  // Sequences with no key: the reference divides 0 by 0.
  for (uint32_t b = blockIdx.x; b < p.batch; b += gridDim.x)
    if (s_pre[b + 1] == s_pre[b])
      for (uint32_t idx = tid; idx < p.q_heads * D; idx += THREADS)
        p.out[(int64_t)b * p.o_seq + (int64_t)(idx / D) * p.o_head + idx % D] = 0x7e00;
  const uint64_t total = s_pre[p.batch];
  // At least kStreamMinKeys per workgroup; the rest of the grid idles.
  const uint64_t W = min((uint64_t)gridDim.x, max((uint64_t)1, total / kStreamMinKeys));
  // 32-bit division when the total fits (a 64-bit one is a long sequence).
  const uint64_t seg = total + W - 1 <= 0xffffffffull
                           ? (uint64_t)((uint32_t)(total + W - 1) / (uint32_t)W)
                           : (total + W - 1) / W;
  const uint32_t w = blockIdx.x;
  uint64_t pos = (uint64_t)w * seg;
  const uint64_t end = min(pos + seg, total);
  if (pos >= end) {
    tl.now(2);
    return;
  }
  // The sequence holding key `at`: the last b with s_pre[b] <= at (which
  // skips sequences without keys).
  // s_pre is nondecreasing, so that b is the count of b' in [1, batch) with
  // s_pre[b'] <= at: each lane tests one b' per 64, a ballot counts them
  // (with the 32-bit segment division above, measured on MI355X, c4:
  // 103.87-103.95 against 103.98-104.08 us per call with a binary search
  // and a 64-bit division, bit-identical).
  auto find_seq = [&](uint64_t at) -> uint32_t {
    uint32_t count = 0;
    for (uint32_t c0 = 1; c0 < p.batch; c0 += 64) {
      const uint32_t bb = c0 + lane;
      const bool le = bb < p.batch && s_pre[bb] <= at;
      count += (uint32_t)__popcll(__ballot(le));
    }
    return count;
  };
  uint32_t b = find_seq(pos);

  // Loop-invariant byte offsets inside a full tile (its base is uniform).
  // K: lane (grp, col) loads key col (+16 for the second half), d 8 grp +
  // 32 j. V: direct-load instruction i writes LDS rows 4i .. 4i + 3, lane L
  // row 4i + L / 16 and physical 16-byte chunk L % 16.
  uint32_t v_off[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int r = 4 * i + (lane >> 4), pc = lane & 15;
    const int chunk = 2 * ((pc >> 1) ^ stream_swizzle(r)) + (pc & 1);
    v_off[i] = (uint32_t)(stream_slot_key(r) * p.v_pos + chunk * 8) * 2u;
  }
  uint32_t k_off[2];
#pragma unroll
  for (int hf = 0; hf < 2; ++hf) k_off[hf] = (uint32_t)((16 * hf + col) * p.k_pos + 8 * grp) * 2u;
  // Transposed V reads: lane (grp, mu) addresses row 8 grp + mu / 4 (and
  // + 4), d 16 dt + 4 (mu % 4).
  const int mu = lane & 15;
  const int tr_row = 8 * grp + (mu >> 2);
  const int tr_base = tr_row * D + 4 * (mu & 1);
  const int tr_hi = (mu & 3) >> 1;
  const int tr_f = stream_swizzle(tr_row);

  // When every key position fits 32 bits (any call below 4 G keys), the
  // divisions of the piece bookkeeping are 32-bit. The lengths come from LDS
  // (measured on MI355X, c4: 104.6-104.7 against 104.8-104.9 us per call
  // re-reading them from global memory with 64-bit divisions, bit-identical).
  const bool narrow = total <= 0xffffffffull;
  tl.now(3);
  while (pos < end) {
    const uint32_t len_b = s_len[b];
    const uint64_t rel = pos - s_pre[b];
    const uint32_t j = narrow ? (uint32_t)rel / len_b : (uint32_t)(rel / len_b);  // unit
    const uint32_t k0 = (uint32_t)(rel - (uint64_t)j * len_b);
    const uint32_t k1 = (uint32_t)min((uint64_t)len_b, k0 + (end - pos));
    const uint32_t kvh = j / p.head_chunks, hc = j % p.head_chunks;
    const uint32_t unit = b * upb + j;
    const uint64_t unit_start = s_pre[b] + (uint64_t)j * len_b;
    const uint64_t unit_last = unit_start + len_b - 1;
    const uint32_t first_wg = narrow ? (uint32_t)unit_start / (uint32_t)seg : (uint32_t)(unit_start / seg);
    const uint32_t last_wg = narrow ? (uint32_t)unit_last / (uint32_t)seg : (uint32_t)(unit_last / seg);
    const uint32_t h0 = kvh * p.group + hc * GC;
    uint16_t *out = p.out + (int64_t)b * p.o_seq + (int64_t)h0 * p.o_head;
    const uint32_t ntiles = (k1 - k0 + KT - 1) / KT;

    h8_t qop[DC];
    {
      const uint16_t *qb = p.q + (int64_t)b * p.q_seq + (int64_t)(h0 + min(col, GC - 1)) * p.q_head + 8 * grp;
#pragma unroll
      for (int c = 0; c < DC; ++c)
        qop[c] = col < GC ? as_h8(*reinterpret_cast<const uint4 *>(qb + 32 * c))
                          : as_h8(make_uint4(0, 0, 0, 0));
    }
    const uint16_t *kb = p.k + (int64_t)b * p.k_seq + (int64_t)kvh * p.k_head;
    const uint16_t *vb = p.v + (int64_t)b * p.v_seq + (int64_t)kvh * p.v_head;
    sf4_t o[DB];
#pragma unroll
    for (int dt = 0; dt < DB; ++dt) o[dt] = sf4_t{0.0f, 0.0f, 0.0f, 0.0f};
    float m_run = -INFINITY, l_run = 0.0f;  // raw-score reference max, row sum

    auto issue = [&](uint32_t ti, uint4 *kr, uint16_t *vst) __attribute__((always_inline)) {
      const uint32_t base = k0 + ti * KT;
      uint16_t *vdst = vst + wave * STAGE;
      if (base + KT <= k1) {
        const char *kt = reinterpret_cast<const char *>(kb + (int64_t)base * p.k_pos);
        const char *vt = reinterpret_cast<const char *>(vb + (int64_t)base * p.v_pos);
#pragma unroll
        for (int hf = 0; hf < 2; ++hf)
#pragma unroll
          for (int c = 0; c < DC; ++c)
            kr[hf * DC + c] = load16_stream(reinterpret_cast<const uint16_t *>(kt + k_off[hf] + 64 * c));
        // V is read once too: non-temporal (c4: 111.3 -> 110.1 us, same run).
#pragma unroll
        for (int i = 0; i < 8; ++i)
          load_lds16_nt(reinterpret_cast<const uint16_t *>(vt + v_off[i]), vdst + i * 512);
      } else {
        // The piece's last, partial tile: rows past it re-read its last key
        // (always in bounds) and are masked.
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) {
          const uint32_t key = min(base + 16 * hf + col, k1 - 1);
#pragma unroll
          for (int c = 0; c < DC; ++c)
            kr[hf * DC + c] = load16_stream(kb + (int64_t)key * p.k_pos + 8 * grp + 32 * c);
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int r = 4 * i + (lane >> 4), pc = lane & 15;
          const int chunk = 2 * ((pc >> 1) ^ stream_swizzle(r)) + (pc & 1);
          const uint32_t key = min(base + (uint32_t)stream_slot_key(r), k1 - 1);
          load_lds16_nt(vb + (int64_t)key * p.v_pos + chunk * 8, vdst + i * 512);
        }
      }
    };
    auto compute = [&](uint32_t ti, const uint4 *kr, const uint16_t *vst) __attribute__((always_inline)) {
      const uint32_t base = k0 + ti * KT;
      sf4_t s[2];  // s[hf][e]: head col, key 16 hf + 4 grp + e
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        s[hf] = sf4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int c = 0; c < DC; ++c)
          s[hf] = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_h8(kr[hf * DC + c]), qop[c], s[hf], 0, 0, 0);
      }
      if (base + KT > k1) {
#pragma unroll
        for (int hf = 0; hf < 2; ++hf)
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (base + 16 * hf + 4 * grp + e >= k1) s[hf][e] = -INFINITY;
      }
      float mx = fmaxf(fmaxf(fmaxf(s[0][0], s[0][1]), fmaxf(s[0][2], s[0][3])),
                       fmaxf(fmaxf(s[1][0], s[1][1]), fmaxf(s[1][2], s[1][3])));
      mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      // Lazy rescale: the reference max moves only when some head outgrows
      // it by 2^8 (always on a piece's first tile), which keeps P <= 256.
      if (__any((mx - m_run) * c2 > 8.0f)) {
        const float m_new = fmaxf(m_run, mx);
        const float alpha = m_new == -INFINITY ? 1.0f : exp2_raw((m_run - m_new) * c2);
        l_run *= alpha;
#pragma unroll
        for (int dt = 0; dt < DB; ++dt) o[dt] *= alpha;
        m_run = m_new;
      }
      const float mc = m_run == -INFINITY ? 0.0f : m_run * c2;
      uint32_t pw[4];  // P as f16 pairs in the PV operand's key order
      float ps = 0.0f;
#pragma unroll
      for (int hf = 0; hf < 2; ++hf)
#pragma unroll
        for (int e = 0; e < 4; e += 2) {
          const uint32_t wv = pack_f16x2(exp2_raw(fmaf(s[hf][e], c2, -mc)),
                                           exp2_raw(fmaf(s[hf][e + 1], c2, -mc)));
          pw[2 * hf + e / 2] = wv;
          // The row sum uses the same f16-rounded weights as P V.
          ps = dot2(wv, 0x3c003c00u, ps);
        }
      l_run += ps;
      const h8_t pb = as_h8(make_uint4(pw[0], pw[1], pw[2], pw[3]));
      const uint16_t *vw = vst + wave * STAGE;
#pragma unroll
      for (int dt = 0; dt < DB; ++dt) {
        const uint16_t *a0 = vw + tr_base + (2 * (dt ^ tr_f) + tr_hi) * 8;
        const uint2 lo = read_tr16(a0), hi = read_tr16(a0 + 4 * D);
        o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_h8(make_uint4(lo.x, lo.y, hi.x, hi.y)), pb,
                                                       o[dt], 0, 0, 0);
      }
    };

    // Wave w takes tiles w, w + 4, ...; the register and LDS stages
    // alternate (loop unrolled by two so each is a compile-time choice).
    uint4 kra[2 * DC], krb[2 * DC];
    uint32_t ti = wave;
    if (ti < ntiles) issue(ti, kra, v_lds_a);
    while (ti < ntiles) {
      uint32_t nx = ti + WAVES;
      if (nx < ntiles) issue(nx, krb, v_lds_b);
      compute(ti, kra, v_lds_a);
      ti = nx;
      if (ti >= ntiles) break;
      nx = ti + WAVES;
      if (nx < ntiles) issue(nx, kra, v_lds_a);
      compute(ti, krb, v_lds_b);
      ti = nx;
    }
    l_run += __shfl_xor(l_run, 16, 64);
    l_run += __shfl_xor(l_run, 32, 64);

    // Merge the waves through LDS, then write the unit's output (a piece
    // that is the whole unit) or this piece's partial.
    __syncthreads();
    const uint64_t tl_loop_end = tl.clock();
    float *s_o = reinterpret_cast<float *>(v_lds_a);  // [WAVES][GC][D]
    if (col < GC) {
      if (grp == 0) {
        s_m[wave][col] = m_run;
        s_l[wave][col] = l_run;
      }
#pragma unroll
      for (int dt = 0; dt < DB; ++dt)
#pragma unroll
        for (int e = 0; e < 4; ++e) s_o[(wave * GC + col) * D + 16 * dt + 4 * grp + e] = o[dt][e];
    }
    __syncthreads();
    const bool direct = first_wg == last_wg;
    // Slot of this piece (kernels.hpp, launch_decode_stream): the unit's own
    // slots when it has few pieces, so that the merge launch can load them
    // with its descriptor in one round trip, else the overflow slots.
    const uint32_t units = p.batch * upb, pieces = last_wg - first_wg + 1;
    const uint32_t S = p.stream_unit_slots;
    const size_t slot = pieces <= S ? (size_t)unit * S + (w - first_wg) : (size_t)units * S + w + unit;
    float *part = p.partial + slot * GC * (D + 2);
    if (w == first_wg && tid == 0)
      reinterpret_cast<uint32_t *>(p.partial + (size_t)units * (S + 1) * GC * (D + 2) +
                                   (size_t)p.stream_workgroups * GC * (D + 2))[unit] =
          first_wg | pieces << 16;
    for (int idx = tid; idx < GC * D; idx += THREADS) {
      const int g = idx / D, d = idx % D;
      float M = -INFINITY;
#pragma unroll
      for (int wv = 0; wv < WAVES; ++wv) M = fmaxf(M, s_m[wv][g]);
      float L = 0.0f, A = 0.0f;
#pragma unroll
      for (int wv = 0; wv < WAVES; ++wv) {
        const float f = s_m[wv][g] == -INFINITY ? 0.0f : exp2_raw((s_m[wv][g] - M) * c2);
        L += s_l[wv][g] * f;
        A += s_o[(wv * GC + g) * D + d] * f;
      }
      if (direct) {
        out[g * p.o_head + d] = f32_to_f16(A / L);
      } else {
        // A piece of a split unit: its partial, for the merge launch that
        // follows on the same stream. The max stays in log2-scaled units,
        // as the rows kernel's.
        part[g * (D + 2) + 2 + d] = A;
        if (d == 0) {
          part[g * (D + 2)] = M == -INFINITY ? -INFINITY : M * c2;
          part[g * (D + 2) + 1] = L;
        }
      }
    }
    // The next piece's loads overwrite both stages.
    __syncthreads();
    tl.add(4, 1 | (uint64_t)ntiles << 16);
    tl.add(5, tl.clock() - tl_loop_end);
    pos += k1 - k0;
    if (pos < end && pos >= s_pre[b + 1]) b = find_seq(pos);
  }
  tl.now(2);
}

// Merges the pieces of the split units of attn_decode_stream_kernel, one
// workgroup per unit, in piece order: the log-sum-exp combine of the
// reference's reduce kernels (transformer.metal:2251-2316). The unit's
// descriptor (first workgroup, pieces), its length and its own
// kStreamUnitSlots slots load together, so a unit of at most that many pieces
// merges after one memory round trip (measured on MI355X, c4: 104.3 against
// 105.1 us per call recomputing the stream kernel's segments from all the
// lengths first, bit-identical); longer units read the overflow slots after.
// Eight slots per unit: a unit of the stream split spans a few workgroups'
// segments (c4: 2-5), and 16-wide passes loaded mostly padding (106.7-107.5
// against 107.7-107.9 us per call). One thread per output element (GC x 128,
// at least 256, at most 1024), so the slots load in one pass (c4, GQA 4:
// 105.7 against 106.0 us with 256 threads and two passes, bit-identical).
template <int GC>
constexpr int stream_merge_threads() {
  return GC * 128 > 1024 ? 1024 : (GC * 128 > 256 ? GC * 128 : 256);
}

template <int GC>
__global__ __launch_bounds__(stream_merge_threads<GC>()) void attn_stream_merge_kernel(
    const RowsParams p) {
  constexpr int D = 128, THREADS = stream_merge_threads<GC>(), ROW = D + 2;
  constexpr int C = kStreamUnitSlots;  // pieces per pass
  const uint32_t S = p.stream_unit_slots;
  const uint32_t upb = p.kv_heads * p.head_chunks;
  const uint32_t unit = blockIdx.x, b = unit / upb, j = unit % upb;
  const uint32_t units = p.batch * upb;
  const float *own = p.partial + (size_t)unit * S * GC * ROW;
  const float *overflow = p.partial + (size_t)units * S * GC * ROW;
  const uint32_t desc = reinterpret_cast<const uint32_t *>(
      overflow + (size_t)(p.stream_workgroups + units) * GC * ROW)[unit];
  const uint32_t len_b = min(p.lengths[b], p.kv_length);
  const uint32_t kvh = j / p.head_chunks, hc = j % p.head_chunks;
  uint16_t *out = p.out + (int64_t)b * p.o_seq + (int64_t)(kvh * p.group + hc * GC) * p.o_head;
  for (int idx = threadIdx.x; idx < GC * D; idx += THREADS) {
    const int g = idx / D, d = idx % D;
    // The unit's own slots, issued before the descriptor is known (in
    // bounds whatever they hold). The compact layout (S = 0) has none: every
    // piece is loaded after the descriptor below.
    float m[C], l[C], a[C];
    if (S != 0) {
#pragma unroll
      for (int i = 0; i < C; ++i) {
        const float *ps = own + (size_t)(i * GC + g) * ROW;
        m[i] = ps[0];
        l[i] = ps[1];
        a[i] = ps[2 + d];
      }
    }
    // Zero keys: NaN, written by the stream kernel (the descriptor is stale).
    const uint32_t pieces = desc >> 16;
    if (len_b == 0 || pieces <= 1) return;
    const float *base = pieces <= S ? own : overflow + (size_t)((desc & 0xffff) + unit) * GC * ROW;
    float M = -INFINITY, Ls = 0.0f, As = 0.0f;
    for (uint32_t s0 = 0; s0 < pieces; s0 += C) {
      if (pieces > S) {
#pragma unroll
        for (int i = 0; i < C; ++i) {
          const float *ps = base + (size_t)(min(s0 + i, pieces - 1) * GC + g) * ROW;
          m[i] = ps[0];
          l[i] = ps[1];
          a[i] = ps[2 + d];
        }
      }
      // Slots past the last piece hold other data: they take no part.
      bool use[C];
#pragma unroll
      for (int i = 0; i < C; ++i) use[i] = s0 + i < pieces && m[i] != -INFINITY;
      float cm = M;
#pragma unroll
      for (int i = 0; i < C; ++i) cm = use[i] ? fmaxf(cm, m[i]) : cm;
      const float r = M == -INFINITY ? 0.0f : exp2_raw(M - cm);
      Ls *= r;
      As *= r;
#pragma unroll
      for (int i = 0; i < C; ++i) {
        const float f = use[i] ? exp2_raw(m[i] - cm) : 0.0f;
        Ls = use[i] ? fmaf(l[i], f, Ls) : Ls;
        As = use[i] ? fmaf(a[i], f, As) : As;
      }
      M = cm;
    }
    out[g * p.o_head + d] = f32_to_f16(As / Ls);
  }
}

// Merges the split partials of one (row, KV head, head chunk) unit: the
// log-sum-exp combine of the reference's reduce kernels
// (transformer.metal:2251-2316). Launched after attn_rows_kernel on the same
// stream, so every partial is visible without any in-kernel fence. One
// thread per output element (GC x D, at least 256, at most 1024), so the
// partials load in one pass where the unit has at most 1024 outputs.
template <int D, int GC>
constexpr int merge_threads() {
  return GC * D > 1024 ? 1024 : (GC * D > 256 ? GC * D : 256);
}

template <int D, int GC>
__global__ __launch_bounds__((merge_threads<D, GC>())) void attn_merge_kernel(const RowsParams p) {
  const uint32_t unit = blockIdx.x;
  const uint32_t units_per_token = p.kv_heads * p.head_chunks;
  const uint32_t bt = unit / units_per_token;
  const uint32_t rest = unit % units_per_token;
  const uint32_t kvh = rest / p.head_chunks, hc = rest % p.head_chunks;
  const uint32_t b = bt / p.tokens, t = bt % p.tokens;
  uint32_t len = p.kv_length, off = p.query_offset;
  if (p.lengths != nullptr) {
    len = min(p.lengths[b], p.kv_length);
    off = len >= p.tokens ? len - p.tokens : 0u;
  }
  const uint64_t window = (uint64_t)off + t + 1;
  const uint32_t available =
      p.causal != 0 ? (uint32_t)min((uint64_t)len, window) : len;
  const uint32_t nsplits = (available + p.block_keys - 1) / p.block_keys;
  if (nsplits <= 1) return;  // written directly by the split kernel
  const uint32_t h0 = kvh * p.group + hc * GC;
  uint16_t *out = p.out + (int64_t)b * p.o_seq + (int64_t)t * p.o_tok +
                  (int64_t)h0 * p.o_head;
  merge_splits<D, GC, merge_threads<D, GC>(), false>(p, unit, nsplits, out);
}

template <int D, int WAVES, int GC>
hipError_t launch_rows_dwg(const RowsParams &p, RowsPhase phase, const Launch &l) {
  if (phase == RowsPhase::Split) {
    const dim3 grid(p.max_splits, p.kv_heads * p.head_chunks,
                    p.batch * p.tokens);
    if constexpr (D == 128 && WAVES == 8) {
      if (p.step_k != nullptr) {
        if (p.counters != nullptr)
          return dispatch(attn_rows_kernel<D, WAVES, GC, true, true>, grid, dim3(WAVES * 64), 0, l, p);
        return dispatch(attn_rows_kernel<D, WAVES, GC, false, true>, grid, dim3(WAVES * 64), 0, l, p);
      }
    }
    if (p.step_k != nullptr) return hipErrorInvalidValue;
    if (p.counters != nullptr)
      return dispatch(attn_rows_kernel<D, WAVES, GC, true>, grid, dim3(WAVES * 64), 0, l, p);
    return dispatch(attn_rows_kernel<D, WAVES, GC, false>, grid, dim3(WAVES * 64), 0, l, p);
  }
  if (p.max_splits <= 1 || p.counters != nullptr) return no_dispatch(l);
  const uint32_t units = p.batch * p.tokens * p.kv_heads * p.head_chunks;
  return dispatch(attn_merge_kernel<D, GC>, dim3(units), dim3(merge_threads<D, GC>()), 0, l, p);
}

template <int D, int WAVES>
hipError_t launch_rows_dw(const RowsParams &p, uint32_t chunk, RowsPhase phase,
                          const Launch &l) {
  switch (chunk) {
    case 8: return launch_rows_dwg<D, WAVES, 8>(p, phase, l);
    case 4: return launch_rows_dwg<D, WAVES, 4>(p, phase, l);
    case 2: return launch_rows_dwg<D, WAVES, 2>(p, phase, l);
    case 1: return launch_rows_dwg<D, WAVES, 1>(p, phase, l);
    default: return hipErrorInvalidValue;
  }
}

template <int D>
hipError_t launch_rows_d(const RowsParams &p, uint32_t waves, uint32_t chunk,
                         RowsPhase phase, const Launch &l) {
  if (waves == 8) return launch_rows_dw<D, 8>(p, chunk, phase, l);
  if (waves == 4) return launch_rows_dw<D, 4>(p, chunk, phase, l);
  if (waves == 2) return launch_rows_dw<D, 2>(p, chunk, phase, l);
  return hipErrorInvalidValue;
}

template <int GC>
hipError_t launch_stream_gc(const RowsParams &p, RowsPhase phase, const Launch &l) {
  if (phase == RowsPhase::Split)
    return dispatch(attn_decode_stream_kernel<GC>, dim3(p.stream_workgroups),
                    dim3(kStreamWaves * 64), 0, l, p);
  const uint32_t units = p.batch * p.kv_heads * p.head_chunks;
  return dispatch(attn_stream_merge_kernel<GC>, dim3(units), dim3(stream_merge_threads<GC>()), 0, l,
                  p);
}

}  // namespace

uint32_t stream_chunk(uint32_t group) {
  for (uint32_t c : {16u, 8u, 4u, 2u}) if (group % c == 0) return c;
  return 1;
}

hipError_t launch_decode_stream(const RowsParams &p, uint32_t chunk, RowsPhase phase,
                                const Launch &l) {
  switch (chunk) {
    case 16: return launch_stream_gc<16>(p, phase, l);
    case 8: return launch_stream_gc<8>(p, phase, l);
    case 4: return launch_stream_gc<4>(p, phase, l);
    case 2: return launch_stream_gc<2>(p, phase, l);
    case 1: return launch_stream_gc<1>(p, phase, l);
    default: return hipErrorInvalidValue;
  }
}

uint32_t rows_chunk(uint32_t group) {
  for (uint32_t c : {8u, 4u, 2u}) if (group % c == 0) return c;
  return 1;
}

hipError_t launch_rows(const RowsParams &p, uint32_t head_dim, uint32_t waves,
                       uint32_t chunk, RowsPhase phase, const Launch &l) {
  switch (head_dim) {
    case 1: return launch_rows_d<1>(p, waves, chunk, phase, l);
    case 2: return launch_rows_d<2>(p, waves, chunk, phase, l);
    case 4: return launch_rows_d<4>(p, waves, chunk, phase, l);
    case 8: return launch_rows_d<8>(p, waves, chunk, phase, l);
    case 16: return launch_rows_d<16>(p, waves, chunk, phase, l);
    case 32: return launch_rows_d<32>(p, waves, chunk, phase, l);
    case 64: return launch_rows_d<64>(p, waves, chunk, phase, l);
    case 128: return launch_rows_d<128>(p, waves, chunk, phase, l);
    case 256: return launch_rows_d<256>(p, waves, chunk, phase, l);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace kernels
}  // namespace mi

#ifdef MI_TIMELINE
extern "C" int32_t mi_timeline_read_rows(void *dst, uint64_t bytes) {
  const uint64_t cap = sizeof(uint64_t) * mi::dev::kTimelineSlots * mi::dev::kTimelineFields;
  if (dst == nullptr || bytes > cap) return hipErrorInvalidValue;
  return hipMemcpyFromSymbol(dst, HIP_SYMBOL(mi::kernels::rows_timeline), bytes, 0,
                             hipMemcpyDeviceToHost);
}
extern "C" int32_t mi_timeline_read_stream(void *dst, uint64_t bytes) {
  const uint64_t cap = sizeof(uint64_t) * mi::dev::kTimelineSlots * mi::dev::kTimelineFields;
  if (dst == nullptr || bytes > cap) return hipErrorInvalidValue;
  return hipMemcpyFromSymbol(dst, HIP_SYMBOL(mi::kernels::stream_timeline), bytes, 0,
                             hipMemcpyDeviceToHost);
}
#endif
