// Kernel parameter blocks and launchers shared by the host runtime and the
// HIP kernels. All strides are in elements; every tensor the fast kernels
// read has a unit innermost stride.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mi {
namespace kernels {

// Where a kernel runs: its stream, and optionally start / stop events that
// hipExtLaunchKernelGGL binds to the dispatch packet itself, so they time
// the kernel's execution without the enqueue latency that separate
// hipEventRecord markers would add.
struct Launch {
  hipStream_t stream = nullptr;
  hipEvent_t start = nullptr;
  hipEvent_t stop = nullptr;
};

template <typename... Params, typename... Args>
hipError_t dispatch(void (*kernel)(Params...), dim3 grid, dim3 block, uint32_t lds,
                    const Launch &l, Args... args) {
  if (l.start == nullptr && l.stop == nullptr)
    kernel<<<grid, block, lds, l.stream>>>(args...);
  else
    hipExtLaunchKernelGGL(kernel, grid, block, lds, l.stream, l.start, l.stop, 0, args...);
  return hipGetLastError();
}

// A launcher with nothing to run still stamps its events, so a profiled
// launch record always has both.
inline hipError_t no_dispatch(const Launch &l) {
  hipError_t err = hipSuccess;
  if (l.start != nullptr) err = hipEventRecord(l.start, l.stream);
  if (err == hipSuccess && l.stop != nullptr) err = hipEventRecord(l.stop, l.stream);
  return err != hipSuccess ? err : hipGetLastError();
}

// Split-K "rows" attention: one workgroup per (sequence*token, KV head,
// head chunk, key split). Serves Tiled, DecodeSplitKv, FlashDecode and the
// batched decode. Q/O are [B, T, Hq, D]; K/V are [B, L, Hkv, D] views.
struct RowsParams {
  const uint16_t *q;
  int64_t q_seq, q_tok, q_head;
  const uint16_t *k;
  int64_t k_seq, k_pos, k_head;
  const uint16_t *v;
  int64_t v_seq, v_pos, v_head;
  uint16_t *out;
  int64_t o_seq, o_tok, o_head;
  float *partial;           // [units][max_splits][chunk][D + 2] f32
  // Arrival counters, one per unit (zero between kernels), or null. Set:
  // the last split of a unit merges (one launch). Null: the merge pass does.
  // Unit u's counter is counters[u * counter_stride].
  uint32_t *counters;
  uint32_t counter_stride;
  const uint32_t *lengths;  // per-sequence KV length, or null
  uint32_t batch;           // B
  uint32_t tokens;          // T
  uint32_t q_heads, kv_heads, group;
  uint32_t head_chunks;     // group / chunk
  uint32_t kv_length;       // L (upper bound when lengths != null)
  uint32_t causal;
  uint32_t query_offset;    // ignored when lengths != null
  uint32_t block_keys;      // keys per split
  uint32_t max_splits;
  uint32_t stream_workgroups;  // stream-K decode: workgroups of the launch
  uint32_t stream_unit_slots;  // stream-K decode: fixed partial slots per unit (0 or kStreamUnitSlots)
  float scale_log2;         // rsqrt(D) * log2(e)
  // Decode step (step_k != null; one token, D = 128, 8 waves): q holds the
  // raw query rows and step_k / step_v the new token's key and value rows
  // [Hkv, D]. The kernel applies qk_norm_rope_cache's per-head RMSNorm +
  // RoPE (position query_offset) to the query and key rows, writes the key
  // and value rows into step_kc / step_vc (the caches k / v point into) at
  // query_offset, and attends over keys 0 .. query_offset.
  const uint16_t *step_k, *step_v, *step_qw, *step_kw;
  int64_t step_k_head, step_v_head;
  uint16_t *step_kc, *step_vc;
  float step_theta, step_eps;
};

// Exact two-pass attention (AttentionKind::Reference).
struct NaiveParams {
  const uint16_t *q;
  int64_t q_tok, q_head;
  const uint16_t *k;
  int64_t k_pos, k_head;
  const uint16_t *v;
  int64_t v_pos, v_head;
  uint16_t *out;
  int64_t o_tok, o_head;
  float *scores;            // [row_count][L] f32 when scores spill from LDS
  uint32_t tokens, q_heads, kv_heads, head_dim, kv_length, causal,
      query_offset;
  float scale;              // rsqrt(D)
};

// KV append: source [T, H, D] -> cache [C, H, D] at `offset`.
struct CopyKvParams {
  const uint16_t *src;
  int64_t s_tok, s_head;
  uint16_t *dst;
  int64_t d_pos, d_head;
  uint32_t tokens, heads, head_dim, offset;
};

// Fused per-head RMSNorm + RoPE, K written into the cache.
struct QkNormRopeParams {
  const uint16_t *q;
  int64_t q_tok, q_head;
  const uint16_t *k;
  int64_t k_tok, k_head;
  const uint16_t *q_weight;
  const uint16_t *k_weight;
  uint16_t *q_out;
  int64_t qo_tok, qo_head;
  uint16_t *cache;
  int64_t c_pos, c_head;
  // Optional value append (v != null): rows v[T, Hkv, D] are copied to
  // v_cache at position offset + token by workgroups after the Q/K rows.
  const uint16_t *v;
  int64_t v_tok, v_head;
  uint16_t *v_cache;
  int64_t vc_pos, vc_head;
  uint32_t tokens, q_heads, kv_heads, head_dim, offset;
  float theta, epsilon;
};

// MFMA flash prefill (FlashPrefill at head_dim 64 / 128 / 256).
// Split prefill plans with at most this many pieces per KV head launch them
// in an order chosen on the host (PrefillParams::order).
constexpr uint32_t kPrefillOrderMax = 64;

struct PrefillParams {
  const uint16_t *q;
  int64_t q_tok, q_head;
  const uint16_t *k;
  int64_t k_pos, k_head;
  const uint16_t *v;
  int64_t v_pos, v_head;
  uint16_t *out;
  int64_t o_tok, o_head;
  uint32_t tokens, q_heads, kv_heads, group, kv_length, causal, query_offset;
  uint32_t row_tiles;       // ceil(T * group / block_m)
  uint32_t block_m;         // packed rows per workgroup: 128, or 256 at D = 128
  float scale_log2;
  // Split-K over keys (small grids). Each split of a row tile that needs
  // several writes its rows to `partial`, laid out
  // [splits][row_tiles][kv_heads][block_m / 32 waves][kPrefillPartialSlots(D)][64 lanes]
  // 8-byte slots: (m, l) as f32, then O[D] / l rounded to f16, four values
  // per slot; then counts its arrival in counters[(tile * kv_heads +
  // kv_head) * counter_stride]; the last split to arrive merges all of them
  // in split order and resets the counter to zero.
  float *partial;
  uint32_t *counters;
  uint32_t counter_stride;
  uint32_t split_tiles;
  uint32_t splits;
  // pieces_per_head != 0: the grid is (pieces_per_head, kv_heads) and the
  // workgroup at position `rest` of its KV head runs the piece
  // order[rest] = row tile << 4 | split, where a row tile of n key tiles has
  // s = ceil(n / split_tiles) splits and split z covers key tiles
  // [z n / s, (z + 1) n / s). pieces_per_head = 0: the grid is (row_tiles,
  // kv_heads, splits) and split z covers key tiles [z * split_tiles,
  // (z + 1) * split_tiles), or all of them when split_tiles = 0.
  uint32_t pieces_per_head;
  uint16_t order[kPrefillOrderMax];
};

// Split pass (one workgroup per key block; writes the output directly when a
// row has one block) and merge pass (combines the partials of rows with more
// than one block; no launch when max_splits <= 1 or when counters are set,
// in which case the split pass merges). Same stream, in order. waves: 2, 4
// or 8 per workgroup.
enum class RowsPhase { Split, Merge };
hipError_t launch_rows(const RowsParams &p, uint32_t head_dim, uint32_t waves,
                       uint32_t chunk, RowsPhase phase, const Launch &l);
// Largest head chunk (of 8, 4, 2, 1) that divides `group`.
uint32_t rows_chunk(uint32_t group);

// Batched decode (one query token per sequence, head_dim 128) on MFMA with
// a stream-K split: p.stream_workgroups workgroups share the keys of all
// sequences equally (each at least kStreamMinKeys). RowsParams as for the
// rows kernel with tokens = 1, head_chunks = group / chunk and per-sequence
// `lengths` (required); `partial` holds stream_partial_floats(units,
// stream_workgroups, chunk, stream_unit_slots) floats: stream_unit_slots
// slots per unit, then stream_workgroups + units overflow slots, each slot
// chunk * (D + 2) floats, then one u32 descriptor per unit. The Split phase
// streams the keys and writes units held by one workgroup directly; the
// first piece of every unit writes its descriptor, first workgroup |
// pieces << 16; a unit of at most stream_unit_slots pieces keeps piece i in
// its own slot i, a longer one in overflow slot (workgroup + unit). With
// stream_unit_slots = 0 (the compact layout, for a fixed buffer too small
// for the unit slots) every piece takes an overflow slot and the merge
// loads them after the descriptor. The Merge phase (next on the same
// stream) merges the pieces of split units, in piece order either way.
// batch <= kStreamMaxBatch; a full 32-key tile of K or V must span less
// than 4 GiB (32 * pos stride * 2 bytes).
constexpr uint32_t kStreamMaxBatch = 1024;
constexpr uint32_t kStreamMinKeys = 512;
constexpr uint32_t kStreamUnitSlots = 8;
constexpr uint64_t stream_partial_floats(uint64_t units, uint64_t workgroups, uint32_t chunk,
                                         uint32_t unit_slots) {
  return (units * unit_slots + workgroups + units) * chunk * (128 + 2) + units;
}
hipError_t launch_decode_stream(const RowsParams &p, uint32_t chunk, RowsPhase phase,
                                const Launch &l);
// Head chunk of the stream kernel: the largest of 16, 8, 4, 2, 1 dividing `group`.
uint32_t stream_chunk(uint32_t group);

// Runs rows [row_begin, row_begin + row_count) of the flattened
// (token, head) grid. Scores of up to kNaiveLdsKeys keys live in LDS; longer
// rows spill to NaiveParams::scores, which must hold row_count * L floats.
hipError_t launch_naive(const NaiveParams &p, uint32_t row_begin,
                        uint32_t row_count, const Launch &l);
constexpr uint32_t kNaiveLdsKeys = 12288;

hipError_t launch_copy_kv(const CopyKvParams &p, const Launch &l);
hipError_t launch_qk_norm_rope(const QkNormRopeParams &p, const Launch &l);

// Rows of up to four dimensions addressed as (i0, i1, i2) over the leading
// dimensions (n1, n2 the inner two; unused ones have size 1), each row
// `width` elements at unit stride.
struct RowIndex {
  uint32_t n1, n2;
  int64_t s0, s1, s2;
};

// RMSNorm over the last dimension: out = x * rsqrt(mean(x^2) + eps) * w.
struct RmsNormParams {
  const uint16_t *x;
  RowIndex x_rows;
  const uint16_t *weight;
  uint16_t *out;
  RowIndex o_rows;
  uint32_t rows, width;
  float epsilon;
};

// RoPE of [T, H, D] (pairs (i, i + D/2)) at position offset + token.
struct RopeParams {
  const uint16_t *x;
  int64_t x_tok, x_head;
  uint16_t *out;
  int64_t o_tok, o_head;
  uint32_t tokens, heads, head_dim, offset;
  float theta;
};

// out[m, n] = x[m, k] . w[n, k]^T with f32 accumulation, for few rows of x:
// the weight is streamed from HBM once per kMatvecRows rows of x.
struct MatvecParams {
  const uint16_t *x;
  int64_t x_row;
  const uint16_t *w;
  int64_t w_row;
  uint16_t *out;
  int64_t o_row;
  uint32_t m, n, k;
};
constexpr uint32_t kMatvecRows = 8;
// Skinny GEMM for kMatvecRows < m <= kSkinnyMaxRows, bound by streaming the
// weight: one workgroup per 16 output features. Requires n % 16 == 0 with
// n / 16 at most the device's CUs, k % (8 * kSkinnyChunkSteps * 64) == 0 and
// x, w rows 16-byte aligned.
constexpr uint32_t kSkinnyMaxRows = 32;
constexpr uint32_t kSkinnyChunkSteps = 2;  // 64-key steps per LDS chunk
bool skinny_gemm_supported(const MatvecParams &p, uint32_t compute_units);
hipError_t launch_skinny_gemm(const MatvecParams &p, uint32_t compute_units, const Launch &l);

hipError_t launch_rms_norm(const RmsNormParams &p, uint32_t compute_units, const Launch &l);
hipError_t launch_rope(const RopeParams &p, const Launch &l);
hipError_t launch_matvec(const MatvecParams &p, const Launch &l);

// Rows of the packed (token, head-in-group) M dimension per prefill
// workgroup, and keys per KV tile.
constexpr uint32_t kPrefillBlockM = 128;
constexpr uint32_t kPrefillBlockM2 = 256;  // large D = 128 grids
constexpr uint32_t kPrefillBlockN = 64;
// Most key splits of one prefill row tile.
constexpr uint32_t kMaxPrefillSplits = 8;
// 8-byte slots per lane of a split partial: (m, l), then O[D] / l as f16,
// four per slot (each lane holds D / 2 values of its row).
constexpr uint32_t kPrefillPartialSlots(uint32_t head_dim) { return 1 + head_dim / 8; }
bool prefill_supported(uint32_t head_dim);
// 128-row prefill workgroups resident per CU: two, or one at head_dim 256.
constexpr uint32_t prefill_workgroups_per_cu(uint32_t head_dim) { return head_dim == 256 ? 1 : 2; }
// One launch, split merges included: grid (pieces_per_head, kv_heads) for an
// ordered split plan, else (row_tiles, kv_heads, splits), where a key split
// past its row tile's last key tile returns at once. Q, K, V and the output
// rows are 16-byte aligned (base and outer strides multiples of 8 elements).
hipError_t launch_prefill(const PrefillParams &p, uint32_t head_dim, const Launch &l);
// Capacity of a context's split-K arrival counters (u32 words: units of a
// fused rows plan, row tiles x KV heads of a split prefill grid, each at
// counter_stride words).
constexpr uint32_t kSplitCounters = 16384;
// Words between two arrival counters: one 128-byte line each where the
// counters fit, else the largest power of two that fits (at least 1).
// Arrivals on one line queue behind each other whatever their addresses
// (measured on MI355X, c2, 8 units x 16 splits: 7.35 against 8.02 us per
// call with the 8 counters packed in one line; the one-launch decode step
// 7.72 against 8.69 us; a 64-byte stride measured the same as 128).
constexpr uint32_t kCounterStride = 32;
constexpr uint32_t counter_stride(uint64_t counters, uint64_t capacity) {
  uint32_t stride = kCounterStride;
  while (stride > 1 && counters * stride > capacity) stride /= 2;
  return stride;
}

}  // namespace kernels
}  // namespace mi
