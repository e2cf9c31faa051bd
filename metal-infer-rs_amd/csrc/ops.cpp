// Attention and KV-cache operations of the C ABI. Validation order and
// error text follow crates/metal-infer-core/src/ops.rs (attention
// :1050-1247, copy_into_cache :1249-1285, qk_norm_rope_cache :917-977);
// the kernel choice is MI355X-specific.
#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "kernels.hpp"
#include "runtime.hpp"

namespace mi {
namespace {

enum class Family { Naive, Rows, Prefill };

struct AttnPlan {
  Family family = Family::Rows;
  uint32_t T = 0, Hq = 0, Hkv = 0, D = 0, L = 0, G = 0;
  uint32_t waves = 4, chunk = 1, block_keys = 0, splits = 1;
  bool fused = false;            // rows: the last split merges (no merge launch)
  uint64_t units = 0;            // rows-kernel (row, KV head, chunk) units
  uint64_t scratch_bytes = 0;
  uint32_t grid[3] = {0, 0, 0};
  uint32_t threads = 0;
  uint32_t block_m = kernels::kPrefillBlockM;  // prefill: packed rows per workgroup
  // Prefill split plans: pieces per KV head in launch order (0: the
  // (row tile, KV head, split) grid); the entry format of PrefillParams::order.
  uint32_t pieces_per_head = 0;
  uint16_t order[kernels::kPrefillOrderMax] = {};
  const char *kernel = "";
};

constexpr uint32_t kU32Max = 0xffffffffu;

bool pow2(uint64_t x) { return x != 0 && (x & (x - 1)) == 0; }

mi_status to_u32(int64_t value, const char *label, uint32_t *out) {
  if (value < 0 || (uint64_t)value > kU32Max)
    return fail(MI_ERR_SHAPE, std::string(label) + " does not fit in u32");
  *out = (uint32_t)value;
  return MI_OK;
}

uint32_t ceil_div(uint64_t a, uint64_t b) { return (uint32_t)((a + b - 1) / b); }

// Whether a rank-3 f16 view can feed the 128-bit-load kernels: unit
// innermost stride, outer strides and base aligned to `vec` halves.
bool vector_friendly(const mi_tensor &t, uint32_t vec) {
  if (t.stride[t.rank - 1] != 1) return false;
  for (int32_t i = 0; i < t.rank - 1; ++i)
    if (t.stride[i] % vec != 0) return false;
  return reinterpret_cast<uintptr_t>(t.data) % (vec * 2) == 0;
}

// Whether tiles of `rows` key rows can be addressed by unsigned 32-bit byte
// offsets from a tile base (the MFMA kernels' direct and register loads):
// both position strides non-negative and a tile spanning less than 4 GiB,
// with a 512-byte margin for the in-row offset.
bool pos_stride_fits_u32(int64_t k_pos, int64_t v_pos, uint32_t rows) {
  if (k_pos < 0 || v_pos < 0) return false;
  return (uint64_t)std::max(k_pos, v_pos) * rows * 2 + 512 < (1ull << 32);
}

// Default split size: about one workgroup per CU, but at least 128 keys
// per split (each split costs a partial write and a merge read). Measured on
// MI355X for the 2048-key decode: 128-key splits beat 32/64/256.
uint32_t default_block(const Context *ctx, uint64_t units, uint32_t keys) {
  const uint64_t cus = std::max<uint32_t>(ctx ? ctx->compute_units : 256, 1);
  const uint64_t most = std::max<uint64_t>(1, (keys + 127) / 128);
  const uint64_t splits = std::min<uint64_t>(most, std::max<uint64_t>(1, (cus + units - 1) / units));
  const uint64_t block = ((keys + splits - 1) / splits + 63) / 64 * 64;
  return (uint32_t)std::max<uint64_t>(64, block);
}

// FlashDecode (block, threads) for a length (context.rs:258-267): the tuned
// table's entry (returns true), else (128, 256) and false, which the planner
// runs as the library default (8 waves, merge inside the launch). A table
// entry with threads 0 is the tuner keeping that default for its lengths.
// The reference's (64, 256) default is an Apple-GPU choice; 128-key splits
// measured fastest here.
bool flash_config_for_length(const Context *ctx, uint64_t length, uint32_t *block,
                             uint32_t *threads) {
  if (ctx != nullptr)
    for (const auto &e : ctx->flash_decode)
      if (length <= e.limit) {
        if (e.threads == 0) break;  // the tuner kept the library default here
        *block = e.block_keys;
        *threads = e.threads;
        return true;
      }
  *block = 128;
  *threads = 256;
  return false;
}

// threads = 0 picks the default: for one decode token of one sequence, 8
// waves per workgroup and the split merge inside the launch (measured on
// MI355X at c2: 9.2 us per call against 10.1 us for 4 waves plus a merge
// launch); otherwise 4 waves. 128 / 256 are the reference's threadgroup
// sizes (2 / 4 waves, separate merge).
mi_status plan_rows(const Context *ctx, AttnPlan *p, uint64_t batch, uint32_t max_keys,
                    uint32_t block_keys, uint32_t threads, bool batched = false) {
  p->family = Family::Rows;
  p->kernel = "attn_rows";
  const bool single_decode = threads == 0 && batch == 1 && p->T == 1;
  p->waves = single_decode ? 8 : threads == 128 ? 2 : 4;
  p->threads = p->waves * 64;
  p->chunk = kernels::rows_chunk(p->G);
  const uint64_t units = batch * p->T * p->Hkv * (p->G / p->chunk);
  p->units = units;
  p->block_keys = block_keys != 0 ? block_keys : default_block(ctx, units, max_keys);
  p->splits = std::max<uint32_t>(1, ceil_div(std::max<uint32_t>(max_keys, 1), p->block_keys));
  const uint64_t counters = ctx ? ctx->split_counter_count : kernels::kSplitCounters;
  // The batched decode merges inside its launch too (4 waves; with the
  // streamed K/V loads measured 2.5% faster at 32 sequences than a merge
  // launch).
  p->fused = (single_decode || batched) && p->splits > 1 && units <= counters;
  p->scratch_bytes =
      p->splits > 1 ? units * p->splits * p->chunk * (uint64_t)(p->D + 2) * sizeof(float) : 0;
  if (batch * p->T > 0xffffu || (uint64_t)p->Hkv * (p->G / p->chunk) > 0xffffu)
    return fail(MI_ERR_SHAPE, "attention grid exceeds the launch limits");
  p->grid[0] = p->splits;
  p->grid[1] = p->Hkv * (p->G / p->chunk);
  p->grid[2] = (uint32_t)(batch * p->T);
  return MI_OK;
}

// Key tiles of each prefill row tile: the kernel's causal window of the row
// tile's last row, in 64-key tiles.
std::vector<uint32_t> prefill_key_tiles(const AttnPlan &p, bool causal, uint32_t query_offset,
                                        uint32_t block_m) {
  std::vector<uint32_t> tiles(ceil_div((uint64_t)p.T * p.G, block_m));
  for (uint64_t t = 0; t < tiles.size(); ++t) {
    const uint64_t last_row = std::min<uint64_t>((uint64_t)p.T * p.G, (t + 1) * block_m) - 1;
    const uint64_t t_last = last_row / p.G;
    const uint64_t kmax = causal ? std::min<uint64_t>(p.L, (uint64_t)query_offset + t_last + 1) : p.L;
    tiles[t] = ceil_div(kmax, kernels::kPrefillBlockN);
  }
  return tiles;
}

// Key splits for prefill grids too small to fill the chip (fewer than the
// resident workgroups: two per CU, one at D = 256): the causally heavy row
// tiles are cut into ranges of whole key tiles, so no workgroup walks the
// full key range while CUs idle. The split count is the largest (up to
// kMaxPrefillSplits) whose non-empty pieces still fit on the chip at once: beyond that
// the pieces queue and each one's fixed cost (Q load, first K/V round trip,
// partial write) outweighs the balance. The last split of a row tile to
// finish merges the f32 partials. Problems with fewer than 8 key tiles are
// not split. `block_m` is the plan's row tile and `per_cu` its resident
// workgroups per CU.
void plan_prefill_splits(const Context *ctx, AttnPlan *p, bool causal, uint32_t query_offset,
                         uint32_t block_m, uint32_t per_cu) {
  p->splits = 1;
  p->block_keys = 0;
  const uint64_t row_tiles = p->grid[0];
  const uint64_t wgs = row_tiles * p->grid[1];
  const uint64_t cus = std::max<uint32_t>(ctx ? ctx->compute_units : 256, 1) * per_cu;
  const uint64_t counters = ctx ? ctx->split_counter_count : kernels::kSplitCounters;
  if (wgs >= cus || wgs > counters) return;
  const std::vector<uint32_t> tiles = prefill_key_tiles(*p, causal, query_offset, block_m);
  const uint32_t max_tiles = *std::max_element(tiles.begin(), tiles.end());
  if (max_tiles < 8) return;
  for (uint32_t want = kernels::kMaxPrefillSplits; want >= 2; --want) {
    const uint32_t per_split = ceil_div(max_tiles, want);
    const uint32_t splits = ceil_div(max_tiles, per_split);
    uint64_t pieces = 0;
    for (uint32_t n : tiles) pieces += ceil_div(n, per_split);
    if (splits < 2 || pieces * p->grid[1] > cus) continue;
    p->splits = splits;
    p->block_keys = per_split * kernels::kPrefillBlockN;
    p->grid[2] = splits;
    p->scratch_bytes = (uint64_t)splits * wgs * (block_m / 32) * kernels::kPrefillPartialSlots(p->D) * 64 *
                       2 * sizeof(float);
    return;
  }
}

// Launch order of a split prefill plan's pieces. Each row tile that needs
// several splits is cut into ceil(tiles / split_tiles) ranges of equal
// length (within one key tile), so no split is longer than it must be. A
// workgroup's piece comes from its position within its KV head; the
// positions are dealt longest piece first. With two resident workgroups per
// CU, workgroups w and w + CUs share a CU (the hardware fills every CU once
// before it fills any twice), and the first of the two issues ahead of the
// second and runs faster while both run: the first CUs positions (CUs / Hkv
// per head) take the longest pieces in order, the rest take the remaining
// pieces shortest first, so each CU's long piece meets a short one (longest
// processing time first, paired). Measured on MI355X, c3 (504 pieces): 34.2-
// 34.8 us per call against 37.1-37.3 us for the (row tile, KV head, split)
// grid with fixed split_tiles ranges, same box. Plans with more than
// kPrefillOrderMax pieces per KV head, and head_dim 256 (one workgroup per
// CU, so no pairing), keep that grid.
void order_prefill_pieces(const Context *ctx, AttnPlan *p, bool causal, uint32_t query_offset,
                          uint32_t per_cu) {
  p->pieces_per_head = 0;
  if (p->splits <= 1 || per_cu != 2 || p->block_m != kernels::kPrefillBlockM) return;
  const uint32_t per_split = p->block_keys / kernels::kPrefillBlockN;
  const std::vector<uint32_t> tiles = prefill_key_tiles(*p, causal, query_offset, p->block_m);
  struct Piece {
    uint32_t len, tile, split;
  };
  std::vector<Piece> pieces;
  for (uint32_t t = 0; t < tiles.size(); ++t) {
    const uint32_t n = tiles[t], ns = ceil_div(n, per_split);
    for (uint32_t s = 0; s < ns; ++s) {
      const uint32_t b = (uint32_t)((uint64_t)s * n / ns), e = (uint32_t)((uint64_t)(s + 1) * n / ns);
      pieces.push_back({e - b, t, s});
    }
    if (pieces.size() > kernels::kPrefillOrderMax || t >= (1u << 12)) return;
  }
  std::stable_sort(pieces.begin(), pieces.end(), [](const Piece &a, const Piece &b) {
    if (a.len != b.len) return a.len > b.len;
    if (a.tile != b.tile) return a.tile > b.tile;
    return a.split < b.split;
  });
  const uint32_t cus = std::max<uint32_t>(ctx ? ctx->compute_units : 256, 1);
  const size_t first = std::min<size_t>(pieces.size(), ceil_div(cus, p->Hkv));
  std::reverse(pieces.begin() + first, pieces.end());
  p->pieces_per_head = (uint32_t)pieces.size();
  for (size_t i = 0; i < pieces.size(); ++i)
    p->order[i] = (uint16_t)(pieces[i].tile << 4 | pieces[i].split);
  p->grid[0] = p->pieces_per_head;
  p->grid[2] = 1;
}

mi_status plan_attention(const Context *ctx, const mi_tensor *q, const mi_tensor *k,
                         const mi_tensor *v, const mi_attention_config *config, int32_t kind,
                         uint32_t block_keys, uint32_t threads, bool flash_explicit,
                         const mi_tensor *out, AttnPlan *plan) {
  if (q == nullptr || k == nullptr || v == nullptr || config == nullptr)
    return fail(MI_ERR_INVALID_ARGUMENT, "null tensor or config");
  if (kind < MI_ATTN_REFERENCE || kind > MI_ATTN_FLASH_DECODE)
    return fail(MI_ERR_INVALID_ARGUMENT, "unknown attention kind");
  mi_status st;
  if ((st = require_f16(q)) != MI_OK || (st = require_f16(k)) != MI_OK ||
      (st = require_f16(v)) != MI_OK)
    return st;
  if (q->rank != 3) return fail(MI_ERR_SHAPE, "query must have rank 3");
  if (k->rank != 3) return fail(MI_ERR_SHAPE, "key must have rank 3");
  if (v->rank != 3) return fail(MI_ERR_SHAPE, "value must have rank 3");
  const int64_t tokens = q->shape[0], kv_length = k->shape[0];
  if (q->shape[1] != (int64_t)config->query_heads || q->shape[2] != (int64_t)config->head_dim ||
      k->shape[1] != (int64_t)config->kv_heads || k->shape[2] != (int64_t)config->head_dim ||
      v->shape[0] != kv_length || v->shape[1] != k->shape[1] || v->shape[2] != k->shape[2])
    return fail(MI_ERR_SHAPE, "attention tensor shapes do not match config");
  if (config->kv_heads == 0 || config->query_heads % config->kv_heads != 0)
    return fail(MI_ERR_SHAPE, "query_heads must be divisible by kv_heads");
  if (kind != MI_ATTN_REFERENCE && (!pow2(config->head_dim) || config->head_dim > 256))
    return fail(MI_ERR_SHAPE, "tiled attention requires a power-of-two head_dim <= 256");
  uint32_t flash_block = 0, flash_threads = 0;
  bool flash_default = false;  // untuned and not explicit: the library default
  if (kind == MI_ATTN_FLASH_DECODE) {
    if (flash_explicit) {
      flash_block = block_keys;
      flash_threads = threads;
    } else {
      flash_default = !flash_config_for_length(ctx, (uint64_t)kv_length, &flash_block,
                                               &flash_threads);
    }
    if (flash_block != 32 && flash_block != 64 && flash_block != 128 && flash_block != 256)
      return fail(MI_ERR_SHAPE, "flash decode block size must be 32, 64, 128, or 256");
    if (flash_threads != 128 && flash_threads != 256)
      return fail(MI_ERR_SHAPE, "flash decode threadgroup size must be 128 or 256");
  }
  if (out != nullptr) {
    if ((st = require_f16(out)) != MI_OK) return st;
    if (out->rank != 3 || out->shape[0] != q->shape[0] || out->shape[1] != q->shape[1] ||
        out->shape[2] != q->shape[2])
      return fail(MI_ERR_SHAPE, "attention output must have the query's shape");
  }
  AttnPlan p;
  uint32_t causal = config->causal != 0 ? 1 : 0;
  (void)causal;
  if ((st = to_u32(tokens, "tokens", &p.T)) != MI_OK) return st;
  if ((st = to_u32(kv_length, "kv_length", &p.L)) != MI_OK) return st;
  p.Hq = config->query_heads;
  p.Hkv = config->kv_heads;
  p.D = config->head_dim;
  p.G = p.Hq / p.Hkv;
  if ((kind == MI_ATTN_DECODE_SPLIT_KV || kind == MI_ATTN_FLASH_DECODE) && tokens != 1)
    return fail(MI_ERR_SHAPE, "decode attention requires exactly one query token");
  // The reference rejects FlashDecode unless Hq == 2 * Hkv (ops.rs:1141);
  // the rows kernel serves every ratio, so that check is lifted.
  const uint64_t window = (uint64_t)config->query_offset + 1;
  const uint32_t available_last =
      config->causal != 0 ? (uint32_t)std::min<uint64_t>(p.L, window + p.T - 1) : p.L;
  if (kind == MI_ATTN_FLASH_DECODE && available_last == 0)
    return fail(MI_ERR_SHAPE, "flash decode requires at least one available key");

  const uint32_t vec = std::min<uint32_t>(8, p.D);
  const bool vectorized = vector_friendly(*q, vec) && vector_friendly(*k, vec) &&
                          vector_friendly(*v, vec) &&
                          (out == nullptr || vector_friendly(*out, 1));
  if (kind == MI_ATTN_REFERENCE || !vectorized) {
    p.family = Family::Naive;
    p.kernel = "attn_naive";
    p.threads = 256;
    p.grid[0] = p.T * p.Hq;
    p.grid[1] = p.grid[2] = 1;
    if (p.L > kernels::kNaiveLdsKeys)
      p.scratch_bytes = (uint64_t)std::min<uint64_t>(p.grid[0], 4096) * p.L * sizeof(float);
    *plan = p;
    return MI_OK;
  }
  if (kind == MI_ATTN_FLASH_PREFILL && kernels::prefill_supported(p.D) &&
      vector_friendly(*q, 8) && vector_friendly(*k, 8) && vector_friendly(*v, 8) &&
      (out == nullptr || vector_friendly(*out, 8)) && (uint64_t)p.T * p.G < (1ull << 31) &&
      // A key tile's per-lane byte offsets (64 rows from the tile base) are
      // unsigned 32-bit: both position strides non-negative, and 64 rows
      // span less than 4 GiB. Other views take the rows kernel (int64).
      pos_stride_fits_u32(k->stride[0], v->stride[0], kernels::kPrefillBlockN)) {
    p.family = Family::Prefill;
    p.kernel = "attn_prefill";
    p.threads = 256;
    p.grid[0] = ceil_div((uint64_t)p.T * p.G, kernels::kPrefillBlockM);
    p.grid[1] = p.Hkv;
    p.grid[2] = 1;
    // Resident 128-row workgroups per CU: two (D = 256: one, by registers and
    // LDS).
    plan_prefill_splits(ctx, &p, config->causal != 0, config->query_offset,
                        kernels::kPrefillBlockM, kernels::prefill_workgroups_per_cu(p.D));
    // The 8-wave row tile (256 rows, one workgroup per CU) shares each K/V
    // tile between twice the rows. Unsplit grids of at least four such
    // workgroups per CU take it (measured on MI355X: c5 +3%; c3 unsplit, 128
    // such workgroups, 30% slower). Grids that take key splits keep the
    // 128-row tile at two workgroups per CU: c3 (3 x 11 key tiles, 504
    // non-empty pieces in a grid of 768) ran 36.2-38.6 us per call against
    // 38.9-39.5 us with 256-row tiles (256 pieces, one per CU), same box.
    const uint64_t cus = std::max<uint32_t>(ctx ? ctx->compute_units : 256, 1);
    const uint64_t big_tiles = ceil_div((uint64_t)p.T * p.G, kernels::kPrefillBlockM2);
    if (p.splits == 1 && p.D == 128 && big_tiles * p.Hkv >= 4 * cus) {
      p.block_m = kernels::kPrefillBlockM2;
      p.threads = 512;
      p.grid[0] = (uint32_t)big_tiles;
    }
    order_prefill_pieces(ctx, &p, config->causal != 0, config->query_offset,
                         kernels::prefill_workgroups_per_cu(p.D));
    *plan = p;
    return MI_OK;
  }
  const uint32_t rows_block = kind == MI_ATTN_FLASH_DECODE ? flash_block : 0;
  uint32_t rows_threads = 256;
  if (kind == MI_ATTN_FLASH_DECODE) rows_threads = flash_default ? 0 : flash_threads;
  if (kind == MI_ATTN_DECODE_SPLIT_KV) rows_threads = 0;
  st = plan_rows(ctx, &p, 1, available_last, rows_block, rows_threads);
  if (st != MI_OK) return st;
  *plan = p;
  return MI_OK;
}

void fill_info(const AttnPlan &p, mi_attention_plan_info *info) {
  std::memset(info, 0, sizeof *info);
  std::snprintf(info->kernel, sizeof info->kernel, "%s", p.kernel);
  for (int i = 0; i < 3; ++i) info->grid[i] = p.grid[i];
  info->block_threads = p.threads;
  info->block_keys = p.family != Family::Naive ? p.block_keys : 0;
  info->splits = p.family != Family::Naive ? p.splits : 1;
  info->scratch_bytes = p.scratch_bytes;
}

mi_status run_rows(Batch *batch, const AttnPlan &p, kernels::RowsParams rp,
                   const ScratchSource &src = ScratchSource{}) {
  Context *ctx = batch->ctx;
  void *scratch = nullptr;
  mi_status st;
  if (p.splits > 1) {
    if ((st = scratch_take(batch, src, p.scratch_bytes, &scratch)) != MI_OK) return st;
  }
  const bool events = src.fixed == nullptr;
  rp.partial = static_cast<float *>(scratch);
  rp.counters = p.fused ? ctx->split_counters : nullptr;
  rp.counter_stride = kernels::counter_stride(p.units, ctx->split_counter_count);
  rp.block_keys = p.block_keys;
  rp.max_splits = p.splits;
  rp.head_chunks = p.G / p.chunk;
  rp.group = p.G;
  st = launch(batch, p.kernel, [&](const kernels::Launch &s) {
    return kernels::launch_rows(rp, p.D, p.waves, p.chunk, kernels::RowsPhase::Split, s);
  }, events);
  if (st == MI_OK && p.splits > 1 && !p.fused)
    st = launch(batch, "attn_merge", [&](const kernels::Launch &s) {
      return kernels::launch_rows(rp, p.D, p.waves, p.chunk, kernels::RowsPhase::Merge, s);
    }, events);
  // In-order execution makes the range reusable by later work of the batch.
  scratch_give(ctx, src, scratch);
  return st;
}

mi_status run_attention(Batch *batch, const mi_tensor *q, const mi_tensor *k,
                        const mi_tensor *v, const mi_attention_config *config, int32_t kind,
                        uint32_t block_keys, uint32_t threads, bool flash_explicit,
                        const mi_tensor *out) {
  if (batch == nullptr || out == nullptr)
    return fail(MI_ERR_INVALID_ARGUMENT, "null batch or output");
  if (batch->committed) return fail(MI_ERR_RESOURCE, "batch was already committed");
  AttnPlan p;
  mi_status st = plan_attention(batch->ctx, q, k, v, config, kind, block_keys, threads,
                                flash_explicit, out, &p);
  if (st != MI_OK) return st;
  const float scale = 1.0f / std::sqrt((float)p.D);
  const float log2e = 1.4426950408889634f;
  auto qd = static_cast<const uint16_t *>(q->data);
  auto kd = static_cast<const uint16_t *>(k->data);
  auto vd = static_cast<const uint16_t *>(v->data);
  auto od = static_cast<uint16_t *>(out->data);
  if (p.family == Family::Naive) {
    kernels::NaiveParams np{};
    np.q = qd, np.q_tok = q->stride[0], np.q_head = q->stride[1];
    np.k = kd, np.k_pos = k->stride[0], np.k_head = k->stride[1];
    np.v = vd, np.v_pos = v->stride[0], np.v_head = v->stride[1];
    np.out = od, np.o_tok = out->stride[0], np.o_head = out->stride[1];
    np.tokens = p.T, np.q_heads = p.Hq, np.kv_heads = p.Hkv, np.head_dim = p.D;
    np.kv_length = p.L, np.causal = config->causal != 0, np.query_offset = config->query_offset;
    np.scale = scale;
    if (q->stride[2] != 1 || k->stride[2] != 1 || v->stride[2] != 1 || out->stride[2] != 1)
      return fail(MI_ERR_SHAPE, "attention tensors need a unit innermost stride");
    const uint32_t rows = p.T * p.Hq;
    uint32_t chunk_rows = rows;
    void *scores = nullptr;
    if (p.L > kernels::kNaiveLdsKeys) {
      chunk_rows = (uint32_t)(p.scratch_bytes / ((uint64_t)p.L * sizeof(float)));
      if ((st = scratch_alloc(batch, p.scratch_bytes, &scores)) != MI_OK) return st;
      np.scores = static_cast<float *>(scores);
    }
    for (uint32_t begin = 0; begin < rows && st == MI_OK; begin += chunk_rows) {
      const uint32_t count = std::min(chunk_rows, rows - begin);
      st = launch(batch, p.kernel,
                  [&](const kernels::Launch &s) { return kernels::launch_naive(np, begin, count, s); });
    }
    if (scores != nullptr) scratch_free(batch->ctx, scores);
    return st;
  }
  if (p.family == Family::Prefill) {
    kernels::PrefillParams pp{};
    pp.q = qd, pp.q_tok = q->stride[0], pp.q_head = q->stride[1];
    pp.k = kd, pp.k_pos = k->stride[0], pp.k_head = k->stride[1];
    pp.v = vd, pp.v_pos = v->stride[0], pp.v_head = v->stride[1];
    pp.out = od, pp.o_tok = out->stride[0], pp.o_head = out->stride[1];
    pp.tokens = p.T, pp.q_heads = p.Hq, pp.kv_heads = p.Hkv, pp.group = p.G;
    pp.kv_length = p.L, pp.causal = config->causal != 0, pp.query_offset = config->query_offset;
    pp.row_tiles = ceil_div((uint64_t)p.T * p.G, p.block_m);
    pp.block_m = p.block_m;
    pp.scale_log2 = scale * log2e;
    pp.splits = p.splits;
    pp.split_tiles = p.splits > 1 ? p.block_keys / kernels::kPrefillBlockN : 0;
    pp.pieces_per_head = p.pieces_per_head;
    std::copy(std::begin(p.order), std::end(p.order), std::begin(pp.order));
    void *scratch = nullptr;
    mi_status st;
    if (p.splits > 1) {
      if ((st = scratch_alloc(batch, p.scratch_bytes, &scratch)) != MI_OK) return st;
    }
    pp.partial = static_cast<float *>(scratch);
    pp.counters = batch->ctx->split_counters;
    pp.counter_stride =
        kernels::counter_stride((uint64_t)pp.row_tiles * p.Hkv, batch->ctx->split_counter_count);
    st = launch(batch, p.kernel, [&](const kernels::Launch &s) {
      return kernels::launch_prefill(pp, p.D, s);
    });
    // In-order execution makes the range reusable by later work of the batch.
    if (scratch != nullptr) scratch_free(batch->ctx, scratch);
    return st;
  }
  kernels::RowsParams rp{};
  rp.q = qd, rp.q_seq = 0, rp.q_tok = q->stride[0], rp.q_head = q->stride[1];
  rp.k = kd, rp.k_seq = 0, rp.k_pos = k->stride[0], rp.k_head = k->stride[1];
  rp.v = vd, rp.v_seq = 0, rp.v_pos = v->stride[0], rp.v_head = v->stride[1];
  rp.out = od, rp.o_seq = 0, rp.o_tok = out->stride[0], rp.o_head = out->stride[1];
  rp.lengths = nullptr;
  rp.batch = 1, rp.tokens = p.T, rp.q_heads = p.Hq, rp.kv_heads = p.Hkv;
  rp.kv_length = p.L, rp.causal = config->causal != 0, rp.query_offset = config->query_offset;
  rp.scale_log2 = scale * log2e;
  return run_rows(batch, p, rp);
}

// copy_into_cache's validation (ops.rs:1249-1285): source [T, H, D] into
// cache [C, H, D] at `offset`.
mi_status check_kv_append(const mi_tensor *source, const mi_tensor *cache, uint64_t offset) {
  mi_status st;
  if ((st = require_f16(source)) != MI_OK || (st = require_f16(cache)) != MI_OK) return st;
  if (source->rank != 3) return fail(MI_ERR_SHAPE, "KV source must have rank 3");
  if (cache->rank != 3) return fail(MI_ERR_SHAPE, "KV cache must have rank 3");
  if (source->shape[1] != cache->shape[1] || source->shape[2] != cache->shape[2])
    return fail(MI_ERR_SHAPE, "KV source/cache shapes are incompatible");
  if (offset + (uint64_t)source->shape[0] > (uint64_t)cache->shape[0])
    return fail(MI_ERR_SHAPE, "KV cache capacity exceeded");
  if (source->stride[2] != 1 || cache->stride[2] != 1)
    return fail(MI_ERR_SHAPE, "KV rows need a unit innermost stride");
  uint32_t tmp;
  if ((st = to_u32(source->shape[0], "tokens", &tmp)) != MI_OK) return st;
  if ((st = to_u32((int64_t)offset, "offset", &tmp)) != MI_OK) return st;
  if ((st = to_u32(source->shape[1] * source->shape[2], "stride", &tmp)) != MI_OK) return st;
  return MI_OK;
}

// qk_norm_rope_cache's validation (ops.rs:917-977) and its kernel parameters.
mi_status prepare_qk_norm_rope(mi_batch *batch, const mi_tensor *q, const mi_tensor *k,
                               const mi_tensor *q_weight, const mi_tensor *k_weight,
                               const mi_tensor *key_cache,
                               const mi_qk_norm_rope_cache_config *config,
                               const mi_tensor *q_out, kernels::QkNormRopeParams *out) {
  if (batch == nullptr || q == nullptr || k == nullptr || q_weight == nullptr ||
      k_weight == nullptr || key_cache == nullptr || config == nullptr || q_out == nullptr)
    return fail(MI_ERR_INVALID_ARGUMENT, "null batch, tensor or config");
  if (batch->committed) return fail(MI_ERR_RESOURCE, "batch was already committed");
  mi_status st;
  if ((st = require_f16(q)) != MI_OK || (st = require_f16(k)) != MI_OK ||
      (st = require_f16(q_weight)) != MI_OK || (st = require_f16(k_weight)) != MI_OK ||
      (st = require_f16(key_cache)) != MI_OK)
    return st;
  if (q->rank != 3) return fail(MI_ERR_SHAPE, "query must have rank 3");
  if (k->rank != 3) return fail(MI_ERR_SHAPE, "key must have rank 3");
  if (key_cache->rank != 3) return fail(MI_ERR_SHAPE, "key cache must have rank 3");
  const int64_t tokens = q->shape[0], head_dim = q->shape[2];
  if (tokens != k->shape[0] || head_dim != k->shape[2] || k->shape[1] != key_cache->shape[1] ||
      head_dim != key_cache->shape[2] || q_weight->rank != 1 || q_weight->shape[0] != head_dim ||
      k_weight->rank != 1 || k_weight->shape[0] != head_dim)
    return fail(MI_ERR_SHAPE, "Q/K transform tensor shapes are incompatible");
  if (head_dim % 2 != 0 || (uint64_t)config->offset + (uint64_t)tokens > (uint64_t)key_cache->shape[0])
    return fail(MI_ERR_SHAPE, "Q/K transform has invalid head_dim or cache offset");
  if ((st = require_f16(q_out)) != MI_OK) return st;
  if (q_out->rank != 3 || q_out->shape[0] != q->shape[0] || q_out->shape[1] != q->shape[1] ||
      q_out->shape[2] != q->shape[2])
    return fail(MI_ERR_SHAPE, "Q/K transform output must have the query's shape");
  if (q->stride[2] != 1 || k->stride[2] != 1 || key_cache->stride[2] != 1 ||
      q_out->stride[2] != 1 || q_weight->stride[0] != 1 || k_weight->stride[0] != 1)
    return fail(MI_ERR_SHAPE, "Q/K transform tensors need a unit innermost stride");
  kernels::QkNormRopeParams &qp = *out;
  qp = kernels::QkNormRopeParams{};
  if ((st = to_u32(tokens, "tokens", &qp.tokens)) != MI_OK) return st;
  if ((st = to_u32(q->shape[1], "query heads", &qp.q_heads)) != MI_OK) return st;
  if ((st = to_u32(k->shape[1], "KV heads", &qp.kv_heads)) != MI_OK) return st;
  if ((st = to_u32(head_dim, "head dim", &qp.head_dim)) != MI_OK) return st;
  qp.offset = config->offset;
  qp.theta = config->theta;
  qp.epsilon = config->epsilon;
  qp.q = static_cast<const uint16_t *>(q->data), qp.q_tok = q->stride[0], qp.q_head = q->stride[1];
  qp.k = static_cast<const uint16_t *>(k->data), qp.k_tok = k->stride[0], qp.k_head = k->stride[1];
  qp.q_weight = static_cast<const uint16_t *>(q_weight->data);
  qp.k_weight = static_cast<const uint16_t *>(k_weight->data);
  qp.q_out = static_cast<uint16_t *>(q_out->data);
  qp.qo_tok = q_out->stride[0], qp.qo_head = q_out->stride[1];
  qp.cache = static_cast<uint16_t *>(key_cache->data);
  qp.c_pos = key_cache->stride[0], qp.c_head = key_cache->stride[1];
  return MI_OK;
}

// mi_attention_decode_batched with the split partials from `src`.
mi_status decode_batched(mi_batch *batch, const mi_tensor *q, const mi_tensor *k,
                         const mi_tensor *v, const mi_tensor *lengths,
                         const mi_attention_config *config, uint32_t block_keys,
                         const mi_tensor *out, const ScratchSource &src) {
  if (batch == nullptr || q == nullptr || k == nullptr || v == nullptr || lengths == nullptr ||
      config == nullptr || out == nullptr)
    return fail(MI_ERR_INVALID_ARGUMENT, "null batch, tensor or config");
  if (batch->committed) return fail(MI_ERR_RESOURCE, "batch was already committed");
  mi_status st;
  if ((st = require_f16(q)) != MI_OK || (st = require_f16(k)) != MI_OK ||
      (st = require_f16(v)) != MI_OK || (st = require_f16(out)) != MI_OK)
    return st;
  if (lengths->dtype != MI_U32)
    return fail(MI_ERR_DTYPE, std::string("unsupported dtype: expected u32, got ") +
                                  dtype_name(lengths->dtype));
  if (q->rank != 3) return fail(MI_ERR_SHAPE, "query must have rank 3");
  if (k->rank != 4 || v->rank != 4) return fail(MI_ERR_SHAPE, "batched KV must have rank 4");
  if (lengths->rank != 1) return fail(MI_ERR_SHAPE, "lengths must have rank 1");
  const int64_t B = q->shape[0], C = k->shape[1];
  if (q->shape[1] != (int64_t)config->query_heads || q->shape[2] != (int64_t)config->head_dim ||
      k->shape[0] != B || k->shape[2] != (int64_t)config->kv_heads ||
      k->shape[3] != (int64_t)config->head_dim || v->shape[0] != B || v->shape[1] != C ||
      v->shape[2] != k->shape[2] || v->shape[3] != k->shape[3] || lengths->shape[0] != B ||
      out->rank != 3 || out->shape[0] != B || out->shape[1] != q->shape[1] ||
      out->shape[2] != q->shape[2])
    return fail(MI_ERR_SHAPE, "attention tensor shapes do not match config");
  if (config->kv_heads == 0 || config->query_heads % config->kv_heads != 0)
    return fail(MI_ERR_SHAPE, "query_heads must be divisible by kv_heads");
  if (!pow2(config->head_dim) || config->head_dim > 256)
    return fail(MI_ERR_SHAPE, "tiled attention requires a power-of-two head_dim <= 256");
  const uint32_t vec = std::min<uint32_t>(8, config->head_dim);
  if (!vector_friendly(*q, vec) || !vector_friendly(*k, vec) || !vector_friendly(*v, vec) ||
      !vector_friendly(*out, 1))
    return fail(MI_ERR_SHAPE, "batched decode needs unit-stride, vector-aligned rows");
  AttnPlan p;
  if ((st = to_u32(B, "batch", &p.T)) != MI_OK) return st;
  if ((st = to_u32(C, "kv capacity", &p.L)) != MI_OK) return st;
  p.T = 1;
  p.Hq = config->query_heads, p.Hkv = config->kv_heads, p.D = config->head_dim;
  p.G = p.Hq / p.Hkv;
  // Tensor views and per-sequence lengths, shared by both kernels.
  kernels::RowsParams rp{};
  rp.q = static_cast<const uint16_t *>(q->data);
  rp.q_seq = q->stride[0], rp.q_tok = 0, rp.q_head = q->stride[1];
  rp.k = static_cast<const uint16_t *>(k->data);
  rp.k_seq = k->stride[0], rp.k_pos = k->stride[1], rp.k_head = k->stride[2];
  rp.v = static_cast<const uint16_t *>(v->data);
  rp.v_seq = v->stride[0], rp.v_pos = v->stride[1], rp.v_head = v->stride[2];
  rp.out = static_cast<uint16_t *>(out->data);
  rp.o_seq = out->stride[0], rp.o_tok = 0, rp.o_head = out->stride[1];
  rp.lengths = static_cast<const uint32_t *>(lengths->data);
  rp.batch = (uint32_t)B, rp.tokens = 1, rp.q_heads = p.Hq, rp.kv_heads = p.Hkv;
  rp.kv_length = p.L, rp.causal = 1, rp.query_offset = 0;
  rp.scale_log2 = (1.0f / std::sqrt((float)p.D)) * 1.4426950408889634f;
  // Default: the stream-K MFMA kernel (head_dim 128), which gives every
  // workgroup the same share of all sequences' keys (2 per CU), then its
  // merge launch. Explicit split sizes keep the rows kernel.
  if (block_keys == 0 && p.D == 128 && (uint64_t)B <= kernels::kStreamMaxBatch &&
      pos_stride_fits_u32(k->stride[1], v->stride[1], 32)) {
    const uint32_t chunk = kernels::stream_chunk(p.G);
    const uint64_t units = (uint64_t)B * p.Hkv * (p.G / chunk);
    const uint32_t workgroups = 2 * std::max<uint32_t>(batch->ctx->compute_units, 1);
    rp.group = p.G, rp.head_chunks = p.G / chunk;
    rp.stream_workgroups = workgroups;
    // Fixed slots per unit, so that the merge loads a unit's pieces with its
    // descriptor; a fixed buffer too small for them takes the compact layout
    // (every piece in an overflow slot, same merge order and results).
    uint32_t unit_slots = kernels::kStreamUnitSlots;
    uint64_t bytes = kernels::stream_partial_floats(units, workgroups, chunk, unit_slots) * sizeof(float);
    if (src.fixed != nullptr && bytes > src.limit) {
      unit_slots = 0;
      bytes = kernels::stream_partial_floats(units, workgroups, chunk, 0) * sizeof(float);
    }
    rp.stream_unit_slots = unit_slots;
    void *scratch = nullptr;
    if ((st = scratch_take(batch, src, bytes, &scratch)) != MI_OK) return st;
    rp.partial = static_cast<float *>(scratch);
    const bool events = src.fixed == nullptr;
    st = launch(batch, "attn_decode_stream", [&](const kernels::Launch &s) {
      return kernels::launch_decode_stream(rp, chunk, kernels::RowsPhase::Split, s);
    }, events);
    if (st == MI_OK)
      st = launch(batch, "attn_decode_stream_merge", [&](const kernels::Launch &s) {
        return kernels::launch_decode_stream(rp, chunk, kernels::RowsPhase::Merge, s);
      }, events);
    // In-order execution makes the range reusable by later work of the batch.
    scratch_give(batch->ctx, src, scratch);
    return st;
  }
  // 768-key splits (measured at B=32, L ~ U[1024, 8192], whole call: 768 ->
  // 4.7 TB/s; 640-960 -> 4.5-4.7; every power of two 512-4096 -> 3.8-4.1).
  // Power-of-two splits start every workgroup at the same offset modulo a
  // large power of two, so the workgroups, which stream in lockstep, keep
  // landing on the same HBM channels.
  if (block_keys == 0) block_keys = std::min<uint32_t>(768, std::max<uint32_t>(64, p.L));
  if ((st = plan_rows(batch->ctx, &p, (uint64_t)B, p.L, block_keys, 256, true)) != MI_OK)
    return st;
  p.kernel = "attn_rows_batched";
  return run_rows(batch, p, rp, src);
}

}  // namespace
}  // namespace mi

using namespace mi;

extern "C" {

mi_status mi_attention(mi_batch *batch, const mi_tensor *q, const mi_tensor *k,
                       const mi_tensor *v, const mi_attention_config *config, int32_t kind,
                       const mi_tensor *out) {
  return run_attention(batch, q, k, v, config, kind, 0, 0, false, out);
}

mi_status mi_attention_flash_decode_with_block(mi_batch *batch, const mi_tensor *q,
                                               const mi_tensor *k, const mi_tensor *v,
                                               const mi_attention_config *config,
                                               uint32_t block_keys, const mi_tensor *out) {
  return run_attention(batch, q, k, v, config, MI_ATTN_FLASH_DECODE, block_keys, 256, true, out);
}

mi_status mi_attention_flash_decode_with_configuration(
    mi_batch *batch, const mi_tensor *q, const mi_tensor *k, const mi_tensor *v,
    const mi_attention_config *config, uint32_t block_keys, uint32_t threads,
    const mi_tensor *out) {
  return run_attention(batch, q, k, v, config, MI_ATTN_FLASH_DECODE, block_keys, threads, true,
                       out);
}

mi_status mi_attention_plan(const mi_context *ctx, const mi_tensor *q, const mi_tensor *k,
                            const mi_tensor *v, const mi_attention_config *config, int32_t kind,
                            uint32_t block_keys, uint32_t threads,
                            mi_attention_plan_info *info) {
  if (info == nullptr) return fail(MI_ERR_INVALID_ARGUMENT, "null plan output");
  AttnPlan p;
  const bool explicit_flash = block_keys != 0 || threads != 0;
  mi_status st = plan_attention(ctx, q, k, v, config, kind, block_keys, threads,
                                explicit_flash, nullptr, &p);
  if (st != MI_OK) return st;
  fill_info(p, info);
  return MI_OK;
}

mi_status mi_attention_decode_batched(mi_batch *batch, const mi_tensor *q, const mi_tensor *k,
                                      const mi_tensor *v, const mi_tensor *lengths,
                                      const mi_attention_config *config, uint32_t block_keys,
                                      const mi_tensor *out) {
  return decode_batched(batch, q, k, v, lengths, config, block_keys, out, ScratchSource{});
}

mi_status mi_attention_decode_batched_noalloc(mi_batch *batch, const mi_tensor *q,
                                              const mi_tensor *k, const mi_tensor *v,
                                              const mi_tensor *lengths,
                                              const mi_attention_config *config,
                                              uint32_t block_keys, const mi_tensor *out) {
  if (batch == nullptr) return fail(MI_ERR_INVALID_ARGUMENT, "null batch, tensor or config");
  ScratchSource src;
  src.fixed = noalloc_scratch(batch->ctx->device);
  src.limit = kNoAllocScratchBytes;
  if (src.fixed == nullptr)
    return fail(MI_ERR_RESOURCE, "the no-allocation scratch is not set up on this device");
  mi_status st = noalloc_acquire(batch->ctx, batch->capturing);
  if (st != MI_OK) return st;
  st = decode_batched(batch, q, k, v, lengths, config, block_keys, out, src);
  if (st == MI_OK) noalloc_mark(batch->ctx, batch->capturing);
  return st;
}

mi_status mi_flash_decode_configuration_for_length(const mi_context *ctx, uint64_t length,
                                                   uint32_t *block_keys, uint32_t *threads) {
  if (block_keys == nullptr || threads == nullptr)
    return fail(MI_ERR_INVALID_ARGUMENT, "null output");
  flash_config_for_length(ctx, length, block_keys, threads);
  return MI_OK;
}

namespace {

// The tuner's device buffers, freed on every path out of it.
struct TuneBuffers {
  mi_context *ctx;
  mi_tensor q{}, key{}, value{}, out{};
  ~TuneBuffers() {
    for (mi_tensor *t : {&q, &key, &value, &out})
      if (t->data != nullptr) mi_tensor_free(ctx, t);
  }
};

// Median GPU time of `samples` one-call batches of FlashDecode over
// (q, key, value), with the given (block, threads), or the library default
// when `threads` is 0; UINT64_MAX if any call fails.
uint64_t time_flash_decode(mi_context *ctx, const TuneBuffers &b, const mi_tensor &key,
                           const mi_tensor &value, const mi_attention_config &cfg, uint32_t block,
                           uint32_t threads) {
  constexpr int kSamples = 5;
  uint64_t samples[kSamples];
  for (auto &sample : samples) {
    mi_batch *batch = nullptr;
    mi_dispatch_stats stats{};
    if (mi_batch_begin(ctx, &batch) != MI_OK) return UINT64_MAX;
    const mi_status st =
        threads == 0 ? mi_attention(batch, &b.q, &key, &value, &cfg, MI_ATTN_FLASH_DECODE, &b.out)
                     : mi_attention_flash_decode_with_configuration(batch, &b.q, &key, &value, &cfg,
                                                                    block, threads, &b.out);
    if (st != MI_OK) {
      mi_batch_abandon(batch);
      return UINT64_MAX;
    }
    if (mi_batch_finish(batch, &stats) != MI_OK) return UINT64_MAX;
    sample = stats.gpu_ns;
  }
  std::sort(samples, samples + kSamples);
  return samples[kSamples / 2];
}

}  // namespace

mi_status mi_tune_flash_decode(mi_context *ctx, uint32_t query_heads, uint32_t kv_heads,
                               uint32_t head_dim) {
  if (ctx == nullptr) return fail(MI_ERR_INVALID_ARGUMENT, "null context");
  if (kv_heads == 0 || head_dim == 0 || query_heads % kv_heads != 0 || !pow2(head_dim) ||
      head_dim > 256)
    return MI_OK;  // nothing to tune, as the reference's early return
  using clock = std::chrono::steady_clock;
  const auto started = clock::now();
  const auto budget = std::chrono::seconds(2);
  // The reference's lengths and (block, threads) candidates and 2 s budget
  // (context.rs:269-338), plus the library default (threads 0: 8 waves, the
  // split merge inside the launch), which every candidate has to beat by
  // kMargin to replace it. A length the budget leaves untimed keeps the
  // default, so tuning never selects a slower path than no tuning.
  const uint64_t lengths[] = {512, 640, 1024, 2048, 4096, 8192};
  const uint64_t maximum = 8192;
  const uint32_t candidates[8][2] = {{64, 256}, {32, 256},  {128, 256}, {256, 256},
                                     {64, 128}, {32, 128}, {128, 128}, {256, 128}};
  constexpr double kMargin = 0.97;
  const int64_t qshape[3] = {1, query_heads, head_dim};
  const int64_t cshape[3] = {(int64_t)maximum, kv_heads, head_dim};
  TuneBuffers b{ctx};
  mi_status st;
  if ((st = mi_tensor_empty(ctx, qshape, 3, MI_F16, &b.q)) != MI_OK ||
      (st = mi_tensor_empty(ctx, cshape, 3, MI_F16, &b.key)) != MI_OK ||
      (st = mi_tensor_empty(ctx, cshape, 3, MI_F16, &b.value)) != MI_OK ||
      (st = mi_tensor_empty(ctx, qshape, 3, MI_F16, &b.out)) != MI_OK)
    return st;
  // 1.0 queries and 0.5 cache entries (context.rs:282-287).
  hipError_t err = hipSuccess;
  const std::pair<const mi_tensor *, unsigned short> fills[] = {
      {&b.q, 0x3c00}, {&b.key, 0x3800}, {&b.value, 0x3800}};
  for (const auto &[t, bits] : fills)
    if (err == hipSuccess)
      err = hipMemsetD16Async(reinterpret_cast<hipDeviceptr_t>(t->data), bits, element_count(*t),
                              ctx->stream);
  if (err == hipSuccess) err = hipStreamSynchronize(ctx->stream);
  if (err != hipSuccess)
    return fail(MI_ERR_COMMAND, std::string("flash decode tuning inputs: ") + hipGetErrorString(err));
  // Time against the untuned library (a table from an earlier call would
  // redirect the default candidate).
  ctx->flash_decode.clear();
  std::vector<FlashDecodeEntry> chosen;
  for (uint64_t length : lengths) {
    if (clock::now() - started >= budget) break;
    mi_tensor k_prefix, v_prefix;
    if (mi_tensor_prefix(&b.key, (int64_t)length, &k_prefix) != MI_OK ||
        mi_tensor_prefix(&b.value, (int64_t)length, &v_prefix) != MI_OK)
      break;
    const mi_attention_config cfg{query_heads, kv_heads, head_dim, 1, (uint32_t)(length - 1)};
    const uint64_t default_ns = time_flash_decode(ctx, b, k_prefix, v_prefix, cfg, 0, 0);
    uint64_t best_ns = UINT64_MAX;
    uint32_t best_block = 0, best_threads = 0;
    for (const auto &cand : candidates) {
      if (clock::now() - started >= budget) break;
      const uint64_t ns = time_flash_decode(ctx, b, k_prefix, v_prefix, cfg, cand[0], cand[1]);
      if (ns < best_ns) {
        best_ns = ns;
        best_block = cand[0];
        best_threads = cand[1];
      }
    }
    if (default_ns == UINT64_MAX || best_ns == UINT64_MAX ||
        (double)best_ns >= kMargin * (double)default_ns)
      chosen.push_back({length, 0, 0});  // the library default
    else
      chosen.push_back({length, best_block, best_threads});
  }
  // Lengths past the last timed one keep the default too.
  ctx->flash_decode = chosen;
  clear_error();
  return MI_OK;
}

int32_t mi_attention_kind_for_tokens(int32_t configured, uint64_t tokens, uint64_t active_length,
                                     uint64_t query_heads_per_kv) {
  // qwen3.rs:799-822 with the G == 2 condition lifted: the split-K kernel is
  // ratio-generic, so long single-token decodes take FlashDecode for every
  // GQA ratio.
  (void)query_heads_per_kv;
  switch (configured) {
    case MI_ATTN_TILED:
      if (tokens >= 32) return MI_ATTN_FLASH_PREFILL;
      if (tokens == 1) return active_length >= 256 ? MI_ATTN_FLASH_DECODE : MI_ATTN_DECODE_SPLIT_KV;
      return MI_ATTN_TILED;
    case MI_ATTN_DECODE_SPLIT_KV:
      return tokens == 1 ? MI_ATTN_DECODE_SPLIT_KV : MI_ATTN_TILED;
    case MI_ATTN_FLASH_DECODE:
      return tokens == 1 ? MI_ATTN_FLASH_DECODE : MI_ATTN_TILED;
    case MI_ATTN_FLASH_PREFILL:
      if (tokens == 1) return active_length >= 256 ? MI_ATTN_FLASH_DECODE : MI_ATTN_DECODE_SPLIT_KV;
      return MI_ATTN_FLASH_PREFILL;
    default:
      return configured;
  }
}

mi_status mi_copy_into_cache(mi_batch *batch, const mi_tensor *source, const mi_tensor *cache,
                             uint64_t offset) {
  if (batch == nullptr || source == nullptr || cache == nullptr)
    return fail(MI_ERR_INVALID_ARGUMENT, "null batch or tensor");
  if (batch->committed) return fail(MI_ERR_RESOURCE, "batch was already committed");
  mi_status st;
  if ((st = check_kv_append(source, cache, offset)) != MI_OK) return st;
  kernels::CopyKvParams cp{};
  cp.tokens = (uint32_t)source->shape[0];
  cp.offset = (uint32_t)offset;
  cp.src = static_cast<const uint16_t *>(source->data);
  cp.s_tok = source->stride[0], cp.s_head = source->stride[1];
  cp.dst = static_cast<uint16_t *>(cache->data);
  cp.d_pos = cache->stride[0], cp.d_head = cache->stride[1];
  cp.heads = (uint32_t)source->shape[1];
  cp.head_dim = (uint32_t)source->shape[2];
  return launch(batch, "copy_kv", [&](const kernels::Launch &s) { return kernels::launch_copy_kv(cp, s); });
}

mi_status mi_qk_norm_rope_cache(mi_batch *batch, const mi_tensor *q, const mi_tensor *k,
                                const mi_tensor *q_weight, const mi_tensor *k_weight,
                                const mi_tensor *key_cache,
                                const mi_qk_norm_rope_cache_config *config,
                                const mi_tensor *q_out) {
  kernels::QkNormRopeParams qp;
  mi_status st = prepare_qk_norm_rope(batch, q, k, q_weight, k_weight, key_cache, config, q_out, &qp);
  if (st != MI_OK) return st;
  return launch(batch, "qk_norm_rope_cache",
                [&](const kernels::Launch &s) { return kernels::launch_qk_norm_rope(qp, s); });
}

mi_status mi_qk_norm_rope_cache_value(mi_batch *batch, const mi_tensor *q, const mi_tensor *k,
                                      const mi_tensor *value, const mi_tensor *q_weight,
                                      const mi_tensor *k_weight, const mi_tensor *key_cache,
                                      const mi_tensor *value_cache,
                                      const mi_qk_norm_rope_cache_config *config,
                                      const mi_tensor *q_out) {
  if (value == nullptr || value_cache == nullptr)
    return fail(MI_ERR_INVALID_ARGUMENT, "null batch, tensor or config");
  kernels::QkNormRopeParams qp;
  mi_status st = prepare_qk_norm_rope(batch, q, k, q_weight, k_weight, key_cache, config, q_out, &qp);
  if (st != MI_OK) return st;
  if ((st = check_kv_append(value, value_cache, config->offset)) != MI_OK) return st;
  if (value->shape[0] != q->shape[0] || value->shape[1] != k->shape[1] ||
      value->shape[2] != k->shape[2])
    return fail(MI_ERR_SHAPE, "value rows must have the key's shape");
  qp.v = static_cast<const uint16_t *>(value->data);
  qp.v_tok = value->stride[0], qp.v_head = value->stride[1];
  qp.v_cache = static_cast<uint16_t *>(value_cache->data);
  qp.vc_pos = value_cache->stride[0], qp.vc_head = value_cache->stride[1];
  return launch(batch, "qk_norm_rope_cache",
                [&](const kernels::Launch &s) { return kernels::launch_qk_norm_rope(qp, s); });
}

mi_status mi_decode_step_attention(mi_batch *batch, const mi_tensor *q, const mi_tensor *k,
                                   const mi_tensor *value, const mi_tensor *q_weight,
                                   const mi_tensor *k_weight, const mi_tensor *key_cache,
                                   const mi_tensor *value_cache,
                                   const mi_qk_norm_rope_cache_config *qk_config,
                                   const mi_attention_config *config, const mi_tensor *out) {
  if (value == nullptr || value_cache == nullptr || config == nullptr || out == nullptr)
    return fail(MI_ERR_INVALID_ARGUMENT, "null batch, tensor or config");
  // Validation of the three calls this replaces. The rotated query is not
  // returned, so the query itself stands in for q_out's shape check.
  kernels::QkNormRopeParams qp;
  mi_status st = prepare_qk_norm_rope(batch, q, k, q_weight, k_weight, key_cache, qk_config, q, &qp);
  if (st != MI_OK) return st;
  if ((st = check_kv_append(value, value_cache, qk_config->offset)) != MI_OK) return st;
  if (value->shape[0] != q->shape[0] || value->shape[1] != k->shape[1] ||
      value->shape[2] != k->shape[2])
    return fail(MI_ERR_SHAPE, "value rows must have the key's shape");
  if (q->shape[0] != 1) return fail(MI_ERR_SHAPE, "decode attention requires exactly one query token");
  if (config->query_offset != qk_config->offset)
    return fail(MI_ERR_SHAPE, "decode step: the attention's query_offset must be the transform's offset");
  // FlashDecode over the cache prefix that ends with the new token, planned
  // with the library's default split (as for one decode token without a
  // tuned table), whatever mi_tune_flash_decode recorded.
  mi_tensor key = *key_cache, val = *value_cache;
  key.shape[0] = val.shape[0] = (int64_t)qk_config->offset + 1;
  AttnPlan p;
  if ((st = plan_attention(batch->ctx, q, &key, &val, config, MI_ATTN_DECODE_SPLIT_KV, 0, 0, false,
                           out, &p)) != MI_OK)
    return st;
  const bool fused = p.family == Family::Rows && p.D == 128 && p.waves == 8 &&
                     vector_friendly(*k, 8) && vector_friendly(*value, 8) &&
                     vector_friendly(*key_cache, 8) && vector_friendly(*value_cache, 8) &&
                     reinterpret_cast<uintptr_t>(q_weight->data) % 16 == 0 &&
                     reinterpret_cast<uintptr_t>(k_weight->data) % 16 == 0;
  if (!fused) {
    // The same work as the three calls, in their order.
    void *q_rot = nullptr;
    const uint64_t q_bytes = (uint64_t)q->shape[1] * q->shape[2] * sizeof(uint16_t);
    if ((st = scratch_alloc(batch, q_bytes, &q_rot)) != MI_OK) return st;
    mi_tensor qr{};
    qr.data = q_rot, qr.dtype = MI_F16, qr.rank = 3;
    qr.shape[0] = 1, qr.shape[1] = q->shape[1], qr.shape[2] = q->shape[2];
    qr.stride[0] = q->shape[1] * q->shape[2], qr.stride[1] = q->shape[2], qr.stride[2] = 1;
    st = mi_qk_norm_rope_cache_value(batch, q, k, value, q_weight, k_weight, key_cache, value_cache,
                                     qk_config, &qr);
    if (st == MI_OK)
      st = run_attention(batch, &qr, &key, &val, config, MI_ATTN_FLASH_DECODE, 0, 0, false, out);
    // In-order execution makes the range reusable by later work of the batch.
    scratch_free(batch->ctx, q_rot);
    return st;
  }
  const float scale = 1.0f / std::sqrt((float)p.D);
  kernels::RowsParams rp{};
  rp.q = static_cast<const uint16_t *>(q->data), rp.q_tok = q->stride[0], rp.q_head = q->stride[1];
  rp.k = static_cast<const uint16_t *>(key.data), rp.k_pos = key.stride[0], rp.k_head = key.stride[1];
  rp.v = static_cast<const uint16_t *>(val.data), rp.v_pos = val.stride[0], rp.v_head = val.stride[1];
  rp.out = static_cast<uint16_t *>(out->data), rp.o_tok = out->stride[0], rp.o_head = out->stride[1];
  rp.batch = 1, rp.tokens = 1, rp.q_heads = p.Hq, rp.kv_heads = p.Hkv;
  rp.kv_length = p.L, rp.causal = config->causal != 0, rp.query_offset = config->query_offset;
  rp.scale_log2 = scale * 1.4426950408889634f;
  rp.step_k = qp.k, rp.step_k_head = qp.k_head;
  rp.step_v = static_cast<const uint16_t *>(value->data), rp.step_v_head = value->stride[1];
  rp.step_qw = qp.q_weight, rp.step_kw = qp.k_weight;
  rp.step_kc = static_cast<uint16_t *>(key_cache->data);
  rp.step_vc = static_cast<uint16_t *>(value_cache->data);
  rp.step_theta = qp.theta, rp.step_eps = qp.epsilon;
  p.kernel = "attn_decode_step";
  return run_rows(batch, p, rp);
}

}  // extern "C"
