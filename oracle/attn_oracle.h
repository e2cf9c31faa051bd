/*
 * CPU oracle for the causal GQA attention path — TEST INFRASTRUCTURE ONLY.
 *
 * This library is the checker, never the product. Only tests/, the graft
 * entry's smoke() and bench.py's cpu_baseline leg may load it. The product
 * path (libmi_attn.so) never links or calls it.
 *
 * Every function restates a piece of the reference (stratorys/metal-infer-rs,
 * paths relative to the reference root) and cites the lines it follows.
 * tests/test_oracle.py pins each function against checks that share none of
 * its code (numpy's IEEE conversions, torch float64 SDPA fixtures,
 * transformers' Qwen3 RMSNorm/RoPE, closed forms, invariants, brute force)
 * and plants plausible mistakes to show that the pins catch them.
 */
#ifndef MI_ATTN_ORACLE_H
#define MI_ATTN_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* IEEE-754 binary16 <-> binary32 with round-to-nearest-even.
 * Follows half::f16::from_f32 / to_f32 as used by
 * crates/metal-infer-core/src/context.rs:756-774 (upload) and
 * crates/metal-infer-core/src/tensor.rs:228-246 (readback). */
uint16_t orc_f32_to_f16(float value);
float orc_f16_to_f32(uint16_t bits);
void orc_f32_to_f16_array(const float *src, uint16_t *dst, size_t n);
void orc_f16_to_f32_array(const uint16_t *src, float *dst, size_t n);

/* XorShift64 (crates/metal-infer-models/src/qwen3.rs:1011-1034). */
uint64_t orc_xorshift_seed(uint64_t seed);
double orc_xorshift_next_f64(uint64_t *state);
/* Advance a XorShift64 state by `steps` draws in O(64^2 log steps). */
uint64_t orc_xorshift_jump(uint64_t state, uint64_t steps);

/* Seeded N(0,1) f16 values: u1,u2 from XorShift64, z = sqrt(-2 ln(1-u1)) *
 * cos(2 pi u2), rounded f64 -> f32 -> f16 (RNE). Two draws per value.
 * `threads` > 1 splits the stream with orc_xorshift_jump; the output is
 * bit-identical for every thread count. */
void orc_fill_normal_f16(uint64_t seed, uint16_t *out, size_t n, int threads);
/* Uniform integers lo + floor(u * (hi - lo + 1)), one draw each. */
void orc_fill_uniform_u32(uint64_t seed, uint32_t lo, uint32_t hi,
                          uint32_t *out, size_t n);

/* Restatement of attention_reference_f16
 * (crates/metal-infer-core/src/kernels/transformer.metal:1579-1612).
 *
 * Logical layouts: Q [T, Hq, D], K/V [L, Hkv, D] addressed through element
 * strides (so head-major caches are read in place). Rows selects which query
 * tokens to evaluate (NULL = all T, in order); the outputs are [n_rows, Hq, D]
 * contiguous. Any output pointer may be NULL.
 *   out_f16 : half(num / den), RNE           (the reference's output)
 *   out_f32 : num / den before rounding      (f32 pipeline, for error bounds)
 *   out_f64 : the same formula evaluated in f64 throughout
 * A row whose causal window is empty (L == 0) yields NaN like the kernel
 * (0/0). Returns 0, or -1 on invalid geometry. */
typedef struct orc_attention_args {
  const uint16_t *q;
  int64_t q_stride[3];
  const uint16_t *k;
  int64_t k_stride[3];
  const uint16_t *v;
  int64_t v_stride[3];
  uint32_t tokens;
  uint32_t q_heads;
  uint32_t kv_heads;
  uint32_t head_dim;
  uint32_t kv_length;
  uint32_t causal;
  uint32_t query_offset;
  const uint32_t *rows;
  uint32_t n_rows;
  uint16_t *out_f16;
  float *out_f32;
  double *out_f64;
  int threads;
} orc_attention_args;

int orc_attention(const orc_attention_args *args);

/* Restatement of qk_norm_rope_cache_f16
 * (transformer.metal:1533-1577): per-head RMSNorm with weight, then RoPE
 * (theta, position = offset + token) on (pair, pair + D/2). Query rows go to
 * q_out [T, Hq, D]; key rows to key_out [T, Hkv, D] (the caller scatters them
 * into the cache at `offset`). */
int orc_qk_norm_rope(const uint16_t *q, const uint16_t *k, const uint16_t *q_w,
                     const uint16_t *k_w, uint32_t tokens, uint32_t q_heads,
                     uint32_t kv_heads, uint32_t head_dim, uint32_t offset,
                     float theta, float epsilon, uint16_t *q_out,
                     uint16_t *key_out);

/* Restatement of rms_norm_f16 (transformer.metal:1318-1340) for `rows`
 * contiguous rows of `width`: scale = 1 / sqrt(sum(x^2) / width + epsilon)
 * with the squares summed in ascending order in f32, out = f16(x * scale *
 * w). out_f32 (optional) receives the unrounded values. */
int orc_rms_norm(const uint16_t *x, const uint16_t *w, uint64_t rows,
                 uint32_t width, float epsilon, uint16_t *out, float *out_f32);

/* Restatement of rope_f16 (transformer.metal:1514-1531) on contiguous
 * [tokens, heads, head_dim]: pair (i, i + D/2) of token t rotated by
 * (t + offset) * theta^(-2i/D). */
int orc_rope(const uint16_t *x, uint32_t tokens, uint32_t heads,
             uint32_t head_dim, uint32_t offset, float theta, uint16_t *out);

/* Restatement of matmul_f16 (transformer.metal:70-93): out[i][j] =
 * f16(sum_k f32(x[i][k]) * f32(w[j][k])), k ascending, for contiguous x
 * [m, k] and w [n, k]. out_f32 (optional) receives the unrounded sums.
 * Rows of out are spread over `threads` OpenMP threads (0 = default). */
int orc_matmul(const uint16_t *x, const uint16_t *w, uint32_t m, uint32_t n,
               uint32_t k, uint16_t *out, float *out_f32, int threads);

#ifdef __cplusplus
}
#endif

#endif
