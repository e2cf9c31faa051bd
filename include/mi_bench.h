/*
 * mi_bench.h — seeded input generation for the attention benchmark harness.
 *
 * Replaces the input synthesis of `metal-infer-bench attention`
 * (crates/metal-infer-cli/src/bin/bench.rs:973-984), which fills Q/K/V with
 * fixed modular patterns; this harness uses the seeded N(0,1) stream the
 * BASELINE configurations specify instead. Not part of the attention ABI.
 */
#ifndef MI_BENCH_H
#define MI_BENCH_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* n values of the seeded stream: XorShift64 (crates/metal-infer-models/src/
 * qwen3.rs:1011-1034; seed 0 -> 0x9E3779B97F4A7C15) feeding Box-Muller
 * z = sqrt(-2 ln(1 - u1)) cos(2 pi u2), two draws per value, rounded
 * f64 -> f32 -> f16 (RNE); written as f16 bits in stream order. `threads`
 * workers split the stream by GF(2) jump-ahead; output is independent of
 * the thread count. */
void mi_bench_fill_normal_f16(uint64_t seed, uint16_t *out, size_t n,
                              int32_t threads);
/* lo + floor(u * (hi - lo + 1)) for n sequential draws of the stream. */
void mi_bench_fill_uniform_u32(uint64_t seed, uint32_t lo, uint32_t hi,
                               uint32_t *out, size_t n);

#ifdef __cplusplus
}
#endif

#endif
