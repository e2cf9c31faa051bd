/*
 * mi_probe.h — calibration kernels for the benchmark (libmi_probe.so).
 *
 * Not part of the attention ABI and with no counterpart in the reference:
 * these kernels measure the floors under the single-sequence decode (c2) and
 * the achievable streaming read rate under the batched decode (c4), so that a
 * kernel's time can be set against what its launch, its bytes and its
 * split-K exchange cost without the attention arithmetic. Every call
 * enqueues one kernel on `stream` (a hipStream_t) and returns the hipError_t
 * of the launch (0 on success). All pointers are device pointers.
 */
#ifndef MI_PROBE_H
#define MI_PROBE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* An empty kernel on a grid of (grid_x, grid_y) workgroups of `threads`
 * threads (<= 1024): the launch floor of a grid. */
int32_t mi_probe_empty(void *stream, uint32_t grid_x, uint32_t grid_y, uint32_t threads);

/* Streaming read: `workgroups` workgroups of 256 threads each read their own
 * contiguous `bytes_per_workgroup` (a multiple of 16) of `src` with 16-byte
 * non-temporal loads, eight in flight per lane, and write one word per wave
 * to sink[workgroup * 4 + wave] (so the loads are not dead). Reads
 * workgroups * bytes_per_workgroup bytes. */
int32_t mi_probe_read(void *stream, const void *src, uint64_t bytes_per_workgroup,
                      uint32_t workgroups, uint32_t *sink);

/* The c2 decode's memory and exchange pattern without its arithmetic: one
 * 512-thread workgroup per (key split of `block_keys` keys, KV head), over
 * head-major K / V caches (`head_stride` halves between KV heads, 128 halves
 * per key row) of `keys` visible keys, each workgroup loading its K and V
 * rows exactly as the attention rows kernel at head_dim 128 does (one batch
 * of 16-byte loads per lane), folding them into per-wave words and meeting at
 * an LDS reduction.
 *  - publish == 0: each workgroup writes one word to out_words[unit * splits
 *    + split] and ends (the data phase alone);
 *  - publish != 0: each workgroup stores a (max, sum, acc[128]) partial for
 *    each of the `group` query heads of its KV head into `partial` (unit x
 *    split x group x 130 floats) with device-scope stores, waits for them,
 *    counts its arrival on counters[32 * kv head] with an agent-scope
 *    atomic add (one 128-byte line per counter, as the attention kernels),
 *    and the last split to arrive acquires, resets the counter to zero and
 *    merges every split's partial (one load per split per output element)
 *    into out_f16 [group x 128 halves per KV head] — the attention kernel's
 *    split protocol.
 * `counters` holds 32 * kv_heads zeroed words (left zeroed). group <= 8. */
int32_t mi_probe_split_decode(void *stream, const uint16_t *k, const uint16_t *v,
                              uint64_t head_stride, uint32_t kv_heads, uint32_t group,
                              uint32_t keys, uint32_t block_keys, int32_t publish,
                              float *partial, uint32_t *counters, uint32_t *out_words,
                              uint16_t *out_f16);

#ifdef __cplusplus
}
#endif

#endif
