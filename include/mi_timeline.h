/*
 * mi_timeline.h — per-workgroup timestamps of the timeline build
 * (libmi_timeline: libmi_attn_timeline.so, the same sources as
 * libmi_attn.so compiled with MI_TIMELINE).
 *
 * Not part of the attention ABI and with no counterpart in the reference:
 * a measurement aid. It exports everything libmi_attn.so does, plus the
 * readers below. Each kernel launch overwrites the rows of the workgroups it
 * runs; a row is kTimelineFields = 8 u64 words, row i for the workgroup of
 * linear id i (at most 8192 rows). Times are s_memrealtime ticks (100 MHz,
 * one clock for the whole device). Words 0 and 1 of every row: start time,
 * (HW_ID << 8) | XCC_ID.
 *
 * Stream-K batched decode rows (attn_decode_stream_kernel):
 *   2 end time; 3 start of its first piece (after the length prefix sums);
 *   4 pieces | key tiles << 16; 5 ticks spent in piece epilogues (wave merge
 *   and output or partial stores).
 * Prefill rows (attn_prefill_kernel):
 *   2 end time; 3 first K/V tile ready; 4 key loop done; 5 split partial
 *   published (0 if none); 6 arrival counted (0 if none);
 *   7 row tile | split << 16 | first key tile << 20 | end key tile << 40 |
 *   (1 << 63 if it merged the row tile's splits).
 *
 * Rows kernel (attn_rows_kernel: single-sequence decode and the other
 * split-K kinds):
 *   2 end time; 3 the first batch of K/V rows (and the query rows) loaded
 *   (this build waits for them there, before the arithmetic); 4 key loop
 *   done; 5 split partial stored and complete (0 if none); 6 arrival counted
 *   (0 if none); 7 split | splits << 16 | (1 << 63 if it merged the unit's
 *   splits).
 *
 * Every reader copies `bytes` from the start of its kernel's row buffer to
 * the host buffer `dst` (synchronous) and returns the hipError_t (0 on
 * success).
 */
#ifndef MI_TIMELINE_H
#define MI_TIMELINE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

int32_t mi_timeline_read_rows(void *dst, uint64_t bytes);
int32_t mi_timeline_read_stream(void *dst, uint64_t bytes);
int32_t mi_timeline_read_prefill(void *dst, uint64_t bytes);

#ifdef __cplusplus
}
#endif

#endif
