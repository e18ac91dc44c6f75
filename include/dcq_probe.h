/*
 * dcq_probe.h — measurement aids exported by libdcq beside the operator ABI (include/dcq.h).
 *
 * No counterpart in the reference: DenseCore has no GPU path. These entry points exist so the
 * bench can state what the hardware itself allows at the workload's sizes, next to what the
 * operator achieves. They compute nothing the operator uses.
 */
#ifndef DCQ_PROBE_H
#define DCQ_PROBE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Reads `bytes` (a multiple of 16) from the device buffer `src` (16-byte aligned) with 16-byte
 * loads, `per_lane` (1, 2, 4, 8 or 16) loads in flight per lane, 256 threads per workgroup and
 * ceil(bytes / (4096 * per_lane)) workgroups, capped at max_workgroups when that is > 0 (the
 * workgroups then loop). Nothing is written except, with negligible probability, one word at
 * `sink` (a 4-byte aligned device word). Stream-ordered. Returns 0, or a negative DCQ_ERR_*
 * code for a bad argument (nothing launched) or a failed launch. */
int dcq_probe_stream_read(const void* src, size_t bytes, int per_lane, int max_workgroups, uint32_t* sink,
                          void* stream);

#ifdef __cplusplus
}
#endif
#endif /* DCQ_PROBE_H */
