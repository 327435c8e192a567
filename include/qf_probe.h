/*
 * qf_probe.h -- calibration kernel for the roofline figures (no counterpart
 * in the reference; it is measurement infrastructure, not on the hot path).
 *
 *   qf_stream_read  reads `bytes` bytes at `src` with 16-byte non-temporal
 *                   loads (the decode kernels' streaming flavor) spread over
 *                   `workgroups` workgroups (grid-stride) and writes one
 *                   uint32 per wave to `sink` (the XOR of what the wave
 *                   read), so the loads cannot be dropped.  `sink` holds
 *                   4 * workgroups uint32.  The bench times it to report the
 *                   HBM read rate this box reaches at a given size, beside
 *                   the decode kernels' rates.
 *
 * Same conventions as qf_attn.h: device pointers, `stream` as void*, int
 * status, no allocation.  `src` and `bytes` must be 16-byte aligned;
 * 1 <= workgroups <= 65535.
 */
#ifndef QF_PROBE_H
#define QF_PROBE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

int qf_stream_read(const void* src, int64_t bytes, uint32_t* sink, int workgroups, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* QF_PROBE_H */
