/*
 * qf_probe.h -- calibration and comparison kernels for the roofline figures
 * (no counterpart in the reference; they are measurement infrastructure, not
 * on the hot path).
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
 *   qf_launch_probe a kernel of `workgroups` x `threads` threads (the
 *                   launch shape of a decode call) whose only work is
 *                   `round_trips` dependent memory round trips: 0 returns at
 *                   once (the cost of a graph node), 1 has every thread load
 *                   16 bytes of `src` (thread t of workgroup w reads bytes
 *                   16 * (w * threads + t), wrapped into `bytes`) and every
 *                   wave write the XOR to sink[(w * threads + t) / 64], 2
 *                   first reads index[0] (int64, on the device) and offsets
 *                   every load by that many 16-byte units, as a decode split
 *                   waits for kv_last before its first tile.  `sink` holds
 *                   workgroups * threads / 64 uint32.  The bench reports the
 *                   graph-replayed per-launch times as the floor a decode
 *                   launch of that shape cannot go under.
 *
 *   qf_decode_split_valu  the decode split launch of qf_decode_split
 *                   (qf_attn.h) computed with VALU dot products instead of
 *                   GQA-packed MFMA tiles: lane = key for q.k
 *                   (v_dot2_f32_f16), per-query wave reductions, lane = dim
 *                   pair for p.V.  Same partials (acc, m, l), so
 *                   qf_decode_combine merges them.  G must be 7, D 64, no
 *                   bias.  It exists so the MFMA packing decision can be
 *                   re-measured (bench.py --only valu); nothing calls it on
 *                   the hot path.
 *
 * Same conventions as qf_attn.h: device pointers, `stream` as void*, int
 * status, no allocation.  `src` and `bytes` must be 16-byte aligned;
 * 1 <= workgroups <= 65535; qf_launch_probe: threads a multiple of 64 in
 * [64, 1024], round_trips in 0..2 (src, sink and bytes unused at 0).
 */
#ifndef QF_PROBE_H
#define QF_PROBE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

int qf_stream_read(const void* src, int64_t bytes, uint32_t* sink, int workgroups, void* stream);
int qf_launch_probe(const void* src, int64_t bytes, const int64_t* index, uint32_t* sink,
                    int workgroups, int threads, int round_trips, void* stream);
int qf_decode_split_valu(const void* q, int64_t q_sb, int64_t q_sh, int64_t q_sg,
                         const void* k, int64_t k_sb, int64_t k_sh, int64_t k_sn,
                         const void* v, int64_t v_sb, int64_t v_sh, int64_t v_sn,
                         const int64_t* kv_last, int64_t kv_last_sb,
                         float* acc, float* m, float* l, int splits,
                         int B, int KVH, int G, int D, int cap, float scale, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* QF_PROBE_H */
