/* Measurement probes of libslimkv_probe.so: hardware ceilings that measured
 * kernel rates are read against.  Not part of the serving library
 * (libslimkv_hip.so) and without counterpart in the reference.  Return 0, or
 * a negative code with slimkv_probe_last_error() describing it. */
#ifndef SLIMKV_PROBE_H
#define SLIMKV_PROBE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

const char* slimkv_probe_last_error(void);

/* HBM read rate: a grid-stride stream of 16-byte loads over `bytes` of src
 * (16-byte aligned), `depth` (1, 2, 4, 8) loads in flight a thread,
 * waves_per_cu (multiple of 4 in [4, 64]) resident waves a CU, plain or
 * non-temporal loads; one folded word a thread to sink (at least
 * grid * 256 words, grid = CUs * waves_per_cu / 4). */
int slimkv_probe_stream_read(const void* src, int64_t bytes, uint32_t* sink, int64_t sink_words,
                             int32_t waves_per_cu, int32_t depth, int32_t non_temporal, void* stream);

/* HBM read rate of scattered chunks (the access pattern of rows read through
 * a block table): chunk i is `chunk_bytes` (a multiple of 16, at most 16384)
 * at src + ids[i] * stride_bytes + offset_bytes, i < count (ids int64 on the
 * device; a chunk that would end past `bytes` reads chunk 0 instead).  The
 * chunks' 16-byte pieces are dealt grid-stride over waves_per_cu resident
 * waves a CU (consecutive lanes, consecutive pieces), four loads in flight a
 * thread; one folded word a thread to sink (grid * 256 words).  Bytes read =
 * count * chunk_bytes. */
int slimkv_probe_gather_read(const void* src, int64_t bytes, const int64_t* ids, int64_t count, int64_t stride_bytes,
                             int64_t offset_bytes, int32_t chunk_bytes, uint32_t* sink, int64_t sink_words,
                             int32_t waves_per_cu, void* stream);

/* LDS read rate of a CU: workgroups_per_cu (1 or 2) workgroups of 256
 * threads a CU, each with 64 KB of LDS, read it `iters` x 16 times a lane,
 * `width` (8 or 16) bytes a read, conflict free; one word a thread to sink
 * (at least CUs * workgroups_per_cu * 256 words).  Bytes read =
 * CUs * workgroups_per_cu * 256 * iters * 16 * width. */
int slimkv_probe_lds_read(uint32_t* sink, int64_t sink_words, int32_t workgroups_per_cu, int32_t iters,
                          int32_t width, void* stream);

/* The per-launch floor: `workgroups` (1..65536) one-wave workgroups, each
 * storing one word to sink (at least `workgroups` words).  Timed as graph
 * replays of back-to-back launches it gives the cost of a launch and its
 * hand-off alone. */
int slimkv_probe_touch(uint32_t* sink, int64_t sink_words, int32_t workgroups, void* stream);

#ifdef __cplusplus
}
#endif

#endif
