/*
 * read_probe.h - the streaming-read probe, a measurement instrument of the
 * benchmark (libsmx_probe.so).  Not part of the decode path's C ABI
 * (include/smx.h) and not loaded by it; no counterpart in the reference.
 */
#ifndef SMX_READ_PROBE_H
#define SMX_READ_PROBE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SMX_PROBE_ABI_VERSION 1
#define SMX_PROBE_EINVAL 10001 /* an argument failed validation */

int32_t smx_probe_abi_version(void);

/*
 * Reads `bytes` (a multiple of 16) from src once with 16-byte loads,
 * loads_per_lane (1, 2, 4, 8 or 16) of them per lane all in flight, and
 * writes one uint32 per wave into sink: the XOR of every 32-bit word that
 * wave read.  Workgroups of 4 waves; with L = loads_per_lane, wave w of
 * workgroup b reads the 16-byte words b * 256 * L + i * 256 + 64 * w + lane
 * (i < L, lane < 64), an index past the end reading the last word.  Its
 * time is the HBM ceiling of any kernel that moves the same bytes in one
 * launch.  sink_size must equal smx_read_probe_sink_size(bytes,
 * loads_per_lane) (-1 for invalid arguments); src 16-byte and sink 4-byte
 * aligned.  Returns 0, SMX_PROBE_EINVAL or a hipError_t value.
 */
int64_t smx_read_probe_sink_size(int64_t bytes, int32_t loads_per_lane);
int smx_read_probe(void* stream, const void* src, int64_t bytes, uint32_t* sink,
                   int64_t sink_size, int32_t loads_per_lane);

#ifdef __cplusplus
}
#endif

#endif /* SMX_READ_PROBE_H */
