/*
 * purin_probe.h -- ceiling probes for the resident CP kernel's roofline
 * (libpurin_probe.so).  Measurement only: no counterpart in the reference,
 * and not part of the projection ABI (purin_cp.h).  bench.py loads it.
 *
 * Both probes launch ``groups`` workgroups of 1024 threads with ``lds_bytes``
 * of dynamic LDS (the resident kernel's, for the same occupancy), ``reps``
 * times on ``stream``, and return the mean time per launch from HIP events on
 * that stream.  ``sink`` is a device buffer of at least 4096 bytes that the
 * kernels write only to keep their loads live.  Return 0, 1 for an invalid
 * argument, 2 for a HIP error.
 */
#ifndef PURIN_PROBE_H
#define PURIN_PROBE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* L2 -> CU chunk streams: wavefront w of every workgroup reads chunks
 * [w * wave_chunks, (w + 1) * wave_chunks) of ``buf`` (3072-byte chunks,
 * three 16-byte loads per lane each, ``unroll`` in {1, 2, 4} chunks in flight;
 * buf_bytes >= 16 * wave_chunks * 3072), ``iters`` times.  Bytes per launch:
 * groups * 16 * wave_chunks * 3072 * iters. */
int purin_probe_stream(void* stream, const void* buf, int64_t buf_bytes, int64_t wave_chunks,
                       int32_t iters, int32_t groups, int32_t lds_bytes, int32_t unroll,
                       int32_t reps, void* sink, int64_t sink_bytes, double* ms_per_launch);

/* LDS reads: every lane reads 16 bytes (ds_read_b128) at lane-contiguous,
 * bank-conflict-free addresses of a 64 KiB span, ``unroll`` in {1, 2, 4, 8}
 * reads per iteration, ``iters`` iterations (lds_bytes >= 65536).  Bytes per
 * launch: groups * 1024 * 16 * unroll * iters. */
int purin_probe_lds(void* stream, int32_t iters, int32_t groups, int32_t lds_bytes,
                    int32_t unroll, int32_t reps, void* sink, int64_t sink_bytes,
                    double* ms_per_launch);

#ifdef __cplusplus
}
#endif

#endif /* PURIN_PROBE_H */
