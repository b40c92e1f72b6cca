/* Measurement probes of the MI355X PowerSparse build (libpowersparse_probes.so).
 *
 * Not part of the product ABI (include/powersparse_hip.h) and not called by
 * the operators or the preprocessing: these kernels measure the hardware the
 * operators run against (streaming bandwidth, random row-gather throughput,
 * row-update rates, the workgroup-to-XCD dealing) and calibrate the
 * rocprofv3 traffic counters. None has a counterpart in the reference.
 * Same conventions as the product ABI: int status (PS_OK / PS_ERR_*), message
 * in ps_last_error(), opaque streams.
 */
#ifndef POWERSPARSE_PROBES_H
#define POWERSPARSE_PROBES_H

#include <stddef.h>
#include <stdint.h>

#include "powersparse_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Streaming copy of `count` floats with 128-bit loads and stores (a plain
 * kernel, never a DMA engine): the reference point for HBM bandwidth and for
 * scaling the FETCH_SIZE / WRITE_SIZE counters. No reference counterpart. */
int ps_copy_f32_async(float* dst, const float* src, size_t count, ps_stream_t stream);

/* Measurement probe for the operators' row gathers: gathers `n` rows of a
 * rows x row_floats FP32 table (row_floats 32 or 128) at indices hash(seed, i)
 * mod rows, uniformly random, with 128-bit loads and 16 rows in flight per
 * lane, and writes a checksum to out[0]. Its throughput for a given table size
 * is the gather ceiling the SpMM / SDDMM kernels work against. No reference
 * counterpart. */
/* Records in out[b] the XCD (XCC) that runs workgroup b of a launch of
 * `workgroups` workgroups, read from the hardware's XCC_ID register. The
 * operators' workgroup -> task mapping (task_chunk) assumes the hardware's
 * round robin: workgroup b on XCD (x0 + b) mod 8 within a launch, x0 being
 * where the previous dispatch's dealing stopped (0 in a fresh process). No
 * reference counterpart. */
int ps_probe_xcc_ids_async(int* out, int workgroups, ps_stream_t stream);

/* Measurement probe for the operators' C-row writes: `n` updates of 128-byte
 * rows of C (rows x 32 floats) at rows hash(seed, i) mod rows. mode 0: plain
 * 128-bit stores; 1: float atomics with each of 8 lanes adding its own four
 * consecutive floats one by one (the lanes of one instruction 16 bytes apart);
 * 2: float atomics, 8 lanes adding 8 consecutive floats per instruction; 3:
 * float atomics, 32 lanes adding a whole row per instruction. Rows per second
 * by mode is the cost model of the SpMM kernel's atomic row writes. No
 * reference counterpart. */
int ps_probe_row_update_async(float* C, int rows, long long n, int mode, uint64_t seed,
                              ps_stream_t stream);

int ps_probe_gather_async(const float* table, int rows, int row_floats, long long n,
                          uint64_t seed, float* out, ps_stream_t stream);

#ifdef __cplusplus
}  /* extern "C" */
#endif

#endif /* POWERSPARSE_PROBES_H */
