/*
 * gemmainfer_amd_probe.h -- measurement entry points of libgemmainfer_amd.so.
 *
 * No counterpart in the reference: these exist so that the MoE and linear
 * kernels' achieved HBM rates can be reported against a measured ceiling on
 * the same part and the same bytes, beside the 8 TB/s specification figure.
 * Same conventions as gemmainfer_amd.h (plain C, int status, the stream as
 * void*, asynchronous, no allocation).
 */
#ifndef GEMMAINFER_AMD_PROBE_H
#define GEMMAINFER_AMD_PROBE_H

#include <stddef.h>
#include <stdint.h>

#include "gemmainfer_amd.h"

#ifdef __cplusplus
extern "C" {
#endif

#define GI_PROBE_MAX_SEGMENTS 128

/* Pure read of n_seg device segments (seg_ptr / seg_bytes are host arrays;
 * each segment 16-byte aligned, a multiple of 16 bytes, below 2 GiB), one
 * launch: workgroups of 256 threads each read 256 * 16 * loads_per_thread
 * contiguous bytes of one segment (loads_per_thread in {2, 4, 8, 16, 32}),
 * every load issued before any use.  `sink` is a device word that is never
 * written in practice (it keeps the loads live).                            */
int gi_probe_stream_read(const void* const* seg_ptr, const uint64_t* seg_bytes, int n_seg,
                         int loads_per_thread, uint32_t* sink, void* stream);

/* Phase timeline of the decode kernel.  In a library built with the
 * timeline option (python -m gemmainfer_amd.build --timeline, which writes
 * libgemmainfer_amd_timeline.so beside the product library) every later
 * decode-kernel launch writes, per workgroup, 16 uint64 words into the next
 * slot of `buf` (device memory; slots of 1024 x 16 words, used in rotation,
 * bytes / 131072 of them; NULL stops the recording): words 0-9 are the
 * constant 100 MHz clock (s_memrealtime) at the ends of the kernel's phases
 * (0 start, 1 routing and tables, 2 x in LDS, 3 weight loads issued,
 * 4 gate/up items done, 5 activations staged, 6 down products, 7 sums over
 * the waves, 8 output or partial sums written, 9 end), words 14 and 15 the
 * workgroup's gate/up item and down block counts.  The product library
 * returns GI_ERR_UNSUPPORTED.                                              */
int gi_probe_decode_timeline(void* buf, size_t bytes);

#ifdef __cplusplus
}
#endif

#endif /* GEMMAINFER_AMD_PROBE_H */
