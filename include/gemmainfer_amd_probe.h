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
 * decode-kernel launch writes, per workgroup, 32 uint64 words into the next
 * slot of `buf` (device memory; slots of 1024 x 32 words, used in rotation,
 * bytes / 262144 of them; NULL stops the recording): words 0-23 are the
 * constant 100 MHz clock (s_memrealtime) at the ends of the kernel's phases
 * (zero for phases the workgroup skips), word 29 names the kernel (1: the
 * decode kernel, up to 8 rows per launch; 2: the one-token kernel), words 30
 * and 31 the workgroup's role and index.  The phase numbering of each kernel
 * is stated beside its stamps in the kernel source and in bench.py
 * (TIMELINE_PHASES).  The product library returns GI_ERR_UNSUPPORTED.     */
int gi_probe_decode_timeline(void* buf, size_t bytes);

#ifdef __cplusplus
}
#endif

#endif /* GEMMAINFER_AMD_PROBE_H */
