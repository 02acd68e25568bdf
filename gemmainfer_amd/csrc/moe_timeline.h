// Phase stamps of the decode kernels, compiled in only with -DGI_TIMELINE
// (the measurement library libgemmainfer_amd_timeline.so): thread 0 keeps
// the constant 100 MHz clock (s_memrealtime) at each phase end in LDS, and
// the workgroup writes its kStamps words out at its end.  In the product
// library GI_STAMP expands to nothing.
#pragma once

#include "gi_common.h"

namespace gi {
namespace {

constexpr int kStamps = 32;  // words 0-23: clock stamps; 29 kernel id, 30 role, 31 index

#ifdef GI_TIMELINE
__shared__ unsigned long long tl_lds[kStamps];
__device__ __forceinline__ void tl_init() {
  if (threadIdx.x < kStamps) tl_lds[threadIdx.x] = 0ull;
}
__device__ __forceinline__ void tl_stamp(int i) {
  if (threadIdx.x == 0) tl_lds[i] = __builtin_amdgcn_s_memrealtime();
}
// the same from another thread (another wave's view)
__device__ __forceinline__ void tl_stamp_by(int i, int t) {
  if ((int)threadIdx.x == t) tl_lds[i] = __builtin_amdgcn_s_memrealtime();
}
__device__ __forceinline__ void tl_value(int i, unsigned long long v) {
  if (threadIdx.x == 0) tl_lds[i] = v;
}
__device__ __forceinline__ void tl_flush(unsigned long long* dst) {
  lds_barrier();
  if (dst && threadIdx.x < kStamps) dst[blockIdx.x * kStamps + threadIdx.x] = tl_lds[threadIdx.x];
}
#define GI_STAMP(i) tl_stamp(i)
#define GI_STAMP_BY(i, t) tl_stamp_by(i, t)
#else
#define GI_STAMP(i) ((void)0)
#define GI_STAMP_BY(i, t) ((void)0)
#endif

}  // namespace
}  // namespace gi
