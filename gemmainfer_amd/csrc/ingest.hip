// Checkpoint ingest for W4A16 linears (gfx950): compressed-tensors stores a
// linear as weight_packed int32 [N, K/8] (8 int4 codes of one output row per
// word, along K) and weight_scale [N, K/gs]; the kernels here read the
// reference's layout, packed [K/8, N] and scales [K/gs, N] (bf16).  The
// reference converts with `t.t()` and a copy into its preallocated buffers,
// writing gate_proj / up_proj of an expert into columns [0, I) / [I, 2I) of
// gate_up (weights.py:100-159).  This is the same transposition as one tiled
// device pass per tensor: 64 x 64 tiles through LDS, so both the read of a
// source row and the write of a destination row are contiguous across a wave.
// Words are moved unchanged; scales are converted to bf16 with round to
// nearest even (what `.to(dtype=torch.bfloat16)` does).
#include "../../include/gemmainfer_amd.h"
#include "gi_common.h"
#include "gi_internal.h"

namespace gi {

namespace {

constexpr int kTile = 64;

template <typename T>
__device__ __forceinline__ float scale_to_f32(T v);
template <>
__device__ __forceinline__ float scale_to_f32<uint16_t>(uint16_t v) { return bf16_to_f32(v); }
template <>
__device__ __forceinline__ float scale_to_f32<_Float16>(_Float16 v) { return (float)v; }
template <>
__device__ __forceinline__ float scale_to_f32<float>(float v) { return v; }

// out[b][c * ld + r] = conv(in[b][r * cols + c]) for r < rows, c < cols and
// b = blockIdx.z (matrix b of a batch at in + b * in_stride, out + b * out_stride).
template <typename Tin, typename Tout, bool kToBf16>
__global__ __launch_bounds__(256) void transpose_kernel(const Tin* in, Tout* out, int rows, int cols,
                                                         int64_t ld, int64_t in_stride, int64_t out_stride) {
  __shared__ Tout tile[kTile][kTile + 1];
  const int tx = threadIdx.x & (kTile - 1), ty = threadIdx.x >> 6;
  const int c0 = blockIdx.x * kTile, r0 = blockIdx.y * kTile;
  in += (int64_t)blockIdx.z * in_stride;
  out += (int64_t)blockIdx.z * out_stride;
#pragma unroll
  for (int i = 0; i < kTile / 4; ++i) {
    const int r = r0 + ty + 4 * i, c = c0 + tx;
    if (r < rows && c < cols) {
      const Tin v = in[(int64_t)r * cols + c];
      if constexpr (kToBf16)
        tile[ty + 4 * i][tx] = f32_to_bf16(scale_to_f32<Tin>(v));
      else
        tile[ty + 4 * i][tx] = (Tout)v;
    }
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < kTile / 4; ++i) {
    const int c = c0 + ty + 4 * i, r = r0 + tx;
    if (r < rows && c < cols) out[(int64_t)c * ld + r] = tile[tx][ty + 4 * i];
  }
}

template <typename Tin, typename Tout, bool kToBf16>
void launch_transpose(const Tin* in, Tout* out, int rows, int cols, int64_t ld, int batch, int64_t in_stride,
                      int64_t out_stride, hipStream_t stream) {
  const dim3 grid((unsigned)((cols + kTile - 1) / kTile), (unsigned)((rows + kTile - 1) / kTile), (unsigned)batch);
  hipLaunchKernelGGL((transpose_kernel<Tin, Tout, kToBf16>), grid, dim3(256), 0, stream, in, out, rows,
                     cols, ld, in_stride, out_stride);
}

}  // namespace

int launch_w4a16_ingest(const int32_t* weight_packed, const void* weight_scale, int scale_dtype, int N,
                        int K, int n_groups, int32_t* packed_out, void* scales_out, int64_t ld_out,
                        hipStream_t stream) {
  return launch_w4a16_ingest_batched(weight_packed, weight_scale, scale_dtype, 1, N, K, n_groups, 0, 0, packed_out,
                                     scales_out, ld_out, 0, 0, stream);
}

int launch_w4a16_ingest_batched(const int32_t* weight_packed, const void* weight_scale, int scale_dtype, int batch,
                                int N, int K, int n_groups, int64_t src_stride_packed, int64_t src_stride_scale,
                                int32_t* packed_out, void* scales_out, int64_t ld_out, int64_t dst_stride_packed,
                                int64_t dst_stride_scale, hipStream_t stream) {
  if (batch < 0 || batch > 65535) return fail(GI_ERR_INVALID_ARG, "w4a16_ingest: batch must be in [0, 65535]");
  if (batch == 0) return GI_OK;
  if (N < 0 || K < 0 || n_groups < 0 || K % 8 != 0)
    return fail(GI_ERR_INVALID_ARG, "w4a16_ingest: N, K, n_groups >= 0 and K % 8 == 0 required");
  if (ld_out < N) return fail(GI_ERR_INVALID_ARG, "w4a16_ingest: ld_out must be >= N");
  if ((int64_t)N > 65535 * (int64_t)kTile || (int64_t)(K / 8) > 0x7fffffff / kTile)
    return fail(GI_ERR_UNSUPPORTED, "w4a16_ingest: too many rows");
  if (scale_dtype != GI_DTYPE_BF16 && scale_dtype != GI_DTYPE_FP16 && scale_dtype != GI_DTYPE_FP32)
    return fail(GI_ERR_UNSUPPORTED, "w4a16_ingest: weight_scale must be bf16, fp16 or fp32");
  if (N == 0) return GI_OK;
  const int kp = K / 8;
  if (kp > 0 && (!weight_packed || !packed_out)) return fail(GI_ERR_INVALID_ARG, "w4a16_ingest: null packed pointer");
  if (n_groups > 0 && (!weight_scale || !scales_out))
    return fail(GI_ERR_INVALID_ARG, "w4a16_ingest: null scale pointer");
  if (kp > 0) {
    launch_transpose<int32_t, int32_t, false>(weight_packed, packed_out, N, kp, ld_out, batch, src_stride_packed,
                                              dst_stride_packed, stream);
  }
  if (n_groups > 0) {
    uint16_t* so = (uint16_t*)scales_out;
    if (scale_dtype == GI_DTYPE_BF16)
      launch_transpose<uint16_t, uint16_t, true>((const uint16_t*)weight_scale, so, N, n_groups, ld_out, batch,
                                                 src_stride_scale, dst_stride_scale, stream);
    else if (scale_dtype == GI_DTYPE_FP16)
      launch_transpose<_Float16, uint16_t, true>((const _Float16*)weight_scale, so, N, n_groups, ld_out, batch,
                                                 src_stride_scale, dst_stride_scale, stream);
    else
      launch_transpose<float, uint16_t, true>((const float*)weight_scale, so, N, n_groups, ld_out, batch,
                                              src_stride_scale, dst_stride_scale, stream);
  }
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? GI_OK : hip_fail(e, "w4a16_ingest launch");
}

}  // namespace gi
