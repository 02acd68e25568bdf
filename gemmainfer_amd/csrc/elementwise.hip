// Companion kernels the drop-in module must export next to the MoE path:
// final-logit softcap, Gemma RMSNorm and rotate-half RoPE (gfx950).
//
// Reference behaviour restated (paths relative to the GemmaInfer repo):
//   softcap  csrc/softcapping.cu:7-19     x <- cap * tanh(x / cap)
//   rmsnorm  csrc/rmsnorm.cu:16-73         fp32 mean of squares, rsqrt(. + eps),
//                                          times weight or (1 + weight)
//   rope     csrc/rmsnorm.cu:116-164       x1' = x1 c1 - x2 s1, x2' = x2 c2 + x1 s2

#include "../../include/gemmainfer_amd.h"
#include "gi_common.h"
#include "gi_internal.h"

namespace gi {

namespace {

template <typename T>
__device__ __forceinline__ float ld(const T* p, int64_t i);
template <>
__device__ __forceinline__ float ld<uint16_t>(const uint16_t* p, int64_t i) {
  return bf16_to_f32(p[i]);
}
template <>
__device__ __forceinline__ float ld<_Float16>(const _Float16* p, int64_t i) {
  return (float)p[i];
}
template <>
__device__ __forceinline__ float ld<float>(const float* p, int64_t i) {
  return p[i];
}

__device__ __forceinline__ void st(uint16_t* p, int64_t i, float v) { p[i] = f32_to_bf16(v); }
__device__ __forceinline__ void st(_Float16* p, int64_t i, float v) { p[i] = (_Float16)v; }
__device__ __forceinline__ void st(float* p, int64_t i, float v) { p[i] = v; }

template <typename T>
__global__ __launch_bounds__(256) void softcap_kernel(T* x, int64_t n, float cap, float inv_cap) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    st(x, i, tanhf(ld(x, i) * inv_cap) * cap);
}

template <typename T>
__global__ __launch_bounds__(256) void rmsnorm_kernel(const T* in, const T* w, T* out, int hidden,
                                                      float eps, int unit_offset) {
  __shared__ float partial[4];
  const int64_t row = blockIdx.x;
  const T* x = in + row * hidden;
  T* y = out + row * hidden;
  float ss = 0.f;
  for (int i = threadIdx.x; i < hidden; i += blockDim.x) {
    const float v = ld(x, i);
    ss += v * v;
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) ss += __shfl_xor(ss, off, kWave);
  if ((threadIdx.x & 63) == 0) partial[threadIdx.x >> 6] = ss;
  __syncthreads();
  const float total = partial[0] + partial[1] + partial[2] + partial[3];
  const float r = rsqrtf(total / (float)hidden + eps);
  for (int i = threadIdx.x; i < hidden; i += blockDim.x) {
    float v = ld(x, i) * r;
    if (w) {
      const float wv = ld(w, i);
      v *= unit_offset ? 1.f + wv : wv;
    }
    st(y, i, v);
  }
}

template <typename T>
__global__ __launch_bounds__(256) void rope_kernel(T* q, T* k, const T* cs, const T* sn,
                                                   const int64_t* pos, int S, int Hq, int Hk,
                                                   int D, int64_t q_sb, int64_t q_sh,
                                                   int64_t q_ss, int64_t k_sb, int64_t k_sh,
                                                   int64_t k_ss) {
  const int bs = blockIdx.x, head = blockIdx.y;
  const int half = D >> 1;
  const int b = bs / S, s = bs - b * S;
  const int64_t p = pos[bs];
  T* base;
  if (head < Hq) base = q + b * q_sb + head * q_sh + s * q_ss;
  else base = k + b * k_sb + (head - Hq) * k_sh + s * k_ss;
  for (int d = threadIdx.x; d < half; d += blockDim.x) {
    const float c1 = ld(cs, p * D + d), s1 = ld(sn, p * D + d);
    const float c2 = ld(cs, p * D + d + half), s2 = ld(sn, p * D + d + half);
    const float x1 = ld(base, d), x2 = ld(base, d + half);
    st(base, d, x1 * c1 - x2 * s1);
    st(base, d + half, x2 * c2 + x1 * s2);
  }
}

int check_dtype(int dt, const char* who) {
  if (dt != GI_DTYPE_BF16 && dt != GI_DTYPE_FP16 && dt != GI_DTYPE_FP32)
    return fail(GI_ERR_UNSUPPORTED, std::string(who) + ": dtype must be bf16, fp16 or fp32");
  return GI_OK;
}

int after_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? GI_OK : hip_fail(e, what);
}

}  // namespace

int launch_softcap(void* x, int dtype, int64_t n, float cap, hipStream_t stream) {
  int st = check_dtype(dtype, "softcap");
  if (st != GI_OK) return st;
  if (n < 0 || !(cap != 0.f)) return fail(GI_ERR_INVALID_ARG, "softcap: n >= 0 and cap != 0 required");
  if (n == 0) return GI_OK;
  if (!x) return fail(GI_ERR_INVALID_ARG, "softcap: null pointer");
  const int64_t want = (n + 255) / 256;
  const int blocks = (int)(want < 65536 ? want : 65536);
  const float inv = 1.0f / cap;
  if (dtype == GI_DTYPE_BF16)
    hipLaunchKernelGGL(softcap_kernel<uint16_t>, dim3(blocks), dim3(256), 0, stream, (uint16_t*)x, n, cap, inv);
  else if (dtype == GI_DTYPE_FP16)
    hipLaunchKernelGGL(softcap_kernel<_Float16>, dim3(blocks), dim3(256), 0, stream, (_Float16*)x, n, cap, inv);
  else
    hipLaunchKernelGGL(softcap_kernel<float>, dim3(blocks), dim3(256), 0, stream, (float*)x, n, cap, inv);
  return after_launch("softcap launch");
}

int launch_rmsnorm(const void* in, const void* weight, void* out, int dtype, int64_t rows,
                   int hidden, float eps, int add_unit_offset, hipStream_t stream) {
  int st = check_dtype(dtype, "rmsnorm");
  if (st != GI_OK) return st;
  if (rows < 0 || hidden <= 0) return fail(GI_ERR_INVALID_ARG, "rmsnorm: rows >= 0, hidden > 0 required");
  if (rows > 0x7fffffff) return fail(GI_ERR_UNSUPPORTED, "rmsnorm: too many rows");
  if (rows == 0) return GI_OK;
  if (!in || !out) return fail(GI_ERR_INVALID_ARG, "rmsnorm: null pointer");
  const dim3 grid((unsigned)rows);
  if (dtype == GI_DTYPE_BF16)
    hipLaunchKernelGGL(rmsnorm_kernel<uint16_t>, grid, dim3(256), 0, stream, (const uint16_t*)in,
                       (const uint16_t*)weight, (uint16_t*)out, hidden, eps, add_unit_offset);
  else if (dtype == GI_DTYPE_FP16)
    hipLaunchKernelGGL(rmsnorm_kernel<_Float16>, grid, dim3(256), 0, stream, (const _Float16*)in,
                       (const _Float16*)weight, (_Float16*)out, hidden, eps, add_unit_offset);
  else
    hipLaunchKernelGGL(rmsnorm_kernel<float>, grid, dim3(256), 0, stream, (const float*)in,
                       (const float*)weight, (float*)out, hidden, eps, add_unit_offset);
  return after_launch("rmsnorm launch");
}

int launch_rope(void* q, void* k, const void* cos_t, const void* sin_t, const int64_t* pos,
                int dtype, int B, int Hq, int Hk, int S, int D, const int64_t* qs,
                const int64_t* ks, hipStream_t stream) {
  int st = check_dtype(dtype, "rope");
  if (st != GI_OK) return st;
  if (B < 0 || Hq < 0 || Hk < 0 || S < 0 || D <= 0 || (D & 1))
    return fail(GI_ERR_INVALID_ARG, "rope: bad shape (D must be even and positive)");
  if (!k) Hk = 0;
  if (B == 0 || S == 0 || Hq + Hk == 0) return GI_OK;
  if (!q || !cos_t || !sin_t || !pos) return fail(GI_ERR_INVALID_ARG, "rope: null pointer");
  const dim3 grid((unsigned)(B * S), (unsigned)(Hq + Hk));
  const int threads = (D / 2) < 256 ? ((D / 2 + 63) / 64) * 64 : 256;
#define GI_ROPE(T)                                                                            \
  hipLaunchKernelGGL(rope_kernel<T>, grid, dim3(threads), 0, stream, (T*)q, (T*)k,          \
                     (const T*)cos_t, (const T*)sin_t, pos, S, Hq, Hk, D, qs[0], qs[1], qs[2], \
                     ks[0], ks[1], ks[2])
  if (dtype == GI_DTYPE_BF16) GI_ROPE(uint16_t);
  else if (dtype == GI_DTYPE_FP16) GI_ROPE(_Float16);
  else GI_ROPE(float);
#undef GI_ROPE
  return after_launch("rope launch");
}

}  // namespace gi
