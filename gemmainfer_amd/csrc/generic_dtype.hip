// fp16 and fp32 activations for the two drop-in entry points: the reference
// dispatches bf16, fp16 and fp32 (csrc/marlin.cu:694-700 for the MoE,
// :764-770, :816-822, :831-842 for the linear).  bf16 runs the tuned kernels;
// these VALU kernels serve the other two dtypes with fp32 arithmetic and the
// reference's rounding points in the activation dtype T:
//   * the routing weights are cast to T (marlin.cu:634-636),
//   * the activation gelu_tanh(gate) * up is stored in T (:421-423),
//   * the output is rounded to T (the MoE adds to out: :583, one rounding
//     of old + the fixed-order fp32 sum of the slots here).
// Scales are in T like the activations (the reference's tensors share the
// model dtype).
//
// Dequantisation: nibble i of a packed word is the code of row 8pk + i; the
// low nibbles of the four bytes (w & 0x0f0f0f0f) are codes 0, 2, 4, 6 and
// the high ones (w >> 4 & 0x0f0f0f0f) codes 1, 3, 5, 7; v_cvt_f32_ubyte turns
// each byte into a float, and the sum x * (q - 8) is taken as
// sum x * q - 8 * sum x.
//
// Work split:
//   linear   workgroup of 256 threads = 64 output columns x 4 slices of the
//            packed rows, for up to 8 rows of A (grid y for more); the
//            slices are added in LDS in order.
//   MoE      two launches: gate/up per (slot, 32-column tile): 32 gate + 32
//            up columns x 4 slices of H, activation rounded to T into an fp32
//            buffer [S][I] in the workspace; then down + combine per
//            (64-column tile, token): every slot of the token, 4 slices of I,
//            old + sum over slots of w * y in slot order, one rounding.

#include "../../include/gemmainfer_amd.h"
#include "gi_common.h"
#include "gi_internal.h"

namespace gi {

namespace {

constexpr int kGT = 256;     // threads
constexpr int kGCols = 64;   // columns per workgroup
constexpr int kGSlices = kGT / kGCols;
constexpr int kGRows = 8;    // rows of A per linear workgroup

template <typename T>
__device__ __forceinline__ float ld(const T* p, size_t i);
template <>
__device__ __forceinline__ float ld<_Float16>(const _Float16* p, size_t i) {
  return (float)p[i];
}
template <>
__device__ __forceinline__ float ld<float>(const float* p, size_t i) {
  return p[i];
}
// round-to-nearest-even into T (v_cvt_f16_f32 rounds to nearest even)
template <typename T>
__device__ __forceinline__ float round_t(float v);
template <>
__device__ __forceinline__ float round_t<_Float16>(float v) {
  return (float)(_Float16)v;
}
template <>
__device__ __forceinline__ float round_t<float>(float v) {
  return v;
}
template <typename T>
__device__ __forceinline__ void st(T* p, size_t i, float v) {
  p[i] = (T)v;
}

// The 8 codes of a packed word as floats q (0..15).
__device__ __forceinline__ void codes8(uint32_t w, float (&q)[8]) {
  const uint32_t lo = w & 0x0f0f0f0fu, hi = (w >> 4) & 0x0f0f0f0fu;
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    q[2 * b] = (float)((lo >> (8 * b)) & 0xffu);  // v_cvt_f32_ubyte<b>
    q[2 * b + 1] = (float)((hi >> (8 * b)) & 0xffu);
  }
}

// sum_i a[i] * (q[i] - 8) of one packed row
__device__ __forceinline__ float dot8(const float (&a)[8], const float (&q)[8]) {
  float s = 0.f, sa = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    s = fmaf(a[i], q[i], s);
    sa += a[i];
  }
  return fmaf(-8.f, sa, s);
}

// ---------------------------------------------------------------------------
// linear: C[M, N] = A[M, K] @ dequant(B[K/8, N], scales[G, N]), optional softcap
// ---------------------------------------------------------------------------
struct GLinArgs {
  const void* A;
  const int32_t* B;
  const void* S;
  void* C;
  int M, K, N, G, gs;
  float cap;
};

template <typename T>
__global__ __launch_bounds__(kGT) void w4a16_generic_kernel(GLinArgs a) {
  __shared__ float red[kGSlices][kGRows][kGCols];
  const int tid = threadIdx.x, c = tid % kGCols, sl = tid / kGCols;
  const int col = blockIdx.x * kGCols + c;
  const int m0 = blockIdx.y * kGRows;
  const int rows = min(kGRows, a.M - m0);
  const T* A = (const T*)a.A;
  const T* S = (const T*)a.S;
  const int P = a.K / 8;
  const int Pv = min(P, a.G * a.gs / 8);  // packed rows past the last scale group are dropped
  const int per = (Pv + kGSlices - 1) / kGSlices;
  const int p0 = sl * per, p1 = min(Pv, p0 + per);
  float acc[kGRows];
#pragma unroll
  for (int r = 0; r < kGRows; ++r) acc[r] = 0.f;
  if (col < a.N) {
    for (int pk = p0; pk < p1; ++pk) {
      float q[8];
      codes8((uint32_t)a.B[(size_t)pk * a.N + col], q);
      const float s = ld(S, (size_t)(pk * 8 / a.gs) * a.N + col);
#pragma unroll
      for (int r = 0; r < kGRows; ++r) {
        if (r < rows) {
          float x[8];
#pragma unroll
          for (int i = 0; i < 8; ++i) x[i] = ld(A, (size_t)(m0 + r) * a.K + 8 * pk + i);
          acc[r] = fmaf(dot8(x, q), s, acc[r]);
        }
      }
    }
  }
#pragma unroll
  for (int r = 0; r < kGRows; ++r) red[sl][r][c] = acc[r];
  __syncthreads();
  for (int o = tid; o < rows * kGCols; o += kGT) {
    const int r = o / kGCols, cc = o % kGCols, n = blockIdx.x * kGCols + cc;
    if (n >= a.N) continue;
    float y = 0.f;
#pragma unroll
    for (int s2 = 0; s2 < kGSlices; ++s2) y += red[s2][r][cc];
    if (a.cap > 0.f) y = a.cap * tanhf(y / a.cap);
    st((T*)a.C, (size_t)(m0 + r) * a.N + n, y);
  }
}

// ---------------------------------------------------------------------------
// MoE
// ---------------------------------------------------------------------------
struct GMoeArgs {
  const void* x;
  const int32_t* gu_packed;
  const void* gu_scales;
  const int32_t* d_packed;
  const void* d_scales;
  const void* idx;
  const void* w;
  void* out;
  float* act;  // [S][I] the activations, rounded to T
  int idx_is64, w_dtype;
  int M, H, I, E, top_k, gs, Ggu, Gd, S;
};

__device__ __forceinline__ int slot_expert(const GMoeArgs& a, int s) {
  const int e = load_expert_id(a.idx, a.idx_is64, s);
  return (e >= 0 && e < a.E) ? e : -1;
}

template <typename T>
__global__ __launch_bounds__(kGT) void moe_generic_gu_kernel(GMoeArgs a) {
  __shared__ float red[kGSlices][kGCols];
  const int s = blockIdx.x, ct = blockIdx.y;
  const int tid = threadIdx.x, c = tid % kGCols, sl = tid / kGCols;
  const int e = slot_expert(a, s);
  const int tok = s / a.top_k;
  const int twoI = 2 * a.I;
  const int col = (c < 32 ? 0 : a.I) + 32 * ct + (c & 31);
  const bool colok = 32 * ct + (c & 31) < a.I;
  const T* X = (const T*)a.x + (size_t)tok * a.H;
  const T* S = (const T*)a.gu_scales;
  const int P = a.H / 8;
  const int Pv = min(P, a.Ggu * a.gs / 8);
  const int per = (Pv + kGSlices - 1) / kGSlices;
  const int p0 = sl * per, p1 = min(Pv, p0 + per);
  float acc = 0.f;
  if (e >= 0 && colok) {
    const int32_t* Bw = a.gu_packed + (size_t)e * P * twoI;
    const T* Se = S + (size_t)e * a.Ggu * twoI;
    for (int pk = p0; pk < p1; ++pk) {
      float q[8], x[8];
      codes8((uint32_t)Bw[(size_t)pk * twoI + col], q);
#pragma unroll
      for (int i = 0; i < 8; ++i) x[i] = ld(X, (size_t)8 * pk + i);
      acc = fmaf(dot8(x, q), ld(Se, (size_t)(pk * 8 / a.gs) * twoI + col), acc);
    }
  }
  red[sl][c] = acc;
  __syncthreads();
  if (tid < 32) {
    float g = 0.f, u = 0.f;
#pragma unroll
    for (int s2 = 0; s2 < kGSlices; ++s2) {
      g += red[s2][tid];
      u += red[s2][32 + tid];
    }
    const int i = 32 * ct + tid;
    const int Iv = min(a.I, a.Gd * a.gs);  // activations past the last down group are dropped
    if (i < a.I) a.act[(size_t)s * a.I + i] = (e >= 0 && i < Iv) ? round_t<T>(gelu_tanh(g) * u) : 0.f;
  }
}

template <typename T>
__global__ __launch_bounds__(kGT) void moe_generic_down_kernel(GMoeArgs a) {
  extern __shared__ float dred[];  // [top_k][kGSlices][kGCols]
  const int ct = blockIdx.x, tok = blockIdx.y;
  const int tid = threadIdx.x, c = tid % kGCols, sl = tid / kGCols;
  const int col = ct * kGCols + c;
  const int P = a.I / 8;
  const int Pv = min(P, a.Gd * a.gs / 8);
  const int per = (Pv + kGSlices - 1) / kGSlices;
  const int p0 = sl * per, p1 = min(Pv, p0 + per);
  const T* S = (const T*)a.d_scales;
  for (int k = 0; k < a.top_k; ++k) {
    const int s = tok * a.top_k + k;
    const int e = slot_expert(a, s);
    float acc = 0.f;
    if (e >= 0 && col < a.H) {
      const int32_t* Bw = a.d_packed + (size_t)e * P * a.H;
      const T* Se = S + (size_t)e * a.Gd * a.H;
      const float* act = a.act + (size_t)s * a.I;
      for (int pk = p0; pk < p1; ++pk) {
        float q[8], x[8];
        codes8((uint32_t)Bw[(size_t)pk * a.H + col], q);
#pragma unroll
        for (int i = 0; i < 8; ++i) x[i] = act[8 * pk + i];
        acc = fmaf(dot8(x, q), ld(Se, (size_t)(pk * 8 / a.gs) * a.H + col), acc);
      }
    }
    dred[(k * kGSlices + sl) * kGCols + c] = acc;
  }
  __syncthreads();
  if (tid < kGCols && col < a.H) {
    float y = 0.f;
    for (int k = 0; k < a.top_k; ++k) {
      const int s = tok * a.top_k + k;
      if (slot_expert(a, s) < 0) continue;
      // the weight cast to the activation dtype (marlin.cu:634-636)
      float wv;
      if (a.w_dtype == GI_DTYPE_FP32) wv = ((const float*)a.w)[s];
      else if (a.w_dtype == GI_DTYPE_FP16) wv = fp16_to_f32(((const uint16_t*)a.w)[s]);
      else wv = bf16_to_f32(((const uint16_t*)a.w)[s]);
      wv = round_t<T>(wv);
      float yk = 0.f;
#pragma unroll
      for (int s2 = 0; s2 < kGSlices; ++s2) yk += dred[(k * kGSlices + s2) * kGCols + tid];
      y = fmaf(wv, yk, y);
    }
    T* out = (T*)a.out;
    const size_t o = (size_t)tok * a.H + col;
    st(out, o, ld((const T*)out, o) + y);
  }
}

template <typename T>
int launch_linear_t(const GLinArgs& k, hipStream_t stream) {
  const dim3 grid((k.N + kGCols - 1) / kGCols, (k.M + kGRows - 1) / kGRows);
  hipLaunchKernelGGL(w4a16_generic_kernel<T>, grid, dim3(kGT), 0, stream, k);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? GI_OK : hip_fail(e, "w4a16 (fp16/fp32) launch");
}

template <typename T>
int launch_moe_t(const GMoeArgs& k, hipStream_t stream) {
  hipLaunchKernelGGL(moe_generic_gu_kernel<T>, dim3(k.S, (k.I + 31) / 32), dim3(kGT), 0, stream, k);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return hip_fail(e, "fused MoE (fp16/fp32) gate/up launch");
  const size_t lds = (size_t)k.top_k * kGSlices * kGCols * sizeof(float);
  hipLaunchKernelGGL(moe_generic_down_kernel<T>, dim3((k.H + kGCols - 1) / kGCols, k.M), dim3(kGT), lds, stream, k);
  e = hipGetLastError();
  return e == hipSuccess ? GI_OK : hip_fail(e, "fused MoE (fp16/fp32) down launch");
}

}  // namespace

size_t moe_generic_workspace_bytes(int M, int top_k, int I) { return (size_t)M * top_k * I * sizeof(float); }

int launch_moe_generic(const MoeHostArgs& h, int x_dtype, void* act_ws, size_t act_bytes) {
  if (x_dtype != GI_DTYPE_FP16 && x_dtype != GI_DTYPE_FP32)
    return fail(GI_ERR_UNSUPPORTED, "fused MoE: activations must be bf16, fp16 or fp32");
  if (h.logits) return fail(GI_ERR_UNSUPPORTED, "fused MoE: routing from logits takes bf16 activations");
  if (h.M == 0) return GI_OK;
  if ((size_t)h.top_k * kGSlices * kGCols * sizeof(float) > 48 * 1024)
    return fail(GI_ERR_UNSUPPORTED, "fused MoE (fp16/fp32): top_k <= 48");
  if (act_bytes < moe_generic_workspace_bytes(h.M, h.top_k, h.I))
    return fail(GI_ERR_WORKSPACE, "fused MoE (fp16/fp32): workspace too small for the activations");
  GMoeArgs k{};
  k.x = h.x;
  k.gu_packed = h.gu_packed;
  k.gu_scales = h.gu_scales;
  k.d_packed = h.d_packed;
  k.d_scales = h.d_scales;
  k.idx = h.idx;
  k.w = h.w;
  k.out = h.out;
  k.act = (float*)act_ws;
  k.idx_is64 = h.idx_is64;
  k.w_dtype = h.w_dtype;
  k.M = h.M;
  k.H = h.H;
  k.I = h.I;
  k.E = h.E;
  k.top_k = h.top_k;
  k.gs = h.gs;
  k.Ggu = h.Ggu;
  k.Gd = h.Gd;
  k.S = h.M * h.top_k;
  return x_dtype == GI_DTYPE_FP16 ? launch_moe_t<_Float16>(k, h.stream) : launch_moe_t<float>(k, h.stream);
}

int launch_w4a16_generic(const void* A, int a_dtype, const int32_t* B, const void* scales, int n_groups, void* C,
                         int M, int K, int N, int gs, float softcap, hipStream_t stream) {
  if (a_dtype != GI_DTYPE_FP16 && a_dtype != GI_DTYPE_FP32)
    return fail(GI_ERR_UNSUPPORTED, "w4a16: activations must be bf16, fp16 or fp32");
  if (M < 0 || K <= 0 || N <= 0) return fail(GI_ERR_INVALID_ARG, "w4a16: K and N must be positive, M >= 0");
  if (K % 8) return fail(GI_ERR_INVALID_ARG, "w4a16: K must be a multiple of 8 (8 codes per int32)");
  if (gs <= 0 || gs % 8) return fail(GI_ERR_INVALID_ARG, "w4a16: group_size must be a positive multiple of 8");
  if (n_groups <= 0) return fail(GI_ERR_INVALID_ARG, "w4a16: scales need at least one group");
  if (!A || !B || !scales || !C) return fail(GI_ERR_INVALID_ARG, "w4a16: null tensor pointer");
  if (M == 0) return GI_OK;
  GLinArgs k{};
  k.A = A;
  k.B = B;
  k.S = scales;
  k.C = C;
  k.M = M;
  k.K = K;
  k.N = N;
  k.G = n_groups;
  k.gs = gs;
  k.cap = softcap;
  return a_dtype == GI_DTYPE_FP16 ? launch_linear_t<_Float16>(k, stream) : launch_linear_t<float>(k, stream);
}

}  // namespace gi
