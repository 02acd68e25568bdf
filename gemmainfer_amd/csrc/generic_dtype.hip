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
//   MoE      Token-Union, in launches of up to 64 slots: the alignment kernel
//            (unique experts in first-occurrence order, each one's slots);
//            gate/up per (unique expert, 32-column tile): 32 gate + 32 up
//            columns x 4 slices of H, the expert's words read once for all
//            of its slots (their token rows staged in LDS), activation
//            rounded to T into an fp32 buffer [S][I] in the workspace; down
//            per (unique expert, 64-column tile) the same way, each slot's
//            fp32 output row into [S][H]; then the combine: old + the sum
//            over each token's slots of w * y in slot order, one rounding.
// The weights are never rounded: each packed row's codes times the
// activations are summed in fp32 and scaled by the row's group scale (as the
// reference's GPU kernels apply the scale after the codes' sums,
// marlin.cu:412-413, :573).

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
// MoE (Token-Union: each unique expert's words read once per launch)
// ---------------------------------------------------------------------------
constexpr int kGChunkSlots = 64;  // slots per launch
constexpr int kGB = 8;            // slots of one expert per pass over its words (registers, LDS rows)
constexpr int kGK = 1024;         // k values of the staged rows per pass (128 packed rows)

struct GMoeArgs {
  const void* x;
  const int32_t* gu_packed;
  const void* gu_scales;
  const int32_t* d_packed;
  const void* d_scales;
  const void* idx;
  const void* w;
  void* out;
  float* act;             // [S][I] the activations, rounded to T
  float* ys;              // [S][H] each slot's down output (fp32)
  const int32_t* uniq;    // Token-Union tables of the launch's slots (moe_align_kernel)
  const int32_t* nuniq;
  const int32_t* offsets;
  const int32_t* slots;
  int idx_is64, w_dtype;
  int M, H, I, E, top_k, gs, Ggu, Gd, S;
};

__device__ __forceinline__ int slot_expert(const GMoeArgs& a, int s) {
  const int e = load_expert_id(a.idx, a.idx_is64, s);
  return (e >= 0 && e < a.E) ? e : -1;
}

// Unconditional loads through buffer resources: an element past the
// resource (offset kGOob) reads zero with no memory access, so no load sits
// under a per-lane branch (the compiler waits for such a load right away).
constexpr uint32_t kGOob = 0xFFFFFFF0u;
template <typename S>
__device__ __forceinline__ float bload(__amdgpu_buffer_rsrc_t r, size_t i, bool ok);
template <>
__device__ __forceinline__ float bload<_Float16>(__amdgpu_buffer_rsrc_t r, size_t i, bool ok) {
  return fp16_to_f32(__builtin_amdgcn_raw_buffer_load_b16(r, ok ? (uint32_t)(i * 2) : kGOob, 0, 0));
}
template <>
__device__ __forceinline__ float bload<float>(__amdgpu_buffer_rsrc_t r, size_t i, bool ok) {
  return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, ok ? (uint32_t)(i * 4) : kGOob, 0, 0));
}

// Products of one unique expert's 64 columns (thread: column c, slice sl of
// the packed rows) with up to kGB rows staged in LDS, k chunk by k chunk:
// row jj is element rowbase[jj] of the src resource (K values of type S),
// staged as fp32 with every load of the chunk issued before any store; each
// thread's packed rows of the chunk then run kU at a time with their word
// and scale loads issued first.  acc[jj] += scale * sum over the row's codes
// of row[k] * (q - 8).
template <typename T, typename S>
__device__ __forceinline__ void slot_products(__amdgpu_buffer_rsrc_t rw, __amdgpu_buffer_rsrc_t rs, int ld_w,
                                              int col, bool colok, int K, int Pv, int rpg, int nb,
                                              float (*xs)[kGK], __amdgpu_buffer_rsrc_t rsrc,
                                              const size_t (&rowbase)[kGB], float (&acc)[kGB]) {
  const int tid = threadIdx.x, sl = tid / kGCols;
  constexpr int kPer = kGK / kGT;  // staged values per thread and row
#pragma unroll
  for (int jj = 0; jj < kGB; ++jj) acc[jj] = 0.f;
  for (int k0 = 0; k0 < K; k0 += kGK) {
    float v[kGB][kPer];
#pragma unroll
    for (int jj = 0; jj < kGB; ++jj)
#pragma unroll
      for (int n = 0; n < kPer; ++n) {
        const int k = k0 + tid + kGT * n;
        v[jj][n] = bload<S>(rsrc, rowbase[jj] + k, jj < nb && k < K);
      }
    __syncthreads();  // the previous chunk's readers are done
#pragma unroll
    for (int jj = 0; jj < kGB; ++jj)
#pragma unroll
      for (int n = 0; n < kPer; ++n) xs[jj][tid + kGT * n] = v[jj][n];
    __syncthreads();
    // this thread's packed rows of the chunk: a quarter of its 128
    const int pc0 = k0 / 8 + sl * (kGK / 8 / kGSlices);
    const int pc1 = min(Pv, pc0 + kGK / 8 / kGSlices);
    constexpr int kU = 8;  // packed rows whose loads are in flight together
    for (int pb = pc0; pb < pc1; pb += kU) {
      uint32_t wv[kU];
      float sv[kU];
#pragma unroll
      for (int r = 0; r < kU; ++r) {
        const int pk = pb + r;
        const bool ok = colok && pk < pc1;
        const int g = pk / rpg;  // packed rows per scale group: group_size / 8
        wv[r] = __builtin_amdgcn_raw_buffer_load_b32(rw, ok ? (uint32_t)(pk * ld_w + col) * 4u : kGOob, 0, 0);
        sv[r] = bload<T>(rs, (size_t)g * ld_w + col, ok);  // zero scale: the row adds nothing
      }
#pragma unroll
      for (int r = 0; r < kU; ++r) {
        float q[8];
        codes8(wv[r], q);
        const int kk = (min(pb + r, pc1 - 1) - k0 / 8) * 8;
#pragma unroll
        for (int jj = 0; jj < kGB; ++jj) {
          if (jj < nb) {
            const float4 v0 = *(const float4*)&xs[jj][kk], v1 = *(const float4*)&xs[jj][kk + 4];
            const float x[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
            acc[jj] = fmaf(dot8(x, q), sv[r], acc[jj]);
          }
        }
      }
    }
  }
}

// Workgroup (u, ct): unique expert u's gate columns [32ct, 32ct+32) and the
// same up columns (64 threads) x 4 slices of H, for every slot routed to u
// (kGB slots per pass over the words: one pass when the expert serves at
// most kGB slots, as at M <= 8 with distinct ids per token).
template <typename T>
__global__ __launch_bounds__(kGT) void moe_generic_gu_kernel(GMoeArgs a) {
  __shared__ float red[kGSlices][kGB][kGCols];
  __shared__ float xs[kGB][kGK];
  const int u = blockIdx.x, ct = blockIdx.y;
  if (u >= *a.nuniq) return;
  const int tid = threadIdx.x, c = tid % kGCols, sl = tid / kGCols;
  const int e = a.uniq[u], j0 = a.offsets[u], j1 = a.offsets[u + 1];
  const int twoI = 2 * a.I;
  const int col = (c < 32 ? 0 : a.I) + 32 * ct + (c & 31);
  const bool colok = 32 * ct + (c & 31) < a.I;
  const int Pv = min(a.H / 8, a.Ggu * a.gs / 8);  // packed rows past the last scale group are dropped
  const __amdgpu_buffer_rsrc_t rw = buffer_rsrc(a.gu_packed + (size_t)e * (a.H / 8) * twoI,
                                                (uint32_t)((size_t)(a.H / 8) * twoI * 4));
  const __amdgpu_buffer_rsrc_t rs = buffer_rsrc((const T*)a.gu_scales + (size_t)e * a.Ggu * twoI,
                                                (uint32_t)((size_t)a.Ggu * twoI * sizeof(T)));
  const __amdgpu_buffer_rsrc_t rx = buffer_rsrc(a.x, (uint32_t)((size_t)a.M * a.H * sizeof(T)));
  const int Iv = min(a.I, a.Gd * a.gs);  // activations past the last down group are dropped
  for (int jb = j0; jb < j1; jb += kGB) {
    const int nb = min(kGB, j1 - jb);
    // the batch's slots in one load (lane jj holds slot jj), then made uniform
    const int slot_v = a.slots[jb + min((int)(threadIdx.x & 63), nb - 1)];
    size_t rowbase[kGB];
#pragma unroll
    for (int jj = 0; jj < kGB; ++jj) rowbase[jj] = (size_t)(__builtin_amdgcn_readlane(slot_v, jj) / a.top_k) * a.H;
    float acc[kGB];
    slot_products<T, T>(rw, rs, twoI, col, colok, a.H, Pv, a.gs / 8, nb, xs, rx, rowbase, acc);
#pragma unroll
    for (int jj = 0; jj < kGB; ++jj) red[sl][jj][c] = acc[jj];
    __syncthreads();
    {
      const int jj = tid >> 5, i = 32 * ct + (tid & 31);
      if (jj < nb && i < a.I) {
        float g = 0.f, up = 0.f;
#pragma unroll
        for (int s2 = 0; s2 < kGSlices; ++s2) {
          g += red[s2][jj][tid & 31];
          up += red[s2][jj][32 + (tid & 31)];
        }
        a.act[(size_t)a.slots[jb + jj] * a.I + i] = i < Iv ? round_t<T>(gelu_tanh(g) * up) : 0.f;
      }
    }
  }
}

// Workgroup (u, ct): unique expert u's down columns [64ct, 64ct+64) x 4
// slices of I, for every slot routed to u: each slot's fp32 output row
// ys[slot] (its words read once per kGB slots).
template <typename T>
__global__ __launch_bounds__(kGT) void moe_generic_down_kernel(GMoeArgs a) {
  __shared__ float red[kGSlices][kGB][kGCols];
  __shared__ float xs[kGB][kGK];
  const int u = blockIdx.x, ct = blockIdx.y;
  if (u >= *a.nuniq) return;
  const int tid = threadIdx.x, c = tid % kGCols, sl = tid / kGCols;
  const int e = a.uniq[u], j0 = a.offsets[u], j1 = a.offsets[u + 1];
  const int col = kGCols * ct + c;
  const bool colok = col < a.H;
  const int Pv = min(a.I / 8, a.Gd * a.gs / 8);
  const __amdgpu_buffer_rsrc_t rw = buffer_rsrc(a.d_packed + (size_t)e * (a.I / 8) * a.H,
                                                (uint32_t)((size_t)(a.I / 8) * a.H * 4));
  const __amdgpu_buffer_rsrc_t rs = buffer_rsrc((const T*)a.d_scales + (size_t)e * a.Gd * a.H,
                                                (uint32_t)((size_t)a.Gd * a.H * sizeof(T)));
  const __amdgpu_buffer_rsrc_t ra = buffer_rsrc(a.act, (uint32_t)((size_t)a.S * a.I * 4));
  for (int jb = j0; jb < j1; jb += kGB) {
    const int nb = min(kGB, j1 - jb);
    const int slot_v = a.slots[jb + min((int)(threadIdx.x & 63), nb - 1)];
    size_t rowbase[kGB];
#pragma unroll
    for (int jj = 0; jj < kGB; ++jj) rowbase[jj] = (size_t)__builtin_amdgcn_readlane(slot_v, jj) * a.I;
    float acc[kGB];
    slot_products<T, float>(rw, rs, a.H, col, colok, a.I, Pv, a.gs / 8, nb, xs, ra, rowbase, acc);
#pragma unroll
    for (int jj = 0; jj < kGB; ++jj) red[sl][jj][c] = acc[jj];
    __syncthreads();
    for (int o = tid; o < nb * kGCols; o += kGT) {
      const int jj = o / kGCols, cc = o % kGCols, n = kGCols * ct + cc;
      if (n < a.H)
        a.ys[(size_t)a.slots[jb + jj] * a.H + n] =
            ((red[0][jj][cc] + red[1][jj][cc]) + red[2][jj][cc]) + red[3][jj][cc];
    }
  }
}

// out[tok] = old + sum over the token's slots, in slot order, of the weight
// (cast to the activation dtype, marlin.cu:634-636) times the slot's output;
// one rounding.  Slots whose id is outside [0, E) add nothing.
template <typename T>
__global__ __launch_bounds__(kGT) void moe_generic_combine_kernel(GMoeArgs a) {
  const int tok = blockIdx.y, n = blockIdx.x * kGT + threadIdx.x;
  if (n >= a.H) return;
  float y = 0.f;
  for (int k = 0; k < a.top_k; ++k) {
    const int s = tok * a.top_k + k;
    if (slot_expert(a, s) < 0) continue;
    float wv;
    if (a.w_dtype == GI_DTYPE_FP32) wv = ((const float*)a.w)[s];
    else if (a.w_dtype == GI_DTYPE_FP16) wv = fp16_to_f32(((const uint16_t*)a.w)[s]);
    else wv = bf16_to_f32(((const uint16_t*)a.w)[s]);
    y = fmaf(round_t<T>(wv), a.ys[(size_t)s * a.H + n], y);
  }
  T* out = (T*)a.out;
  const size_t oi = (size_t)tok * a.H + n;
  st(out, oi, ld((const T*)out, oi) + y);
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
  const int umax = k.S < k.E ? k.S : k.E;
  hipLaunchKernelGGL(moe_generic_gu_kernel<T>, dim3(umax, (k.I + 31) / 32), dim3(kGT), 0, stream, k);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return hip_fail(e, "fused MoE (fp16/fp32) gate/up launch");
  hipLaunchKernelGGL(moe_generic_down_kernel<T>, dim3(umax, (k.H + kGCols - 1) / kGCols), dim3(kGT), 0, stream, k);
  e = hipGetLastError();
  if (e != hipSuccess) return hip_fail(e, "fused MoE (fp16/fp32) down launch");
  hipLaunchKernelGGL(moe_generic_combine_kernel<T>, dim3((k.H + kGT - 1) / kGT, k.M), dim3(kGT), 0, stream, k);
  e = hipGetLastError();
  return e == hipSuccess ? GI_OK : hip_fail(e, "fused MoE (fp16/fp32) combine launch");
}

// workspace: the activations [S][I] and slot outputs [S][H] (fp32), then the
// Token-Union tables
constexpr size_t kGTables = 4 * (3 * kGChunkSlots + 2 + kGChunkSlots);  // uniq, nuniq, offsets, slots, s2u

int chunk_rows(int top_k) { return top_k >= kGChunkSlots ? 1 : kGChunkSlots / top_k; }

size_t slot_bufs_bytes(int M, int top_k, int H, int I) {
  const int rows = M < chunk_rows(top_k) ? M : chunk_rows(top_k);
  return ((size_t)rows * top_k * (H + I) * sizeof(float) + 255) / 256 * 256;
}

}  // namespace

size_t moe_generic_workspace_bytes(int M, int top_k, int H, int I) {
  return slot_bufs_bytes(M, top_k, H, I) + kGTables;
}

int launch_moe_generic(const MoeHostArgs& h, int x_dtype, void* act_ws, size_t act_bytes) {
  if (x_dtype != GI_DTYPE_FP16 && x_dtype != GI_DTYPE_FP32)
    return fail(GI_ERR_UNSUPPORTED, "fused MoE: activations must be bf16, fp16 or fp32");
  if (h.logits) return fail(GI_ERR_UNSUPPORTED, "fused MoE: routing from logits takes bf16 activations");
  if (h.M == 0) return GI_OK;
  if (h.top_k > kGChunkSlots) return fail(GI_ERR_UNSUPPORTED, "fused MoE (fp16/fp32): top_k <= 64");
  if (act_bytes < moe_generic_workspace_bytes(h.M, h.top_k, h.H, h.I))
    return fail(GI_ERR_WORKSPACE, "fused MoE (fp16/fp32): workspace too small for the activations");
  const int per = chunk_rows(h.top_k);
  int32_t* tab = (int32_t*)((char*)act_ws + slot_bufs_bytes(h.M, h.top_k, h.H, h.I));
  GMoeArgs k{};
  k.gu_packed = h.gu_packed;
  k.gu_scales = h.gu_scales;
  k.d_packed = h.d_packed;
  k.d_scales = h.d_scales;
  k.act = (float*)act_ws;
  k.ys = (float*)act_ws + (size_t)(h.M < per ? h.M : per) * h.top_k * h.I;
  k.uniq = tab;
  k.nuniq = tab + kGChunkSlots;
  k.offsets = tab + kGChunkSlots + 1;
  k.slots = tab + 2 * kGChunkSlots + 2;
  int32_t* s2u = tab + 3 * kGChunkSlots + 2;
  k.idx_is64 = h.idx_is64;
  k.w_dtype = h.w_dtype;
  k.H = h.H;
  k.I = h.I;
  k.E = h.E;
  k.top_k = h.top_k;
  k.gs = h.gs;
  k.Ggu = h.Ggu;
  k.Gd = h.Gd;
  const size_t xes = x_dtype == GI_DTYPE_FP16 ? 2 : 4;
  const size_t ies = h.idx_is64 ? 8 : 4;
  const size_t wes = h.w_dtype == GI_DTYPE_FP32 ? 4 : 2;
  // launches of up to 64 slots, in order on the stream (each reuses the
  // activation buffer and the tables once the previous one has finished)
  for (int r0 = 0; r0 < h.M; r0 += per) {
    const int rows = h.M - r0 < per ? h.M - r0 : per;
    const size_t s0 = (size_t)r0 * h.top_k;
    k.x = (const char*)h.x + (size_t)r0 * h.H * xes;
    k.out = (char*)h.out + (size_t)r0 * h.H * xes;
    k.idx = (const char*)h.idx + s0 * ies;
    k.w = (const char*)h.w + s0 * wes;
    k.M = rows;
    k.S = rows * h.top_k;
    int st = launch_moe_align(k.idx, h.idx_is64, rows, h.top_k, h.E, tab, tab + kGChunkSlots, s2u,
                              tab + kGChunkSlots + 1, tab + 2 * kGChunkSlots + 2, h.stream);
    if (st != GI_OK) return st;
    st = x_dtype == GI_DTYPE_FP16 ? launch_moe_t<_Float16>(k, h.stream) : launch_moe_t<float>(k, h.stream);
    if (st != GI_OK) return st;
  }
  return GI_OK;
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
