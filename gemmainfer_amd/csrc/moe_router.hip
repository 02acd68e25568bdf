// Router front-end of the MoE block in one launch (gfx950): the statement
//
//   x_normed = router_norm(x) * (router_scale * H^-0.5);  logits = gate(x_normed)
//
// of gemma.py:75-76, with every rounding the bf16 model performs:
//   n[m][h]      = bf16( x[m][h] * rsqrt(sum_h x[m][h]^2 / H + eps) )
//                  GemmaRMSNorm(with_scale=False), norm.py:28-40 -> rmsnorm.cu:16-73
//                  (fp32 sum of squares, one rsqrt per row, bf16 store);
//   s[h]         = bf16( router_scale[h] * (float)H^-0.5 )
//                  (a bf16 parameter times a Python float: fp32 product, bf16 result);
//   xr[m][h]     = bf16( n[m][h] * s[h] )          (bf16 * bf16 -> bf16);
//   logits[m][e] = bf16( sum_h xr[m][h] * gate[e][h] )
//                  (nn.Linear over bf16: fp32 accumulation, one rounding).
// The fp32 sums run in a fixed order of our own (the reference's order is the
// BLAS library's), so a logit can differ from the reference's by one bf16 ulp
// where the fp32 sum lands next to a rounding boundary.
//
// Layout: gate is the nn.Linear weight [E, H] (row e = expert e), x [M, H],
// logits [M, E], all bf16 row-major.  Two kernels:
//   * moe_router_rows_kernel (M <= 8, decode and verify): one workgroup per
//     (row, expert), every thread owning one 16-byte column vector, so nothing
//     is staged; a latency-bound step that reads the ~H*E*2 gate bytes
//     (720 KB for Gemma's 2816 x 128 gate) once.
//   * moe_router_kernel (M > 8): rows in blocks of 8 normalised once into LDS
//     per workgroup, 4*EPW experts per workgroup.
// Every bf16 rounding uses the hardware round-to-nearest-even conversion
// (v_cvt_pk_bf16_f32).
#include "../../include/gemmainfer_amd.h"
#include "gi_common.h"
#include "gi_internal.h"
#include "moe_shared.h"

#include <cmath>

namespace gi {

namespace {

constexpr int kRouterWaves = 4;
constexpr int kRouterMaxJ = 8;     // 512 columns per step: H <= 4096
constexpr uint32_t kRouterOob = 0xFFFFFFF0u;  // buffer offset past the resource: the load returns zeros

struct RouterArgs {
  const uint16_t* x;       // [M, H]
  const uint16_t* rscale;  // [H] or null (all ones)
  const uint16_t* gate;    // [E, H]
  uint16_t* logits;        // [M, E]
  int M, H, E;
  float eps, c;            // c = (float)H^-0.5
};

__device__ __forceinline__ float sq8(uint4 d, float s) {
  const uint32_t w[4] = {d.x, d.y, d.z, d.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float lo = bf16lo(w[i]), hi = bf16hi(w[i]);
    s = fmaf(lo, lo, s);
    s = fmaf(hi, hi, s);
  }
  return s;
}

__device__ __forceinline__ float dot8(uint4 g, uint4 x, float acc) {
  acc = fdot2(g.x, x.x, acc);
  acc = fdot2(g.y, x.y, acc);
  acc = fdot2(g.z, x.z, acc);
  return fdot2(g.w, x.w, acc);
}

// Workgroup: 4 waves, rows m0 .. m0 + R - 1 (R a power of two <= 8; rows past
// M are masked), experts e0 .. e0 + 4*EPW - 1 (one group of EPW per wave).
//   A. Every thread owns 16-byte column vectors v = tid + 256 ja (ja < 2) of
//      every row: sum of squares -> per-row workgroup total (LDS, one
//      barrier) -> x_normed = bf16(bf16(x r) s) into LDS [R][H/8] vectors.
//   B. Each wave dots its gate rows (in registers since the start) with every
//      LDS row and reduces across its 64 lanes.
template <int EPW, int J, int R>
__global__ __launch_bounds__(256) void moe_router_kernel(RouterArgs a) {
  extern __shared__ uint4 xs[];  // [R][H / 8]
  __shared__ float red[R][kRouterWaves];
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid >> 6;
  const int hv = a.H >> 3;  // 16-byte vectors per row
  const int m0 = blockIdx.y * R;
  const int nrows = min(R, a.M - m0);
  const int e0 = (blockIdx.x * kRouterWaves + wave) * EPW;

  // Every global load is issued up front, without per-lane branches (masked
  // vectors read zeros through the buffer range check): this wave's gate rows,
  // then the router scale and the rows at this thread's columns.
  const __amdgpu_buffer_rsrc_t rg = buffer_rsrc(a.gate, (uint32_t)((size_t)a.E * a.H * 2));
  uint4 g[EPW][J];
#pragma unroll
  for (int q = 0; q < EPW; ++q)
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const int v = lane + kWave * j, e = e0 + q;
      const uint32_t off = (v < hv && e < a.E) ? (uint32_t)(((size_t)e * a.H + 8 * v) * 2) : kRouterOob;
      const u32x4_t d = __builtin_amdgcn_raw_buffer_load_b128(rg, off, 0, 0);
      g[q][j] = make_uint4(d.x, d.y, d.z, d.w);
    }
  constexpr int JA = 2;  // 256 threads x 2 vectors x 8 columns = 4096 >= H
  const __amdgpu_buffer_rsrc_t rs = buffer_rsrc(a.rscale, a.rscale ? (uint32_t)(a.H * 2) : 0u);
  const __amdgpu_buffer_rsrc_t rx =
      buffer_rsrc(a.x + (size_t)m0 * a.H, (uint32_t)((size_t)nrows * a.H * 2));
  uint4 sa[JA];
  uint4 xa[R][JA];
#pragma unroll
  for (int ja = 0; ja < JA; ++ja) {
    const int v = tid + 256 * ja;
    const u32x4_t d = __builtin_amdgcn_raw_buffer_load_b128(rs, v < hv ? (uint32_t)(16 * v) : kRouterOob, 0, 0);
    sa[ja] = make_uint4(d.x, d.y, d.z, d.w);
  }
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int ja = 0; ja < JA; ++ja) {
      const int v = tid + 256 * ja;
      const uint32_t off = (r < nrows && v < hv) ? (uint32_t)((r * a.H + 8 * v) * 2) : kRouterOob;
      const u32x4_t d = __builtin_amdgcn_raw_buffer_load_b128(rx, off, 0, 0);
      xa[r][ja] = make_uint4(d.x, d.y, d.z, d.w);
    }
  // keep every load above this point: one memory round trip for all of them
  __builtin_amdgcn_sched_barrier(0);

  // Per-row sums of squares over the workgroup.
#pragma unroll
  for (int r = 0; r < R; ++r) {
    float ss = 0.f;
#pragma unroll
    for (int ja = 0; ja < JA; ++ja) ss = sq8(xa[r][ja], ss);
    ss = wave_sum_f32(ss);
    if (lane == 0) red[r][wave] = ss;
  }
  // s[h] = bf16(router_scale[h] * c) as fp32; a missing router_scale is ones.
  float sf[JA][8];
#pragma unroll
  for (int ja = 0; ja < JA; ++ja) {
    const uint32_t w[4] = {sa[ja].x, sa[ja].y, sa[ja].z, sa[ja].w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t src = a.rscale ? w[i] : 0x3f803f80u;
      const uint32_t p = pack_bf16x2(bf16lo(src) * a.c, bf16hi(src) * a.c);
      sf[ja][2 * i] = bf16lo(p);
      sf[ja][2 * i + 1] = bf16hi(p);
    }
  }
  __syncthreads();
#pragma unroll
  for (int r = 0; r < R; ++r) {
    if (r < nrows) {
      const float tot = (red[r][0] + red[r][1]) + (red[r][2] + red[r][3]);
      const float rr = rsqrtf(tot / (float)a.H + a.eps);
#pragma unroll
      for (int ja = 0; ja < JA; ++ja) {
        const int v = tid + 256 * ja;
        if (v < hv) {
          const uint32_t w[4] = {xa[r][ja].x, xa[r][ja].y, xa[r][ja].z, xa[r][ja].w};
          uint32_t o[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const uint32_t n = pack_bf16x2(bf16lo(w[i]) * rr, bf16hi(w[i]) * rr);
            o[i] = pack_bf16x2(bf16lo(n) * sf[ja][2 * i], bf16hi(n) * sf[ja][2 * i + 1]);
          }
          xs[r * hv + v] = make_uint4(o[0], o[1], o[2], o[3]);
        }
      }
    }
  }
  __syncthreads();

  float acc[EPW][R];
#pragma unroll
  for (int q = 0; q < EPW; ++q)
#pragma unroll
    for (int r = 0; r < R; ++r) acc[q][r] = 0.f;
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int v = lane + kWave * j;
    if (v < hv) {
#pragma unroll
      for (int r = 0; r < R; ++r) {
        if (r < nrows) {
          const uint4 xv = xs[r * hv + v];
#pragma unroll
          for (int q = 0; q < EPW; ++q) acc[q][r] = dot8(g[q][j], xv, acc[q][r]);
        }
      }
    }
  }
#pragma unroll
  for (int q = 0; q < EPW; ++q) {
    const int e = e0 + q;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if (r < nrows) {
        const float t = wave_sum_f32(acc[q][r]);
        if (lane == 0 && e < a.E) a.logits[(size_t)(m0 + r) * a.E + e] = f32_to_bf16(t);
      }
    }
  }
}

// Decode shape (M <= 8): one workgroup of 512 threads per (row, expert).
// Thread t owns the 8 columns of 16-byte vector t (H <= 4096), so the row's
// normalised values, the gate values and their products stay in its
// registers: the sum of squares and the dot product are each one wave
// reduction plus an 8-entry LDS sum in a fixed order.  Every workgroup
// normalises its row again; at this size that costs nothing next to the
// memory round trip, and it keeps each workgroup's chain of work short.
__global__ __launch_bounds__(512) void moe_router_rows_kernel(RouterArgs a) {
  constexpr int kW = 8;  // waves
  __shared__ float red[kW];
  __shared__ float part[kW];
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid >> 6;
  const int hv = a.H >> 3;
  const int e = blockIdx.x, m = blockIdx.y;
  const bool valid = tid < hv;

  const __amdgpu_buffer_rsrc_t rg = buffer_rsrc(a.gate, (uint32_t)((size_t)a.E * a.H * 2));
  const __amdgpu_buffer_rsrc_t rs = buffer_rsrc(a.rscale, a.rscale ? (uint32_t)(a.H * 2) : 0u);
  const __amdgpu_buffer_rsrc_t rx = buffer_rsrc(a.x + (size_t)m * a.H, (uint32_t)(a.H * 2));
  u32x4_t t = __builtin_amdgcn_raw_buffer_load_b128(
      rg, valid ? (uint32_t)(((size_t)e * a.H + 8 * tid) * 2) : kRouterOob, 0, 0);
  const uint4 g = make_uint4(t.x, t.y, t.z, t.w);
  t = __builtin_amdgcn_raw_buffer_load_b128(rs, valid ? (uint32_t)(16 * tid) : kRouterOob, 0, 0);
  const uint4 sv = make_uint4(t.x, t.y, t.z, t.w);
  t = __builtin_amdgcn_raw_buffer_load_b128(rx, valid ? (uint32_t)(16 * tid) : kRouterOob, 0, 0);
  const uint4 xv = make_uint4(t.x, t.y, t.z, t.w);
  __builtin_amdgcn_sched_barrier(0);

  const float ss = wave_sum_f32(sq8(xv, 0.f));
  if (lane == 0) red[wave] = ss;
  float sf[8];
  {
    const uint32_t w[4] = {sv.x, sv.y, sv.z, sv.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t src = a.rscale ? w[i] : 0x3f803f80u;
      const uint32_t p = pack_bf16x2(bf16lo(src) * a.c, bf16hi(src) * a.c);
      sf[2 * i] = bf16lo(p);
      sf[2 * i + 1] = bf16hi(p);
    }
  }
  __syncthreads();
  const float tot = ((red[0] + red[1]) + (red[2] + red[3])) + ((red[4] + red[5]) + (red[6] + red[7]));
  const float rr = rsqrtf(tot / (float)a.H + a.eps);
  const uint32_t w[4] = {xv.x, xv.y, xv.z, xv.w};
  uint32_t o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t n = pack_bf16x2(bf16lo(w[i]) * rr, bf16hi(w[i]) * rr);
    o[i] = pack_bf16x2(bf16lo(n) * sf[2 * i], bf16hi(n) * sf[2 * i + 1]);
  }
  const float acc = wave_sum_f32(valid ? dot8(g, make_uint4(o[0], o[1], o[2], o[3]), 0.f) : 0.f);
  if (lane == 0) part[wave] = acc;
  __syncthreads();
  if (tid == 0) {
    const float d = ((part[0] + part[1]) + (part[2] + part[3])) + ((part[4] + part[5]) + (part[6] + part[7]));
    a.logits[(size_t)m * a.E + e] = f32_to_bf16(d);
  }
}

// Prefill shape (M > 8, H % 32 == 0): the gate product on matrix cores.  A
// workgroup of 8 waves owns 16 rows and 16 experts: its waves normalise 2 rows
// each into LDS as bf16 (the same roundings as above), then each wave runs
// v_mfma_f32_16x16x32_bf16 over an eighth of K with A = the 16 normalised rows
// and B = the 16 gate rows (lane l: expert l % 16, 8 consecutive k at
// 8 (l / 16)), all of its k blocks loaded before the first product; the eight
// partial products are added in LDS.
using moe::f32x4_t;
constexpr int kRmRows = 16;
constexpr int kRmWaves = 8;
constexpr int kRmMaxKbq = 16;  // k blocks per wave: H <= 4096
constexpr size_t kRmMaxLds = 132 * 1024;

__global__ __launch_bounds__(512) void moe_router_mfma_kernel(RouterArgs a) {
  extern __shared__ uint4 xn[];  // [16][H / 8] normalised rows (bf16)
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid >> 6;
  const int hv = a.H >> 3, KB = a.H >> 5;
  const int m0 = blockIdx.y * kRmRows;
  const int e0 = blockIdx.x * 16;
  constexpr uint32_t kOob = kRouterOob;

  // rows m0 + wave + 8i, i < 2: every load first (router scale, then the two
  // rows), then sum of squares, rsqrt, bf16(bf16(x r) s) into LDS
  const __amdgpu_buffer_rsrc_t rs = buffer_rsrc(a.rscale, a.rscale ? (uint32_t)(a.H * 2) : 0u);
  const __amdgpu_buffer_rsrc_t rx = buffer_rsrc(a.x, (uint32_t)((size_t)a.M * a.H * 2));
  constexpr int kRw = kRmRows / kRmWaves;  // rows per wave
  uint4 sv[kRouterMaxJ];
#pragma unroll
  for (int j = 0; j < kRouterMaxJ; ++j) {
    const int v = lane + kWave * j;
    const u32x4_t t = __builtin_amdgcn_raw_buffer_load_b128(rs, v < hv ? (uint32_t)(16 * v) : kOob, 0, 0);
    sv[j] = make_uint4(t.x, t.y, t.z, t.w);
  }
  uint4 xv[kRw][kRouterMaxJ];
#pragma unroll
  for (int i = 0; i < kRw; ++i) {
    const int m = m0 + wave + kRmWaves * i;
#pragma unroll
    for (int j = 0; j < kRouterMaxJ; ++j) {
      const int v = lane + kWave * j;
      const u32x4_t d = __builtin_amdgcn_raw_buffer_load_b128(
          rx, (m < a.M && v < hv) ? (uint32_t)(((size_t)m * a.H + 8 * v) * 2) : kOob, 0, 0);
      xv[i][j] = make_uint4(d.x, d.y, d.z, d.w);
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  // s = bf16(router_scale * c) as packed pairs; a missing router_scale is ones
#pragma unroll
  for (int j = 0; j < kRouterMaxJ; ++j) {
    uint32_t w[4] = {sv[j].x, sv[j].y, sv[j].z, sv[j].w};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t src = a.rscale ? w[q] : 0x3f803f80u;
      w[q] = pack_bf16x2(bf16lo(src) * a.c, bf16hi(src) * a.c);
    }
    sv[j] = make_uint4(w[0], w[1], w[2], w[3]);
  }
#pragma unroll
  for (int i = 0; i < kRw; ++i) {
    const int r = wave + kRmWaves * i;
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < kRouterMaxJ; ++j) ss = sq8(xv[i][j], ss);
    const float rr = rsqrtf(wave_sum_f32(ss) / (float)a.H + a.eps);
#pragma unroll
    for (int j = 0; j < kRouterMaxJ; ++j) {
      const int v = lane + kWave * j;
      if (v < hv) {
        const uint32_t sw[4] = {sv[j].x, sv[j].y, sv[j].z, sv[j].w};
        const uint32_t w[4] = {xv[i][j].x, xv[i][j].y, xv[i][j].z, xv[i][j].w};
        uint32_t o[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const uint32_t n = pack_bf16x2(bf16lo(w[q]) * rr, bf16hi(w[q]) * rr);
          o[q] = pack_bf16x2(bf16lo(n) * bf16lo(sw[q]), bf16hi(n) * bf16hi(sw[q]));
        }
        xn[r * hv + v] = make_uint4(o[0], o[1], o[2], o[3]);
      }
    }
  }
  __syncthreads();

  // gate products: the 8 waves split K; lane l holds expert e0 + l % 16 at
  // k = 32 kb + 8 (l / 16); every k block of a wave is loaded before the first
  // product (the normalisation above has released its registers)
  const int lr = lane & 15, lq = lane >> 4;
  const int e = e0 + lr;
  const int kbq = (KB + kRmWaves - 1) / kRmWaves, kbw0 = wave * kbq;
  const __amdgpu_buffer_rsrc_t rg = buffer_rsrc(a.gate, (uint32_t)((size_t)a.E * a.H * 2));
  const uint32_t gbase = (uint32_t)(((size_t)e * a.H + 8 * lq) * 2);
  uint4 g[kRmMaxKbq];
#pragma unroll
  for (int s = 0; s < kRmMaxKbq; ++s) {
    const int kb = kbw0 + s;
    const u32x4_t d = __builtin_amdgcn_raw_buffer_load_b128(
        rg, (e < a.E && s < kbq && kb < KB) ? gbase + (uint32_t)(kb * 64) : kOob, 0, 0);
    g[s] = make_uint4(d.x, d.y, d.z, d.w);
  }
  const uint4* arow = xn + lr * hv + lq;  // A: row lr, k = 32 kb + 8 lq
  const f32x4_t zf = {0.f, 0.f, 0.f, 0.f};
  f32x4_t acc0 = zf, acc1 = zf;
#pragma unroll
  for (int s = 0; s < kRmMaxKbq; ++s) {
    const int kb = kbw0 + s;
    if (s < kbq && kb < KB) {
      const uint4 A = arow[4 * kb];
      if (s & 1) acc1 = moe::mfma_bf16(A, g[s], acc1);
      else acc0 = moe::mfma_bf16(A, g[s], acc0);
    }
  }
  // D: row 4 lq + j, expert lr; the 8 waves' K ranges summed in a fixed order
  float* red = (float*)(xn + kRmRows * hv);  // [8 waves][16 rows][16 experts]
#pragma unroll
  for (int j = 0; j < 4; ++j) red[(wave * 16 + 4 * lq + j) * 16 + lr] = acc0[j] + acc1[j];
  __syncthreads();
  if (tid < 256) {
    const int r = tid >> 4, c = tid & 15;
    const int m = m0 + r, ee = e0 + c;
    if (m < a.M && ee < a.E) {
      float v = 0.f;
#pragma unroll
      for (int w2 = 0; w2 < kRmWaves; ++w2) v += red[(w2 * 16 + r) * 16 + c];
      a.logits[(size_t)m * a.E + ee] = f32_to_bf16(v);
    }
  }
}

int launch_router_mfma(const RouterArgs& a, hipStream_t stream) {
  static bool attr_set[64];
  int dev = 0;
  hipError_t e0 = hipGetDevice(&dev);
  if (e0 != hipSuccess) return hip_fail(e0, "hipGetDevice");
  if (dev >= 0 && dev < 64 && !attr_set[dev]) {
    e0 = hipFuncSetAttribute((const void*)moe_router_mfma_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                             (int)kRmMaxLds);
    if (e0 != hipSuccess) return hip_fail(e0, "hipFuncSetAttribute(max dynamic LDS)");
    attr_set[dev] = true;
  }
  const dim3 grid((unsigned)((a.E + 15) / 16), (unsigned)((a.M + kRmRows - 1) / kRmRows));
  hipLaunchKernelGGL(moe_router_mfma_kernel, grid, dim3(kRmWaves * kWave), (size_t)kRmRows * a.H * 2 + kRmWaves * 256 * 4,
                     stream, a);
  return GI_OK;
}

template <int EPW, int J, int R>
void launch_router_variant(const RouterArgs& a, hipStream_t stream) {
  const dim3 grid((unsigned)((a.E + kRouterWaves * EPW - 1) / (kRouterWaves * EPW)),
                  (unsigned)((a.M + R - 1) / R));
  const size_t lds = (size_t)R * a.H * 2;
  hipLaunchKernelGGL((moe_router_kernel<EPW, J, R>), grid, dim3(kRouterWaves * kWave), lds, stream, a);
}

template <int EPW, int R>
void launch_router_j(const RouterArgs& a, hipStream_t stream) {
  const int j = (a.H / 8 + kWave - 1) / kWave;  // 16-byte gate vectors per lane
  if (j <= 2) launch_router_variant<EPW, 2, R>(a, stream);
  else if (j <= 4) launch_router_variant<EPW, 4, R>(a, stream);
  else if (j <= 6) launch_router_variant<EPW, 6, R>(a, stream);
  else launch_router_variant<EPW, 8, R>(a, stream);
}

}  // namespace

int launch_moe_router(const void* x, const void* router_scale, const void* gate, void* logits, int M,
                      int H, int E, float eps, hipStream_t stream) {
  if (M < 0 || H <= 0 || E <= 0) return fail(GI_ERR_INVALID_ARG, "moe_router: M >= 0, H > 0, E > 0 required");
  if (H % 8 != 0 || H > 8 * kWave * kRouterMaxJ)
    return fail(GI_ERR_UNSUPPORTED, "moe_router: H must be a multiple of 8 and at most 4096");
  if (E > 65536) return fail(GI_ERR_UNSUPPORTED, "moe_router: at most 65536 experts");
  if (!(eps >= 0.f)) return fail(GI_ERR_INVALID_ARG, "moe_router: eps must be >= 0");
  if (M == 0) return GI_OK;
  if (!x || !gate || !logits) return fail(GI_ERR_INVALID_ARG, "moe_router: null pointer");
  if ((size_t)M * H > 0x3fffffffu || (size_t)M * E > 0x7fffffffu)
    return fail(GI_ERR_UNSUPPORTED, "moe_router: input too large for 32-bit offsets");
  RouterArgs a{};
  a.x = (const uint16_t*)x;
  a.rscale = (const uint16_t*)router_scale;
  a.gate = (const uint16_t*)gate;
  a.logits = (uint16_t*)logits;
  a.M = M;
  a.H = H;
  a.E = E;
  a.eps = eps;
  a.c = (float)std::pow((double)H, -0.5);  // hidden_size ** -0.5 as a float operand
  if (M > 8 && H % 32 == 0) {
    const int st = launch_router_mfma(a, stream);
    if (st != GI_OK) return st;
  } else if (M > 64) launch_router_j<4, 8>(a, stream);
  else if (M > 8) launch_router_j<1, 8>(a, stream);
  else hipLaunchKernelGGL(moe_router_rows_kernel, dim3((unsigned)E, (unsigned)M), dim3(512), 0, stream, a);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? GI_OK : hip_fail(e, "moe_router launch");
}

}  // namespace gi
