// Chunked-prefill replacement: the fused W4A16 MoE for many token rows as a
// sorted-by-expert grouped GEMM on the matrix cores.
//
// Reference behaviour restated (paths relative to the GemmaInfer repo): the
// reference runs prefill through fused_batched_moe on 8-row slices
// (gemmainfer/models/gemma.py:99-112 -> csrc/marlin.cu:612-702), so every
// slice re-reads each expert it touches (~26x the ideal weight bytes at 512
// rows).  Here every (token, slot) pair is grouped by expert once and each
// active expert's weights stream through the GPU once:
//
//   align    one workgroup: per-expert counts, offsets, the pairs of each
//            expert (pos -> pair) and the inverse map (pair -> pos); the
//            routing weights rounded to bf16 (marlin.cu:631-636)
//   gate/up  grid (I/32 column tiles, E): 16-token row tiles of the expert's
//            pairs (A = gathered x rows) times the unpacked int4 words (B),
//            v_mfma_f32_16x16x32_bf16; k split over the 8 waves, summed in
//            wave order; act = bf16(gelu_tanh(gate) * up) (marlin.cu:414-423)
//   down     grid (H/64 column units, E): the same over the act rows, fp32
//            results per pair
//   combine  one workgroup per token: out[t] (+)= sum over its slots in slot
//            order of w * y, one bf16 rounding (the reference adds bf16
//            atomics, marlin.cu:583; the order here is fixed)
//
// The int4 words enter the products as bf16 16 + q (byte permutes) with one
// more product against a constant -24 operand per 32-k block for the offset,
// as in the decode kernel; scales apply per group (y += s * (D + Db)).  Rows
// of a pair's result do not depend on where the pair sits in its tile, so the
// atomically assigned positions leave the output deterministic.

#include "../../include/gemmainfer_amd.h"
#include "gi_common.h"
#include "gi_internal.h"
#include "moe_shared.h"

namespace gi {

namespace {

using moe::f32x4_t;
constexpr int kPThreads = 512;
constexpr int kPWaves = kPThreads / kWave;
constexpr int kPRT = 2;          // 16-token row tiles per pass
constexpr int kPMaxKbw = 12;     // gate/up k blocks per wave: H <= 3072
constexpr int kPMaxKbwD = 3;     // down k blocks per wave: I <= 768
constexpr int kAlignThreads = 1024;
constexpr uint32_t kOob = 0xFFFFFFF0u;

struct PfArgs {
  const uint16_t* x;
  const int32_t* gu;
  const uint16_t* gus;
  const int32_t* dn;
  const uint16_t* dns;
  const int* offsets;  // [E + 1]
  const int* order;    // [P] pair at each position
  uint16_t* act;       // [P][I] bf16, positions in expert order
  float* y;            // [P][H] fp32
  int M, H, I, E, top_k, Ggu, Gd, gsh;  // group size = 32 << gsh
  uint32_t x_bytes, gu_bytes, gu_total, dn_bytes, dn_total, act_bytes;
};

// ---------------------------------------------------------------------------
// align
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kAlignThreads) void prefill_align_kernel(
    const void* idx, int idx_is64, const void* w, int w_dtype, int P, int E, int* offsets, int* order,
    int* posmap, float* wts) {
  __shared__ int cnt[1024];
  __shared__ int fill[1024];
  __shared__ int wsum[kAlignThreads / kWave];
  const int tid = threadIdx.x;
  for (int e = tid; e < E; e += kAlignThreads) {
    cnt[e] = 0;
    fill[e] = 0;
  }
  __syncthreads();
  for (int p = tid; p < P; p += kAlignThreads) {
    const int e = load_expert_id(idx, idx_is64, p);
    if (e >= 0 && e < E) atomicAdd(&cnt[e], 1);
  }
  __syncthreads();
  // exclusive scan of the counts (E <= 1024: one expert per thread)
  const int lane = tid & (kWave - 1), wave = tid >> 6;
  const int c = tid < E ? cnt[tid] : 0;
  int incl = c;
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const int v = __shfl_up(incl, off, kWave);
    if (lane >= off) incl += v;
  }
  if (lane == kWave - 1) wsum[wave] = incl;
  __syncthreads();
  int base = 0;
  for (int w2 = 0; w2 < wave; ++w2) base += wsum[w2];
  const int excl = base + incl - c;
  if (tid < E) {
    offsets[tid] = excl;
    cnt[tid] = excl;
  }
  if (tid == E - 1) offsets[E] = excl + c;
  __syncthreads();
  for (int p = tid; p < P; p += kAlignThreads) {
    const int e = load_expert_id(idx, idx_is64, p);
    int pos = -1;
    if (e >= 0 && e < E) {
      pos = cnt[e] + atomicAdd(&fill[e], 1);
      order[pos] = p;
    }
    posmap[p] = pos;
    wts[p] = load_weight_as_bf16(w, w_dtype, p);
  }
}

// ---------------------------------------------------------------------------
// gate/up
// ---------------------------------------------------------------------------
// x operand of one lane for row tile rt at k block kb: 16 bytes of its
// token's row (zeros past the expert's pairs: offset past the resource).
__device__ __forceinline__ uint4 x_operand(__amdgpu_buffer_rsrc_t rx, uint32_t row_off, int kb, int lq) {
  const uint32_t off = row_off == kOob ? kOob : row_off + (uint32_t)(32 * kb + 8 * lq) * 2u;
  const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(rx, off, 0, 0);
  return moe::mfma_k_order(make_uint4(v.x, v.y, v.z, v.w));
}

template <int KBW>
__global__ __launch_bounds__(kPThreads) void prefill_gu_kernel(PfArgs a) {
  __shared__ float red[kPWaves][16][64];
  extern __shared__ uint2 gsc[];  // [Ggu][16]: scales of the lane's 4 columns (8 gate | 8 up lanes)
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid >> 6;
  const int lq = lane >> 4, lr = lane & 15;
  const int tile = blockIdx.x, e = blockIdx.y;
  const int off_e = a.offsets[e], n_e = a.offsets[e + 1] - off_e;
  if (n_e <= 0) return;
  const int twoI = 2 * a.I;
  const int KB = a.H >> 5;
  const int kb0 = wave * KB / kPWaves, nkb = (wave + 1) * KB / kPWaves - kb0;
  const int col = (lr < 8 ? 0 : a.I) + 32 * tile + 4 * (lr & 7);
  for (int i = tid; i < a.Ggu * 16; i += kPThreads) {
    const int g = i >> 4, l = i & 15;
    const int c2 = (l < 8 ? 0 : a.I) + 32 * tile + 4 * (l & 7);
    gsc[i] = *(const uint2*)(a.gus + ((size_t)e * a.Ggu + g) * twoI + c2);
  }
  __syncthreads();
  const __amdgpu_buffer_rsrc_t rw = buffer_rsrc(a.gu, a.gu_total);
  const __amdgpu_buffer_rsrc_t rx = buffer_rsrc(a.x, a.x_bytes);
  const uint32_t mq = q4_magic();
  const f32x4_t zf = {0.f, 0.f, 0.f, 0.f};
  const uint4 bc = make_uint4(moe::kQ4BiasPair, moe::kQ4BiasPair, moe::kQ4BiasPair, moe::kQ4BiasPair);
  const int kbpg = 1 << a.gsh;
  for (int base = 0; base < n_e; base += 16 * kPRT) {
    // this wave's weight words (a fixed count: past its k blocks, zeros)
    uint4 w[KBW];
#pragma unroll
    for (int j = 0; j < KBW; ++j) {
      const uint32_t row = 4 * (kb0 + j) + lq;
      const uint32_t off = j < nkb ? (row * twoI + col) * 4u : kOob;
      const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(rw, off, e * a.gu_bytes, 2);
      w[j] = make_uint4(v.x, v.y, v.z, v.w);
    }
    // the lanes' token rows of each row tile
    uint32_t xoff[kPRT];
#pragma unroll
    for (int rt = 0; rt < kPRT; ++rt) {
      const int j = base + 16 * rt + lr;
      xoff[rt] = j < n_e ? (uint32_t)(a.order[off_e + j] / a.top_k) * (uint32_t)a.H * 2u : kOob;
    }
    f32x4_t y[kPRT][4], D[kPRT][4], Db[kPRT];
#pragma unroll
    for (int rt = 0; rt < kPRT; ++rt) {
      Db[rt] = zf;
#pragma unroll
      for (int q = 0; q < 4; ++q) y[rt][q] = D[rt][q] = zf;
    }
    uint4 A[kPRT];
#pragma unroll
    for (int rt = 0; rt < kPRT; ++rt) A[rt] = x_operand(rx, xoff[rt], kb0, lq);
#pragma unroll
    for (int j = 0; j < KBW; ++j) {
      // the next k block's x goes out unconditionally (zeros past the
      // wave's k blocks), so that every wait keeps an exact count
      uint4 An[kPRT];
#pragma unroll
      for (int rt = 0; rt < kPRT; ++rt) An[rt] = x_operand(rx, j + 1 < nkb ? xoff[rt] : kOob, kb0 + j + 1, lq);
      if (j < nkb) {
        const int kb = kb0 + j;
        const uint4 q0 = moe::q4_operand(w[j].x, mq), q1 = moe::q4_operand(w[j].y, mq);
        const uint4 q2 = moe::q4_operand(w[j].z, mq), q3 = moe::q4_operand(w[j].w, mq);
#pragma unroll
        for (int rt = 0; rt < kPRT; ++rt) {
          D[rt][0] = moe::mfma_bf16(A[rt], q0, D[rt][0]);
          D[rt][1] = moe::mfma_bf16(A[rt], q1, D[rt][1]);
          D[rt][2] = moe::mfma_bf16(A[rt], q2, D[rt][2]);
          D[rt][3] = moe::mfma_bf16(A[rt], q3, D[rt][3]);
          Db[rt] = moe::mfma_bf16(A[rt], bc, Db[rt]);
        }
        if (((kb + 1) & (kbpg - 1)) == 0 || j == nkb - 1) {
          const int g = kb >> a.gsh;
          if (g < a.Ggu) {
            const uint2 sv = gsc[g * 16 + lr];
            const float sc[4] = {bf16lo(sv.x), bf16hi(sv.x), bf16lo(sv.y), bf16hi(sv.y)};
#pragma unroll
            for (int rt = 0; rt < kPRT; ++rt)
#pragma unroll
              for (int q = 0; q < 4; ++q)
#pragma unroll
                for (int jj = 0; jj < 4; ++jj) y[rt][q][jj] += sc[q] * (D[rt][q][jj] + Db[rt][jj]);
          }
#pragma unroll
          for (int rt = 0; rt < kPRT; ++rt) {
            Db[rt] = zf;
#pragma unroll
            for (int q = 0; q < 4; ++q) D[rt][q] = zf;
          }
        }
      }
#pragma unroll
      for (int rt = 0; rt < kPRT; ++rt) A[rt] = An[rt];
    }
    // sums over the waves in wave order, then the activation, per row tile
#pragma unroll
    for (int rt = 0; rt < kPRT; ++rt) {
      __syncthreads();
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int jj = 0; jj < 4; ++jj)
          red[wave][4 * lq + jj][(lr < 8 ? 0 : 32) + 4 * (lr & 7) + q] = y[rt][q][jj];
      __syncthreads();
      const int t = tid >> 5, ci = tid & 31;  // 16 tokens x 32 columns
      const int j = base + 16 * rt + t;
      if (j < n_e) {
        float g = 0.f, u = 0.f;
#pragma unroll
        for (int w2 = 0; w2 < kPWaves; ++w2) {
          g += red[w2][t][ci];
          u += red[w2][t][32 + ci];
        }
        a.act[(size_t)(off_e + j) * a.I + 32 * tile + ci] = f32_to_bf16(gelu_tanh(g) * u);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// down
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kPThreads) void prefill_down_kernel(PfArgs a) {
  __shared__ float red[kPWaves][16][64];
  extern __shared__ uint2 dsc[];  // [Gd][16]: scales of the lane's 4 columns
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid >> 6;
  const int lq = lane >> 4, lr = lane & 15;
  const int unit = blockIdx.x, e = blockIdx.y;
  const int off_e = a.offsets[e], n_e = a.offsets[e + 1] - off_e;
  if (n_e <= 0) return;
  const int KB = a.I >> 5;
  const int kb0 = wave * KB / kPWaves, nkb = (wave + 1) * KB / kPWaves - kb0;
  const int col = 64 * unit + 4 * lr;
  for (int i = tid; i < a.Gd * 16; i += kPThreads) {
    const int g = i >> 4, l = i & 15;
    dsc[i] = *(const uint2*)(a.dns + ((size_t)e * a.Gd + g) * a.H + 64 * unit + 4 * l);
  }
  __syncthreads();
  const __amdgpu_buffer_rsrc_t rw = buffer_rsrc(a.dn, a.dn_total);
  const __amdgpu_buffer_rsrc_t ra = buffer_rsrc(a.act, a.act_bytes);
  const uint32_t mq = q4_magic();
  const f32x4_t zf = {0.f, 0.f, 0.f, 0.f};
  const uint4 bc = make_uint4(moe::kQ4BiasPair, moe::kQ4BiasPair, moe::kQ4BiasPair, moe::kQ4BiasPair);
  const int kbpg = 1 << a.gsh;
  for (int base = 0; base < n_e; base += 16 * kPRT) {
    uint4 w[kPMaxKbwD];
#pragma unroll
    for (int j = 0; j < kPMaxKbwD; ++j) {
      const uint32_t row = 4 * (kb0 + j) + lq;
      const uint32_t off = j < nkb ? (row * (uint32_t)a.H + col) * 4u : kOob;
      const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(rw, off, e * a.dn_bytes, 2);
      w[j] = make_uint4(v.x, v.y, v.z, v.w);
    }
    uint4 A[kPMaxKbwD][kPRT];
#pragma unroll
    for (int rt = 0; rt < kPRT; ++rt) {
      const int j = base + 16 * rt + lr;
      const uint32_t roff = j < n_e ? (uint32_t)(off_e + j) * (uint32_t)a.I * 2u : kOob;
#pragma unroll
      for (int jk = 0; jk < kPMaxKbwD; ++jk) A[jk][rt] = x_operand(ra, jk < nkb ? roff : kOob, kb0 + jk, lq);
    }
    f32x4_t y[kPRT][4], D[kPRT][4], Db[kPRT];
#pragma unroll
    for (int rt = 0; rt < kPRT; ++rt) {
      Db[rt] = zf;
#pragma unroll
      for (int q = 0; q < 4; ++q) y[rt][q] = D[rt][q] = zf;
    }
#pragma unroll
    for (int j = 0; j < kPMaxKbwD; ++j) {
      if (j < nkb) {
        const int kb = kb0 + j;
        const uint4 q0 = moe::q4_operand(w[j].x, mq), q1 = moe::q4_operand(w[j].y, mq);
        const uint4 q2 = moe::q4_operand(w[j].z, mq), q3 = moe::q4_operand(w[j].w, mq);
#pragma unroll
        for (int rt = 0; rt < kPRT; ++rt) {
          D[rt][0] = moe::mfma_bf16(A[j][rt], q0, D[rt][0]);
          D[rt][1] = moe::mfma_bf16(A[j][rt], q1, D[rt][1]);
          D[rt][2] = moe::mfma_bf16(A[j][rt], q2, D[rt][2]);
          D[rt][3] = moe::mfma_bf16(A[j][rt], q3, D[rt][3]);
          Db[rt] = moe::mfma_bf16(A[j][rt], bc, Db[rt]);
        }
        if (((kb + 1) & (kbpg - 1)) == 0 || j == nkb - 1) {
          const int g = kb >> a.gsh;
          if (g < a.Gd) {
            const uint2 sv = dsc[g * 16 + lr];
            const float sc[4] = {bf16lo(sv.x), bf16hi(sv.x), bf16lo(sv.y), bf16hi(sv.y)};
#pragma unroll
            for (int rt = 0; rt < kPRT; ++rt)
#pragma unroll
              for (int q = 0; q < 4; ++q)
#pragma unroll
                for (int jj = 0; jj < 4; ++jj) y[rt][q][jj] += sc[q] * (D[rt][q][jj] + Db[rt][jj]);
          }
#pragma unroll
          for (int rt = 0; rt < kPRT; ++rt) {
            Db[rt] = zf;
#pragma unroll
            for (int q = 0; q < 4; ++q) D[rt][q] = zf;
          }
        }
      }
    }
#pragma unroll
    for (int rt = 0; rt < kPRT; ++rt) {
      __syncthreads();
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) red[wave][4 * lq + jj][4 * lr + q] = y[rt][q][jj];
      __syncthreads();
      for (int i = tid; i < 16 * 64; i += kPThreads) {
        const int t = i >> 6, c = i & 63;
        const int j = base + 16 * rt + t;
        if (j < n_e) {
          float s = 0.f;
#pragma unroll
          for (int w2 = 0; w2 < kPWaves; ++w2) s += red[w2][t][c];
          a.y[(size_t)(off_e + j) * a.H + 64 * unit + c] = s;
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// combine: out[t] (+)= sum over slots, in slot order, of w * y[pos]
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void prefill_combine_kernel(const float* y, const int* posmap, const float* wts,
                                                              uint16_t* out, int H, int top_k, int overwrite) {
  const int t = blockIdx.x;
  for (int c = threadIdx.x * 4; c < H; c += 256 * 4) {
    float4 s = overwrite ? make_float4(0.f, 0.f, 0.f, 0.f)
                         : make_float4(bf16_to_f32(out[(size_t)t * H + c]), bf16_to_f32(out[(size_t)t * H + c + 1]),
                                       bf16_to_f32(out[(size_t)t * H + c + 2]), bf16_to_f32(out[(size_t)t * H + c + 3]));
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int k = 0; k < top_k; ++k) {
      const int p = t * top_k + k;
      const int pos = posmap[p];
      if (pos < 0) continue;
      const float wv = wts[p];
      const float4 v = *(const float4*)(y + (size_t)pos * H + c);
      acc.x += wv * v.x;
      acc.y += wv * v.y;
      acc.z += wv * v.z;
      acc.w += wv * v.w;
    }
    s.x += acc.x;
    s.y += acc.y;
    s.z += acc.z;
    s.w += acc.w;
    const uint32_t lo = (uint32_t)f32_to_bf16(s.x) | ((uint32_t)f32_to_bf16(s.y) << 16);
    const uint32_t hi = (uint32_t)f32_to_bf16(s.z) | ((uint32_t)f32_to_bf16(s.w) << 16);
    *(uint2*)(out + (size_t)t * H + c) = make_uint2(lo, hi);
  }
}

constexpr size_t kPAlign = 256;
inline size_t pround(size_t v) { return (v + kPAlign - 1) / kPAlign * kPAlign; }

struct PfLayout {
  size_t idx, w, offsets, order, posmap, wts, act, y, total;
};
PfLayout pf_layout(int M, int top_k, int H, int I, int E) {
  const size_t P = (size_t)M * top_k;
  PfLayout l;
  l.idx = 0;
  l.w = pround(l.idx + P * 4);
  l.offsets = pround(l.w + P * 2);
  l.order = pround(l.offsets + (size_t)(E + 1) * 4);
  l.posmap = pround(l.order + P * 4);
  l.wts = pround(l.posmap + P * 4);
  l.act = pround(l.wts + P * 4);
  l.y = pround(l.act + P * I * 2);
  l.total = pround(l.y + P * H * 4);
  return l;
}

int log2_exact(int v) {
  int s = 0;
  while ((1 << s) < v) ++s;
  return (1 << s) == v ? s : -1;
}

}  // namespace

bool moe_prefill_supported(const MoeHostArgs& h) {
  if (h.M < kPrefillMinRows) return false;
  if (h.H % 64 || h.I % 32 || h.H > 32 * kPWaves * kPMaxKbw || h.I > 32 * kPWaves * kPMaxKbwD) return false;
  if (h.gs % 32 || log2_exact(h.gs / 32) < 0) return false;
  if (h.top_k > 64 || h.E > 1024) return false;
  const long long P = (long long)h.M * h.top_k;
  // 32-bit buffer offsets
  if ((long long)h.E * (h.H / 8) * 2 * h.I * 4 >= (1LL << 32)) return false;
  if ((long long)h.E * (h.I / 8) * h.H * 4 >= (1LL << 32)) return false;
  if ((long long)h.M * h.H * 2 >= (1LL << 32) || P * h.I * 2 >= (1LL << 32)) return false;
  return P <= (1 << 20);
}

size_t moe_prefill_workspace_bytes(int M, int top_k, int H, int I, int E) {
  return pf_layout(M, top_k, H, I, E).total;
}

int launch_moe_prefill(const MoeHostArgs& h, void* workspace, size_t ws_bytes) {
  const PfLayout L = pf_layout(h.M, h.top_k, h.H, h.I, h.E);
  if (!workspace || ws_bytes < L.total)
    return fail(GI_ERR_WORKSPACE, "fused MoE: workspace missing or smaller than gi_fused_moe_workspace_bytes()");
  char* ws = (char*)workspace;
  const int P = h.M * h.top_k;
  const void* idx = h.idx;
  int idx_is64 = h.idx_is64;
  const void* w = h.w;
  int w_dtype = h.w_dtype;
  if (h.logits) {
    // routing into the caller's report buffers when given, else the workspace
    int32_t* ridx = h.out_idx ? h.out_idx : (int32_t*)(ws + L.idx);
    void* rw = h.out_w ? h.out_w : (void*)(ws + L.w);
    const int st = launch_route(h.logits, h.logits_dtype, h.expert_scale, h.M, h.E, h.top_k, ridx, rw,
                                GI_DTYPE_BF16, h.stream);
    if (st != GI_OK) return st;
    idx = ridx;
    idx_is64 = 0;
    w = rw;
    w_dtype = GI_DTYPE_BF16;
  }
  int* offsets = (int*)(ws + L.offsets);
  int* order = (int*)(ws + L.order);
  int* posmap = (int*)(ws + L.posmap);
  float* wts = (float*)(ws + L.wts);
  hipLaunchKernelGGL(prefill_align_kernel, dim3(1), dim3(kAlignThreads), 0, h.stream, idx, idx_is64, w, w_dtype,
                     P, h.E, offsets, order, posmap, wts);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return hip_fail(e, "prefill align launch");

  PfArgs k{};
  k.x = (const uint16_t*)h.x;
  k.gu = h.gu_packed;
  k.gus = (const uint16_t*)h.gu_scales;
  k.dn = h.d_packed;
  k.dns = (const uint16_t*)h.d_scales;
  k.offsets = offsets;
  k.order = order;
  k.act = (uint16_t*)(ws + L.act);
  k.y = (float*)(ws + L.y);
  k.M = h.M;
  k.H = h.H;
  k.I = h.I;
  k.E = h.E;
  k.top_k = h.top_k;
  k.Ggu = h.Ggu;
  k.Gd = h.Gd;
  k.gsh = log2_exact(h.gs / 32);
  k.x_bytes = (uint32_t)((size_t)h.M * h.H * 2);
  k.gu_bytes = (uint32_t)((size_t)(h.H / 8) * 2 * h.I * 4);
  k.gu_total = (uint32_t)((size_t)h.E * k.gu_bytes);
  k.dn_bytes = (uint32_t)((size_t)(h.I / 8) * h.H * 4);
  k.dn_total = (uint32_t)((size_t)h.E * k.dn_bytes);
  k.act_bytes = (uint32_t)((size_t)P * h.I * 2);
  const int kbw = (h.H / 32 + kPWaves - 1) / kPWaves;
  const size_t gl = (size_t)h.Ggu * 16 * sizeof(uint2), dl = (size_t)h.Gd * 16 * sizeof(uint2);
  const dim3 ggrid(h.I / 32, h.E), dgrid(h.H / 64, h.E);
  if (kbw <= 4) hipLaunchKernelGGL(prefill_gu_kernel<4>, ggrid, dim3(kPThreads), gl, h.stream, k);
  else if (kbw <= 8) hipLaunchKernelGGL(prefill_gu_kernel<8>, ggrid, dim3(kPThreads), gl, h.stream, k);
  else hipLaunchKernelGGL(prefill_gu_kernel<kPMaxKbw>, ggrid, dim3(kPThreads), gl, h.stream, k);
  e = hipGetLastError();
  if (e != hipSuccess) return hip_fail(e, "prefill gate/up launch");
  hipLaunchKernelGGL(prefill_down_kernel, dgrid, dim3(kPThreads), dl, h.stream, k);
  e = hipGetLastError();
  if (e != hipSuccess) return hip_fail(e, "prefill down launch");
  hipLaunchKernelGGL(prefill_combine_kernel, dim3(h.M), dim3(256), 0, h.stream, k.y, posmap, wts,
                     (uint16_t*)h.out, h.H, h.top_k, h.overwrite);
  e = hipGetLastError();
  if (e != hipSuccess) return hip_fail(e, "prefill combine launch");
  return GI_OK;
}

}  // namespace gi
