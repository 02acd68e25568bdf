// Device code shared by the fused-MoE kernels: the router (top-k + softmax
// per token, one wave per token) and the bf16 matrix-core helpers used with
// unpacked int4 weights.
//
// Routing restates gemmainfer/models/gemma.py:77-80 (topk of the router
// logits, softmax in fp32, times expert_scale).  The argument struct `A` of
// route_token provides logits, logits_dtype, E, top_k and expert_scale.
#pragma once

#include "../../include/gemmainfer_amd.h"
#include "gi_common.h"

namespace gi {
namespace moe {

constexpr int kRouteMaxExperts = 1024;

// ---------------------------------------------------------------------------
// routing
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t orderable_key(float f) {
  const uint32_t u = __float_as_uint(f);
  if (f != f) return 0xffffffffu;  // NaN ranks above every number
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float key_value(uint32_t k) {
  if (k == 0xffffffffu) return __uint_as_float(0x7fc00000u);
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

__device__ __forceinline__ uint32_t umax(uint32_t a, uint32_t b) { return a > b ? a : b; }

// Maximum over the wave: DPP inside each 16-lane row (quad swaps, half-row
// and row mirrors), then the four row results through readlane.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  v = umax(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false));   // quad_perm [1,0,3,2]
  v = umax(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, false));   // quad_perm [2,3,0,1]
  v = umax(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x141, 0xF, 0xF, false));  // row_half_mirror
  v = umax(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x140, 0xF, 0xF, false));  // row_mirror
  const uint32_t r0 = __builtin_amdgcn_readlane(v, 0), r1 = __builtin_amdgcn_readlane(v, 16);
  const uint32_t r2 = __builtin_amdgcn_readlane(v, 32), r3 = __builtin_amdgcn_readlane(v, 48);
  return umax(umax(r0, r1), umax(r2, r3));
}

// Top-k + softmax of token t by one wave (gemma.py:77-80).  Lane l holds the
// keys of experts l, l+64, ...  Each round takes the wave maximum of the keys
// and, among equal keys, the lowest expert index (first set ballot bit in the
// lowest register), then retires it (key 0; every real value has a non-zero
// key).  Lane r < top_k ends with the r-th expert and its weight.
template <int VPL, class A>
__device__ __forceinline__ void route_token(const A& a, int t, int lane, int* idx_out,
                                            float* w_out) {
  // All VPL loads go out before any is used (clamped indices, no branch
  // around a load: a load under a per-lane condition is waited for at the
  // end of the condition), one dtype path per launch.
  uint32_t keys[VPL];
  float f[VPL], es[VPL];
  const size_t base = (size_t)t * a.E;
  // expert_scale goes out with the logits, so the winners' scales need no
  // load of their own
#pragma unroll
  for (int v = 0; v < VPL; ++v) es[v] = a.expert_scale ? a.expert_scale[min(lane + v * kWave, a.E - 1)] : 1.f;
  if (a.logits_dtype == GI_DTYPE_BF16) {
    const uint16_t* row = (const uint16_t*)a.logits + base;
#pragma unroll
    for (int v = 0; v < VPL; ++v) f[v] = bf16_to_f32(row[min(lane + v * kWave, a.E - 1)]);
  } else {
    const float* row = (const float*)a.logits + base;
#pragma unroll
    for (int v = 0; v < VPL; ++v) f[v] = row[min(lane + v * kWave, a.E - 1)];
  }
#pragma unroll
  for (int v = 0; v < VPL; ++v) {
    const int e = lane + v * kWave;
    keys[v] = e < a.E ? orderable_key(f[v]) : 0u;
  }
  int my_idx = 0;
  float my_val = 0.f, my_es = 1.f;
  for (int r = 0; r < a.top_k; ++r) {
    uint32_t lm = keys[0];
#pragma unroll
    for (int v = 1; v < VPL; ++v) lm = umax(lm, keys[v]);
    const uint32_t m = wave_max_u32(lm);
    int win = -1;
#pragma unroll
    for (int v = 0; v < VPL; ++v) {
      const unsigned long long b = __ballot(keys[v] == m);
      if (win < 0 && b) win = v * kWave + (int)__builtin_ctzll(b);
    }
#pragma unroll
    for (int v = 0; v < VPL; ++v)
      if (lane + v * kWave == win) keys[v] = 0u;
    float ew = 0.f;
#pragma unroll
    for (int v = 0; v < VPL; ++v)
      if ((win >> 6) == v) ew = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(es[v]), win & (kWave - 1)));
    if (lane == r) {
      my_idx = win;
      my_val = key_value(m);
      my_es = ew;
    }
  }
  const float vmax = __shfl(my_val, 0, kWave);
  const float ex = lane < a.top_k ? expf(my_val - vmax) : 0.f;
  float sum = ex;
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) sum += __shfl_xor(sum, off, kWave);
  if (lane < a.top_k) {
    float p = ex / sum;
    p *= my_es;
    idx_out[lane] = my_idx;
    w_out[lane] = p;
  }
}

template <class A>
__device__ __forceinline__ void route_token_any(const A& a, int t, int lane, int* idx_out,
                                                float* w_out) {
  if (a.E <= 2 * kWave) route_token<2, A>(a, t, lane, idx_out, w_out);
  else if (a.E <= 4 * kWave) route_token<4, A>(a, t, lane, idx_out, w_out);
  else route_token<kRouteMaxExperts / kWave, A>(a, t, lane, idx_out, w_out);
}

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr uint32_t kNeg136Pair = 0xC308C308u;  // bf16 -136, twice

__device__ __forceinline__ f32x4_t mfma_bf16(uint4 a, uint4 b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}
// 8 bf16 values in the k order of an unpacked word: (0,4) (2,6) (1,5) (3,7)
__device__ __forceinline__ uint4 mfma_k_order(uint4 d) {
  const uint4 p = pair_permute(d);
  return make_uint4(p.x, p.z, p.y, p.w);
}
__device__ __forceinline__ uint4 q4_operand(uint32_t w, uint32_t m43) {
  const Q4Pairs q = unpack_q4(w, m43);
  return make_uint4(q.p0, q.p1, q.p2, q.p3);
}
// position of element p (0..7) of a packed row in that order
__device__ __forceinline__ int mfma_k_pos(int p) { return (p & 1) * 4 + (p & 2) + (p >> 2); }

}  // namespace moe
}  // namespace gi
