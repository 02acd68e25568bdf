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

__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) {
  v = min(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false));
  v = min(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, false));
  v = min(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x141, 0xF, 0xF, false));
  v = min(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x140, 0xF, 0xF, false));
  const uint32_t r0 = __builtin_amdgcn_readlane(v, 0), r1 = __builtin_amdgcn_readlane(v, 16);
  const uint32_t r2 = __builtin_amdgcn_readlane(v, 32), r3 = __builtin_amdgcn_readlane(v, 48);
  return min(min(r0, r1), min(r2, r3));
}

// Router inputs of one token held by one wave: lane l has experts l + 64v.
template <int VPL>
struct RouteIn {
  uint32_t raw[VPL];  // logit bits: bf16 (zero-extended) or fp32
  uint32_t es[VPL];   // expert_scale bits (zero without a scale tensor)
};

// The loads of token t's logits and of the expert scales, issued before any
// other work so that later loads queue behind them; past E (or without a
// scale tensor) the buffer resource returns zeros without a memory access.
template <int VPL, class A>
__device__ __forceinline__ void route_issue(const A& a, int t, int lane, RouteIn<VPL>& r) {
  const bool bf = a.logits_dtype == GI_DTYPE_BF16;
  const uint32_t rowb = (uint32_t)a.E * (bf ? 2u : 4u);
  const __amdgpu_buffer_rsrc_t rl = buffer_rsrc((const char*)a.logits + (size_t)t * rowb, rowb);
  const __amdgpu_buffer_rsrc_t rs = buffer_rsrc(a.expert_scale, a.expert_scale ? (uint32_t)a.E * 4u : 0u);
  if (bf) {
#pragma unroll
    for (int v = 0; v < VPL; ++v)
      r.raw[v] = __builtin_amdgcn_raw_buffer_load_b16(rl, (uint32_t)(lane + v * kWave) * 2u, 0, 0);
  } else {
#pragma unroll
    for (int v = 0; v < VPL; ++v)
      r.raw[v] = __builtin_amdgcn_raw_buffer_load_b32(rl, (uint32_t)(lane + v * kWave) * 4u, 0, 0);
  }
#pragma unroll
  for (int v = 0; v < VPL; ++v)
    r.es[v] = __builtin_amdgcn_raw_buffer_load_b32(rs, (uint32_t)(lane + v * kWave) * 4u, 0, 0);
}

// Softmax over the selected top-k (gemma.py:78-80), one wave: lane r < top_k
// holds the r-th expert, its key and its expert scale; writes idx_out[r] and
// w_out[r] = softmax_fp32(values)[r] * expert_scale.
template <class A>
__device__ __forceinline__ void route_softmax(const A& a, int lane, int my_idx, uint32_t my_key, float my_es,
                                              int* idx_out, float* w_out) {
  const float my_val = key_value(my_key);
  const float vmax = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(my_val), 0));
  const float ex = lane < a.top_k ? expf(my_val - vmax) : 0.f;
  // sum of the weights in the order of a butterfly over xor 32, 16, .., 1;
  // with top_k <= 8 every lane past 7 holds zero and the first three steps
  // add exact zeros, so lanes 0-3 need only lane + 4, then the quad swaps
  float sum;
  if (a.top_k <= 8) {
    float s = ex + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(ex), 0x104, 0xF, 0xF, false));  // row_shl:4
    s += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(s), 0x4E, 0xF, 0xF, false));  // quad [2,3,0,1]
    s += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(s), 0xB1, 0xF, 0xF, false));  // quad [1,0,3,2]
    sum = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(s), 0));
  } else {
    sum = ex;
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) sum += __shfl_xor(sum, off, kWave);
  }
  if (lane < a.top_k) {
    float p = ex / sum;
    p *= my_es;
    idx_out[lane] = my_idx;
    w_out[lane] = p;
  }
}

// Top-k + softmax of one token by one wave (gemma.py:77-80) from the loaded
// inputs.  Each round takes the largest remaining key and, among equal keys,
// the lowest expert index, then retires it (key 0; every real value has a
// non-zero key).  Lane r < top_k ends with the r-th expert and its weight.
// With two experts per lane (E <= 128) each lane keeps its pair ordered, so
// a round is one wave maximum, one ballot and a pop on the winning lane.
template <int VPL, class A>
__device__ __forceinline__ void route_finish(const A& a, int lane, const RouteIn<VPL>& r, int* idx_out,
                                             float* w_out) {
  const bool bf = a.logits_dtype == GI_DTYPE_BF16;
  uint32_t keys[VPL];
  float es[VPL];
#pragma unroll
  for (int v = 0; v < VPL; ++v) {
    const int e = lane + v * kWave;
    const float f = __uint_as_float(bf ? r.raw[v] << 16 : r.raw[v]);
    keys[v] = e < a.E ? orderable_key(f) : 0u;
    es[v] = a.expert_scale ? __uint_as_float(r.es[v]) : 1.f;
  }
  int my_idx = 0;
  uint32_t my_key = 0u;
  float my_es = 1.f;
  if constexpr (VPL == 2) {
    const bool sw = keys[1] > keys[0];  // on a tie the lower expert (lane) stays first
    uint32_t hi = sw ? keys[1] : keys[0], lo = sw ? keys[0] : keys[1];
    int hi_i = sw ? lane + kWave : lane;
    const int lo_i = sw ? lane : lane + kWave;
    float hi_s = sw ? es[1] : es[0];
    const float lo_s = sw ? es[0] : es[1];
    bool popped = false;
    for (int rr = 0; rr < a.top_k; ++rr) {
      const uint32_t m = wave_max_u32(hi);
      const unsigned long long b = __ballot(hi == m);
      int w = (int)__builtin_ctzll(b);
      // equal maxima on several lanes: the lowest expert index among them
      // (a lane's second key equal to m has a larger index than its first)
      if (__popcll(b) > 1) w = (int)(wave_min_u32(hi == m ? (uint32_t)hi_i : 0xffffffffu) & (kWave - 1));
      const int wi = __builtin_amdgcn_readlane(hi_i, w);
      const float ws = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(hi_s), w));
      if (lane == w) {
        hi = popped ? 0u : lo;
        hi_i = lo_i;
        hi_s = lo_s;
        popped = true;
      }
      if (lane == rr) {
        my_idx = wi;
        my_key = m;
        my_es = ws;
      }
    }
  } else {
    for (int rr = 0; rr < a.top_k; ++rr) {
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
      if (lane == rr) {
        my_idx = win;
        my_key = m;
        my_es = ew;
      }
    }
  }
  route_softmax(a, lane, my_idx, my_key, my_es, idx_out, w_out);
}

// Loads and selection in one step (kernels with nothing to overlap).
template <int VPL, class A>
__device__ __forceinline__ void route_token(const A& a, int t, int lane, int* idx_out, float* w_out) {
  RouteIn<VPL> r;
  route_issue<VPL>(a, t, lane, r);
  route_finish<VPL>(a, lane, r, idx_out, w_out);
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

constexpr uint32_t kQ4BiasPair = 0xC1C0C1C0u;  // bf16 -24, twice: the offset of the 16+q operands

__device__ __forceinline__ f32x4_t mfma_bf16(uint4 a, uint4 b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}
// 8 bf16 values in the k order of an unpacked word: (0,4) (2,6) (1,5) (3,7)
__device__ __forceinline__ uint4 mfma_k_order(uint4 d) {
  const uint4 p = pair_permute(d);
  return make_uint4(p.x, p.z, p.y, p.w);
}
__device__ __forceinline__ uint4 q4_operand(uint32_t w, uint32_t mq) {
  const Q4Pairs q = unpack_q4(w, mq);
  return make_uint4(q.p0, q.p1, q.p2, q.p3);
}
// position of element p (0..7) of a packed row in that order
__device__ __forceinline__ int mfma_k_pos(int p) { return (p & 1) * 4 + (p & 2) + (p >> 2); }

// ---------------------------------------------------------------------------
// fp16 activations
// ---------------------------------------------------------------------------
// fp16 activations (the reference's fp16 dispatch, marlin.cu:694-700) run on
// the same bf16 matrix-core products: an fp16 value splits exactly into bf16
// hi (its leading 8 significand bits, truncated) and bf16 lo = value - hi
// (at most 3 significant bits), which take two A operand rows; the sum of the
// two rows' products is the fp16 value's product, in fp32.  Scales and out
// are fp16, the activation and the routing weights are rounded to fp16 where
// the bf16 path rounds to bf16.
__device__ __forceinline__ void f16_split2(uint32_t v, uint32_t& hi, uint32_t& lo) {
  const float a = fp16_to_f32((uint16_t)(v & 0xffffu)), b = fp16_to_f32((uint16_t)(v >> 16));
  const uint32_t ha = __float_as_uint(a) & 0xffff0000u, hb = __float_as_uint(b) & 0xffff0000u;
  const float la = a - __uint_as_float(ha), lb = b - __uint_as_float(hb);
  hi = (ha >> 16) | hb;
  lo = (__float_as_uint(la) >> 16) | (__float_as_uint(lb) & 0xffff0000u);
}
__device__ __forceinline__ void f16_split(const uint4 v, uint4& hi, uint4& lo) {
  f16_split2(v.x, hi.x, lo.x);
  f16_split2(v.y, hi.y, lo.y);
  f16_split2(v.z, hi.z, lo.z);
  f16_split2(v.w, hi.w, lo.w);
}
// fp16 weight operands for fp16 activations on the fp16 products: a half
// whose high byte is 0x58 and low byte 0x80 | q << 3 is exactly 144 + q
// (exponent 2^7, q in mantissa bits 3-6), so the bytes of the bf16 16 + q
// operands under 0x58 give 144 + q, and one packed fp16 add of -152 makes
// q - 8 exactly.  The products then need no offset term, and every operand
// and product is exact (fp16 x times a 4-bit integer, summed in fp32).
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
__device__ __forceinline__ uint32_t q4_magic_f16() {
  uint32_t v = 0x58585858u;
  asm volatile("" : "+v"(v));
  return v;
}
__device__ __forceinline__ uint32_t f16_pair_less152(uint32_t p) {
  const f16x2_t c = {(_Float16)-152.0f, (_Float16)-152.0f};
  return __builtin_bit_cast(uint32_t, __builtin_bit_cast(f16x2_t, p) + c);
}
// the four pairs (q0,q4) (q2,q6) (q1,q5) (q3,q7) as fp16 q - 8
__device__ __forceinline__ Q4Pairs unpack_q4_f16(uint32_t w, uint32_t mq16) {
  const Q4Pairs q = unpack_q4(w, mq16);
  return Q4Pairs{f16_pair_less152(q.p0), f16_pair_less152(q.p1), f16_pair_less152(q.p2), f16_pair_less152(q.p3)};
}
__device__ __forceinline__ f32x4_t mfma_f16(uint4 a, uint4 b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b), c,
                                                0, 0, 0);
}
__device__ __forceinline__ float fdot2_f16(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, a), __builtin_bit_cast(f16x2_t, b), c, false);
}
// The activation type's forms: bf16 (16 + q operands, an offset term) or
// fp16 (q - 8 operands, none).
template <bool F16>
__device__ __forceinline__ uint32_t q4_magic_t() {
  if constexpr (F16) return q4_magic_f16();
  else return q4_magic();
}
template <bool F16>
__device__ __forceinline__ Q4Pairs unpack_q4_t(uint32_t w, uint32_t mq) {
  if constexpr (F16) return unpack_q4_f16(w, mq);
  else return unpack_q4(w, mq);
}
template <bool F16>
__device__ __forceinline__ uint4 q4_operand_t(uint32_t w, uint32_t mq) {
  const Q4Pairs q = unpack_q4_t<F16>(w, mq);
  return make_uint4(q.p0, q.p1, q.p2, q.p3);
}
template <bool F16>
__device__ __forceinline__ f32x4_t mfma_act(uint4 a, uint4 b, f32x4_t c) {
  if constexpr (F16) return mfma_f16(a, b, c);
  else return mfma_bf16(a, b, c);
}
template <bool F16>
__device__ __forceinline__ float fdot2_act(uint32_t a, uint32_t b, float c) {
  if constexpr (F16) return fdot2_f16(a, b, c);
  else return fdot2(a, b, c);
}

template <bool F16>
__device__ __forceinline__ float sc_lo(uint32_t v) {
  if constexpr (F16) return fp16_to_f32((uint16_t)(v & 0xffffu));
  else return bf16lo(v);
}
template <bool F16>
__device__ __forceinline__ float sc_hi(uint32_t v) {
  if constexpr (F16) return fp16_to_f32((uint16_t)(v >> 16));
  else return bf16hi(v);
}
template <bool F16>
__device__ __forceinline__ float act_to_f32(uint32_t bits16) {
  if constexpr (F16) return fp16_to_f32((uint16_t)bits16);
  else return bf16_to_f32(bits16);
}
template <bool F16>
__device__ __forceinline__ uint16_t f32_to_act(float f) {
  if constexpr (F16) return __builtin_bit_cast(uint16_t, (_Float16)f);  // round to nearest even
  else return f32_to_bf16(f);
}
template <bool F16>
__device__ __forceinline__ float round_to_act(float f) {
  return act_to_f32<F16>(f32_to_act<F16>(f));
}
// the bit pattern of an activation with NaN made canonical (an all-ones half
// would be stored as zero, "not written", once inverted)
template <bool F16>
__device__ __forceinline__ uint16_t act_signal_bits(float f) {
  uint16_t bits = f32_to_act<F16>(f);
  if constexpr (F16) {
    if ((bits & 0x7fffu) > 0x7c00u) bits = 0x7e00u;
  } else {
    if ((bits & 0x7fffu) > 0x7f80u) bits = 0x7fc0u;
  }
  return bits;
}

}  // namespace moe
}  // namespace gi
