// Device helpers shared by the gfx950 kernels of the W4A16 MoE path.
//
// Conventions
//   * bf16 values travel as uint16_t bit patterns; arithmetic is fp32.
//   * int4 weights: nibble i of a packed int32 word holds the code q of row
//     k = 8*pk + i; the weight is (q - 8) * scale (reference quant.py:41-43,
//     marlin.cu:75-76).
//   * Activations used against packed words are staged "pair-permuted": the 8
//     bf16 values x0..x7 of one packed row are stored as the four dwords
//     (x0|x4), (x1|x5), (x2|x6), (x3|x7) so that one v_dot2_f32_bf16 consumes
//     the two codes that a single mask-and-or extracts from the word.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace gi {

constexpr int kWave = 64;

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

// 16-byte streaming load (non-temporal hint: weights are read once).
__device__ __forceinline__ uint4 load_nt_u4(const void* p) {
  u32x4_t v = __builtin_nontemporal_load((const u32x4_t*)p);
  return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ float bf16_to_f32(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}

// Round-to-nearest-even fp32 -> bf16 bit pattern (NaN stays NaN).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

__device__ __forceinline__ float round_to_bf16(float f) { return bf16_to_f32(f32_to_bf16(f)); }

// The same rounding for two values in one v_cvt_pk_bf16_f32 (gfx950): round to
// nearest even, NaN stays NaN; lo in bits 0-15, hi in bits 16-31.
typedef float f32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const f32x2_t v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

__device__ __forceinline__ float fp16_to_f32(uint16_t bits) {
  _Float16 h = __builtin_bit_cast(_Float16, bits);
  return (float)h;
}

// Load one routing weight of dtype code `dt` (0 bf16, 1 fp16, 2 fp32) and
// round it to bf16, the activation dtype (the reference casts the weights to
// x's dtype, marlin.cu:634-636).
__device__ __forceinline__ float load_weight_as_bf16(const void* w, int dt, int i) {
  float v;
  if (dt == 0) v = bf16_to_f32(((const uint16_t*)w)[i]);
  else if (dt == 1) v = fp16_to_f32(((const uint16_t*)w)[i]);
  else v = ((const float*)w)[i];
  return round_to_bf16(v);
}

__device__ __forceinline__ int load_expert_id(const void* idx, int is64, int i) {
  if (is64) {
    long long v = ((const long long*)idx)[i];
    return (v < -2147483647LL || v > 2147483647LL) ? -1 : (int)v;
  }
  return ((const int*)idx)[i];
}

// Pair-permute 8 consecutive bf16 values (as 4 dwords d0..d3 = x0x1, x2x3,
// x4x5, x6x7) into (x0|x4), (x1|x5), (x2|x6), (x3|x7).
__device__ __forceinline__ uint4 pair_permute(uint4 d) {
  uint4 p;
  p.x = __builtin_amdgcn_perm(d.z, d.x, 0x05040100u);
  p.y = __builtin_amdgcn_perm(d.z, d.x, 0x07060302u);
  p.z = __builtin_amdgcn_perm(d.w, d.y, 0x05040100u);
  p.w = __builtin_amdgcn_perm(d.w, d.y, 0x07060302u);
  return p;
}

// -24 * sum of the 8 bf16 values in d: the bias that turns sum x*(16+q)
// into sum x*(q-8) (see dot8_q4).
__device__ __forceinline__ float q4_bias(uint4 d) {
  float s = bf16_to_f32(d.x & 0xffffu) + bf16_to_f32(d.x >> 16) +
            bf16_to_f32(d.y & 0xffffu) + bf16_to_f32(d.y >> 16) +
            bf16_to_f32(d.z & 0xffffu) + bf16_to_f32(d.z >> 16) +
            bf16_to_f32(d.w & 0xffffu) + bf16_to_f32(d.w >> 16);
  return -24.0f * s;
}

__device__ __forceinline__ float fdot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                         __builtin_bit_cast(bf16x2_t, b), c, false);
}

// sum_{i<8} x_i * (q_i - 8) for one packed word, given pair-permuted x and
// bias = -24 * sum x_i.  A bf16 whose high byte is 0x41 and low byte is
// 0x80 | (q << 3) is exactly 16 + q (exponent 2^4, q in the top four mantissa
// bits: unit spacing from 16 to 32), so v_perm_b32 can assemble two
// dequantised codes per instruction from bytes holding 0x80 | q << 3 and a
// register holding 0x41 bytes; each pair feeds one v_dot2_f32_bf16 and the
// bias removes the 24 = 16 + 8 offset.  (A larger base such as 128 + q costs
// precision: the fp32 sums carry base * sum x, which cancels.)
//   lo = (w << 3) & 0x78787878 | 0x80808080 holds codes (q0, q2, q4, q6),
//   hi = (w >> 1) & 0x78787878 | 0x80808080 holds (q1, q3, q5, q7).
// 0x80808080 held in a vector register, so that (v & 0x78787878) | 0x80808080
// is one v_and_or_b32 (a VOP3 instruction takes no literal and reads at most
// one scalar register here); the empty asm has no side effects, so repeated
// calls fold into one register.
__device__ __forceinline__ uint32_t q4_high_bits() {
  uint32_t v = 0x80808080u;
  asm("" : "+v"(v));
  return v;
}
__device__ __forceinline__ void q4_bytes(uint32_t w, uint32_t& lo, uint32_t& hi) {
  const uint32_t mc = q4_high_bits();
  lo = ((w << 3) & 0x78787878u) | mc;
  hi = ((w >> 1) & 0x78787878u) | mc;
}
__device__ __forceinline__ float dot8_q4(uint32_t w, uint4 xp, float bias, uint32_t mq) {
  uint32_t lo, hi;
  q4_bytes(w, lo, hi);
  float d = fdot2(xp.x, __builtin_amdgcn_perm(mq, lo, 0x04020400u), bias);  // (q0, q4)
  d = fdot2(xp.z, __builtin_amdgcn_perm(mq, lo, 0x04030401u), d);           // (q2, q6)
  d = fdot2(xp.y, __builtin_amdgcn_perm(mq, hi, 0x04020400u), d);           // (q1, q5)
  d = fdot2(xp.w, __builtin_amdgcn_perm(mq, hi, 0x04030401u), d);           // (q3, q7)
  return d;
}

// The same product split in two, so that one unpacked word serves several
// activation rows: unpack_q4 gives the four bf16 pairs (16+q) of dot8_q4,
// dot_unpacked takes them with one row's pair-permuted x and bias.
struct Q4Pairs {
  uint32_t p0, p1, p2, p3;  // (q0,q4) (q2,q6) (q1,q5) (q3,q7)
};
__device__ __forceinline__ Q4Pairs unpack_q4(uint32_t w, uint32_t mq) {
  uint32_t lo, hi;
  q4_bytes(w, lo, hi);
  return Q4Pairs{__builtin_amdgcn_perm(mq, lo, 0x04020400u), __builtin_amdgcn_perm(mq, lo, 0x04030401u),
                 __builtin_amdgcn_perm(mq, hi, 0x04020400u), __builtin_amdgcn_perm(mq, hi, 0x04030401u)};
}
__device__ __forceinline__ float dot_unpacked(const Q4Pairs& d, uint4 xp, float bias) {
  float r = fdot2(xp.x, d.p0, bias);
  r = fdot2(xp.z, d.p1, r);
  r = fdot2(xp.y, d.p2, r);
  return fdot2(xp.w, d.p3, r);
}

// 0x41414141 held in a VGPR (v_perm_b32 may read only one scalar operand).
__device__ __forceinline__ uint32_t q4_magic() {
  uint32_t v = 0x41414141u;
  asm volatile("" : "+v"(v));
  return v;
}

// Makes `v` opaque to the optimiser (no instruction is emitted).  Used on
// prefetched weight words inside loops so their dequantisation is not hoisted
// out as loop-invariant, which would hold 4x the packed bytes in registers.
__device__ __forceinline__ uint4 opaque(uint4 v) {
  asm volatile("" : "+v"(v.x), "+v"(v.y), "+v"(v.z), "+v"(v.w));
  return v;
}

__device__ __forceinline__ uint2 opaque(uint2 v) {
  asm volatile("" : "+v"(v.x), "+v"(v.y));
  return v;
}

__device__ __forceinline__ float bf16lo(uint32_t v) { return __uint_as_float(v << 16); }
__device__ __forceinline__ float bf16hi(uint32_t v) { return __uint_as_float(v & 0xffff0000u); }

// Sum over the lanes that share (lane & (group-1)) within a wave: i.e. reduce
// across lane bits log2(group)..5.  Every lane ends with its group's total.
template <int kGroup>
__device__ __forceinline__ float reduce_across_groups(float v) {
#pragma unroll
  for (int off = kGroup; off < kWave; off <<= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

// Sum over the 64 lanes, returned to every lane (wave-uniform).  Each row of
// 16 lanes is summed with DPP (quad butterflies, then the half-row and row
// mirrors), the four row sums are read with v_readlane and added in the fixed
// order (r0 + r1) + (r2 + r3).
template <int kCtrl>
__device__ __forceinline__ float dpp_f32(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), kCtrl, 0xF, 0xF, false));
}
__device__ __forceinline__ float wave_sum_f32(float v) {
  v += dpp_f32<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp_f32<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp_f32<0x141>(v);  // row_half_mirror
  v += dpp_f32<0x140>(v);  // row_mirror
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return (r0 + r1) + (r2 + r3);
}

// ---- inter-workgroup data and signals ---------------------------------------
// Data handed between workgroups (possibly on different XCDs, whose L2 caches
// are not coherent with each other) is written and read with relaxed
// agent-scope atomic accesses: on gfx950 these are plain loads/stores with the
// sc1 bit, i.e. performed at the device coherence point, so no L2 writeback
// or invalidate (which acquire/release at agent scope would add to every
// flag operation) is needed.  A producer waits for its sc1 stores to complete
// (wait_vmem) before the workgroup barrier that precedes the counter update;
// a consumer observes the counter, crosses a barrier, then issues its sc1 loads.
__device__ __forceinline__ void st_coherent(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_coherent_f32(float* p, float v) {
  __hip_atomic_store((uint32_t*)p, __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_coherent_f32(const float* p) {
  return __uint_as_float(__hip_atomic_load((uint32_t*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
}
__device__ __forceinline__ uint4 ld_coherent_u4(const void* p) {
  unsigned long long* q = (unsigned long long*)p;
  const unsigned long long lo = __hip_atomic_load(q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const unsigned long long hi = __hip_atomic_load(q + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return make_uint4((uint32_t)lo, (uint32_t)(lo >> 32), (uint32_t)hi, (uint32_t)(hi >> 32));
}
// 16-byte forms of the same accesses, through a buffer resource: the cache
// policy argument 16 is the sc1 bit (what the compiler emits for the 4- and
// 8-byte atomics above).  One instruction covers whole cache lines, so a
// wave's 1 KB of partials leaves the L2 as 8 full lines instead of 4 partial
// writes per line.  Offsets past `bytes` read 0 and drop stores.
constexpr int kCpolAgent = 16;
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ void st_coherent_f4(__amdgpu_buffer_rsrc_t r, uint32_t off, float4 v) {
  u32x4_t w;
  w.x = __float_as_uint(v.x);
  w.y = __float_as_uint(v.y);
  w.z = __float_as_uint(v.z);
  w.w = __float_as_uint(v.w);
  __builtin_amdgcn_raw_buffer_store_b128(w, r, off, 0, kCpolAgent);
}
__device__ __forceinline__ float4 ld_coherent_f4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  const u32x4_t w = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kCpolAgent);
  return make_float4(__uint_as_float(w.x), __uint_as_float(w.y), __uint_as_float(w.z), __uint_as_float(w.w));
}
// Wait until every memory operation this wave issued has completed.
__device__ __forceinline__ void wait_vmem() { __builtin_amdgcn_s_waitcnt(0); }

// Workgroup barrier for LDS data: waits for this wave's LDS (and scalar)
// accesses and meets the other waves, leaving global loads in flight.
// __syncthreads() also waits for vmcnt(0) (its workgroup-scope fence), which
// would drain every prefetched weight load at each barrier.  Global data
// handed between waves needs wait_vmem() before this barrier.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// ---- counters (agent scope) -------------------------------------------------
__device__ __forceinline__ int atomic_add_relaxed(int* p, int v) {
  return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int atomic_add_acq_rel(int* p, int v) {
  return __hip_atomic_fetch_add(p, v, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int load_relaxed(int* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_relaxed(int* p, int v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// A bounded wait gave up (never expected: every wait is for work of the same
// launch): the workspace's status bit, and the library's host-visible
// per-device flag when there is one (host memory mapped into the device; the
// drop-in module reads it without a synchronisation).
__device__ __forceinline__ void report_timeout(int* status, int* host_flag) {
  atomicOr(status, 1);  // GI_DEVICE_SPIN_TIMEOUT
  if (host_flag) __hip_atomic_store(host_flag, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

__device__ __forceinline__ float gelu_tanh(float x) {
  // 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3)))  (reference marlin.cu:7-11)
  float inner = 0.7978845608028654f * (x + 0.044715f * x * x * x);
  return 0.5f * x * (1.0f + tanhf(inner));
}

}  // namespace gi
