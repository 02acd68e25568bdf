// Token-Union W4A16 fused MoE for ONE token (decode, M = 1) on gfx950: one
// launch per layer, one wait between workgroups.
//
// Reference behaviour restated (paths relative to the GemmaInfer repo):
//   routing        gemmainfer/models/gemma.py:77-80
//   dedup          csrc/marlin.cu:285-335 (one token: slots with one expert merge)
//   gate_up + GELU csrc/marlin.cu:337-426
//   down + combine csrc/marlin.cu:507-586
//
// A launch has G workgroups of 512 threads, one per CU, all resident.  Every
// workgroup routes the token itself (its threads rank the router logits, or
// wave 0 reads the caller's ids) and derives the same split of the work from
// the number U of unique experts (in rank order, for ids in the order of
// their first slot), Tk = I/32 intermediate column tiles and units = H/32
// output column units:
//
//   items   workgroups w < U*Tk.  Item (u, c): expert u's gate and up columns
//           [32c, 32c+32) over all of H.  The words (16-byte loads, 11 per
//           lane) go out right after the routing, then x (loaded at the
//           start) is staged in LDS;
//           products on the matrix cores, the waves' sums added in LDS,
//           act = bf16(gelu_tanh(gate) * up) (where the reference stores its
//           activation, marlin.cu:421-423) published for the unit workgroups.
//           The item also multiplies its 32 activations with the expert's
//           down rows [32c, 32c+32) over the columns of the folded units (see
//           below) and publishes those routing-weighted fp32 partial sums.
//   units   workgroups w = U*Tk + d, d < n_whole = min(units, G - U*Tk):
//           output columns [32d, 32d+32) over every expert.  The down words of
//           those columns for all U experts (11 16-byte loads per lane at
//           U = 8) go out right after the routing; once every activation has
//           arrived, the products run on the matrix cores (two (expert, k
//           block) pairs per product: A rows 0 and 1 are the two pairs'
//           activations, B columns 0-7 and 8-15 their words), the waves'
//           sums are added in LDS and out is written once.
//   folded  units [n_whole, units) have no workgroup of their own (8 of 88 at
//           U = 8 on 256 CUs); their products come from the items, and item
//           f < n_left, once its own work is done, sums folded unit
//           n_whole + f from every item's partial sums (a wait between
//           items, off the units' path).
//
// At U = 8, 176 items of 92.9 KB (+ 4.5 KB of folded down words) and 80 units
// of 93.2 KB: every CU streams about the same bytes (24.56 MB / 256 = 95.9 KB).
//
// Deterministic: every sum has a fixed order, whatever the timing.
//
// fp16 activations (template parameter F16; x, scales and out in fp16, the
// routing caller-given).  Items: the same bf16 products, each fp16 value of x
// split exactly into a bf16 hi and a bf16 lo part that take A rows 0 and 1,
// the rows' products added in fp32; their int4 unpack, which the items wait
// on, stays the bf16 kernel's.  Units, which unpack their words before the
// activations arrive: fp16 products with the codes unpacked exactly to fp16
// q - 8 (the same bytes under 0x58, less 152), so the activations are staged
// as they arrive, with no split and no offset sums.
//
// Exchange (moe_state.h): activations are stored bit-inverted, 16 bytes at a
// time, into the activation buffer of the launch's parity (expert-major rows
// of I values, matrix-core k order within each 8); partial sums, inverted,
// into the partial buffer ([item][n_left * 32] fp32).  A stored 16-bit (32-bit)
// value is never all ones (canonical NaN), so all-zero means "not written
// yet" and readers poll the data itself, with a bounded wait.  The idle
// workgroups (else the units, while they wait for the activations; else all)
// clear what the previous launch wrote into the other parity (the footprint
// in the epoch word).

#include <mutex>

#include "../../include/gemmainfer_amd.h"
#include "decode1_split.h"
#include "gi_common.h"
#include "gi_internal.h"
#include "moe_shared.h"
#include "moe_state.h"
#include "moe_timeline.h"

namespace gi {

namespace {

using namespace moe;
using moe_state::kActParity;
using moe_state::kEpochSlots;
using moe_state::kPartParity;

constexpr int kT = 512;
constexpr int kW = kT / kWave;         // 8 waves
constexpr int kKbw = 11;               // gate/up k blocks of 32 per wave
constexpr int kMaxH = kW * kKbw * 32;  // 2816
constexpr int kMaxU = kW;              // unique experts: one wave each in the unit workgroups
constexpr int kMaxTk = 24;             // I <= 768
constexpr int kMaxGd = 12;             // down scale groups (group size >= 64)
constexpr int kGuSc = 6;               // scale groups the k blocks of one wave meet (group size >= 64)
constexpr int kMaxLeft = 8;            // folded units
constexpr int kSlots = 64;
constexpr int kDefaultSpin = 1 << 20;
constexpr int kCpolNt = 2;             // non-temporal: weights are read once
constexpr uint32_t kOob = 0xFFFFFFF0u;  // past every buffer resource: the load returns zeros
// Unit workgroups hold their down words back for the time the items' bytes
// take at this rate (bytes per 10 ns tick of the constant clock, ~9.4 TB/s:
// the items' words are then about 60% served at the ~5.5 TB/s the layer
// streams at).  Measured at M=1 (U = 8, 16.4 MB of item bytes): holds of
// 1.5-2.0 us give 12.0 us per layer against 12.7 us with no hold; 4 us, 13.5.
constexpr uint32_t kUnitHoldBytesPerTick = 94208;

__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

// log2(group size / 32): fixed at compile time for the common group sizes
// (GSH 1: 64, 2: 128), so that the scale-group ends of the unrolled loops
// are known to the compiler; GSH 0 reads it from the arguments.
template <int GSH, class A>
__device__ __forceinline__ int gsh_of(const A& a) {
  if constexpr (GSH > 0) return GSH;
  else return a.gsh;
}
__device__ __forceinline__ void lds_fence() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

struct D1Args {
  const uint16_t* x;
  const int32_t* gu_packed;
  const uint16_t* gu_scales;
  const int32_t* d_packed;
  const uint16_t* d_scales;
  const void* idx;
  const void* w;
  const void* logits;
  const float* expert_scale;
  int32_t* out_idx;
  uint16_t* out_w;
  uint16_t* out;
  unsigned long long* epochs;  // [kEpochSlots]
  char* act;                   // two parities of kActParity bytes
  char* part;                  // two parities of kPartParity bytes
  int* status;
  int* host_flag;
  unsigned long long* timeline;
  uint32_t gu_bytes, gus_bytes, dn_bytes, dsc_bytes;  // one expert's tensors
  uint32_t dn_total, dsc_total;                       // whole down tensors
  int idx_is64, w_dtype, logits_dtype;
  int H, I, E, top_k, Ggu, Gd;
  int gsh;  // group size = 32 << gsh
  int Tk, units;
  int overwrite, spin_limit;
};

constexpr int kRankKeys = 128;  // router logits ranked by all threads up to this many experts

struct D1Pro {
  int slot_e[kSlots];
  float slot_w[kSlots];
  uint32_t sel_key[kSlots];   // routing from logits: the selected keys and expert scales by rank
  float sel_es[kSlots];
  uint32_t id_key[kSlots];    // the same in id order (radix select)
  float id_es[kSlots];
  int rpart[kW][kRankKeys];   // rank select: wave w's count of its keys above each key
  __attribute__((aligned(16))) unsigned long long rkeys[kW][16];  // rank select: the 16 keys wave w reads
  int uexp[kMaxU];
  float uw[kMaxU];
  float cb[kMaxH / 8];        // -24 * the sum of each 8-value chunk of x (zero past the scale groups)
  int U;
  int bad;
  unsigned long long epoch;
};

template <bool F16>
struct ItemLds {
  uint4 xs[kMaxH / 8];            // x in the matrix-core k order, per packed row (fp16: the bf16 hi part)
  uint4 xs_lo[F16 ? kMaxH / 8 : 1];  // fp16: the bf16 lo part (A row 1)
  uint4 xz[4 * kKbw];             // zeros: the A operand rows 1-15 (lanes lr > 0) read these
  float4 red[kW][16];             // per-wave sums: lane lr holds 4 gate (lr < 8) or up columns
  uint4 sa[4];                    // the item's 32 activations, matrix-core k order
  float4 fr[4][kMaxLeft * 8];     // folded products per packed row
  float4 rr[kW][8];               // folded unit reduction: each wave's sums (8 column quads)
};
template <bool F16>
struct UnitLds {
  uint4 sact[kMaxU * kMaxTk * 4];   // activation chunks [u][I/8], plain bf16 or fp16 in matrix-core k order
  uint4 dsc[kMaxU * kMaxGd * 4];    // down scales of the unit's columns [u][g][32]
  float4 red[kW][16];
};
template <bool F16>
union D1Lds {
  ItemLds<F16> it;
  UnitLds<F16> un;
};



// Every 16-bit half non-zero.
__device__ __forceinline__ bool chunk_ready(const u32x4_t v) {
  const uint32_t a0 = min(v.x & 0xffffu, v.x >> 16), a1 = min(v.y & 0xffffu, v.y >> 16);
  const uint32_t a2 = min(v.z & 0xffffu, v.z >> 16), a3 = min(v.w & 0xffffu, v.w >> 16);
  return min(min(a0, a1), min(a2, a3)) != 0u;
}
__device__ __forceinline__ uint32_t f32_signal_bits(float v) {
  uint32_t b = __float_as_uint(v);
  if ((b & 0x7fffffffu) > 0x7f800000u) b = 0x7fc00000u;  // canonical NaN: never stored as zero
  return ~b;
}
// sum of a staged chunk (matrix-core k order: pairs (x0,x4) (x2,x6) (x1,x5)
// (x3,x7)) times the unpacked word's 16+q pairs, plus c
__device__ __forceinline__ float dot_chunk(const uint4 A, const Q4Pairs& q, float c) {
  c = fdot2(A.x, q.p0, c);
  c = fdot2(A.y, q.p1, c);
  c = fdot2(A.z, q.p2, c);
  return fdot2(A.w, q.p3, c);
}

// q4_operand (moe_shared.h) in 8 VALU operations per word: the byte of code
// q is 0x80 | q << 3, and v_perm_b32 pairs those bytes with 0x41 bytes into
// bf16 16 + q, in the matrix-core k order (0,4) (2,6) (1,5) (3,7).
__device__ __forceinline__ uint4 q4_operand_fast(uint32_t w, uint32_t mq, uint32_t mc);
// The same bytes as fp16 operands (mq holding 0x58 bytes: 144 + q), less 152:
// exact q - 8 for the fp16 products.
template <bool F16>
__device__ __forceinline__ uint4 q4_operand_fast_t(uint32_t w, uint32_t mq, uint32_t mc) {
  uint4 r = q4_operand_fast(w, mq, mc);
  if constexpr (F16) {
    r.x = f16_pair_less152(r.x);
    r.y = f16_pair_less152(r.y);
    r.z = f16_pair_less152(r.z);
    r.w = f16_pair_less152(r.w);
  }
  return r;
}
__device__ __forceinline__ uint4 q4_operand_fast(uint32_t w, uint32_t mq, uint32_t mc) {
  const uint32_t lo = ((w << 3) & 0x78787878u) | mc;
  const uint32_t hi = ((w >> 1) & 0x78787878u) | mc;
  return make_uint4(__builtin_amdgcn_perm(mq, lo, 0x04020400u), __builtin_amdgcn_perm(mq, lo, 0x04030401u),
                    __builtin_amdgcn_perm(mq, hi, 0x04020400u), __builtin_amdgcn_perm(mq, hi, 0x04030401u));
}

// ---------------------------------------------------------------------------
// start: routing inputs, epoch, x; clearing; routing
// ---------------------------------------------------------------------------
// Routing inputs, loaded first by wave 0: the router row (lane l holds
// logits l + 64v, route_issue) or lane s < top_k the caller's id s and weight s.
template <int VPL>
struct D1In {
  RouteIn<VPL> r;
  uint32_t id_lo, id_hi, wb;
};
template <int VPL>
__device__ __forceinline__ void d1_issue(const D1Args& a, D1In<VPL>& in) {
  const int lane = threadIdx.x & (kWave - 1);
  in.id_lo = in.id_hi = in.wb = 0u;
  if (a.logits) {
    route_issue<VPL>(a, 0, lane, in.r);
  } else {
    const uint32_t S = (uint32_t)a.top_k;
    if (a.idx_is64) {
      const u32x2_t v = __builtin_amdgcn_raw_buffer_load_b64(buffer_rsrc(a.idx, S * 8u), lane * 8u, 0, 0);
      in.id_lo = v.x;
      in.id_hi = v.y;
    } else {
      in.id_lo = __builtin_amdgcn_raw_buffer_load_b32(buffer_rsrc(a.idx, S * 4u), lane * 4u, 0, 0);
    }
    if (a.w_dtype == GI_DTYPE_FP32)
      in.wb = __builtin_amdgcn_raw_buffer_load_b32(buffer_rsrc(a.w, S * 4u), lane * 4u, 0, 0);
    else
      in.wb = __builtin_amdgcn_raw_buffer_load_b16(buffer_rsrc(a.w, S * 2u), lane * 2u, 0, 0);
  }
}

// Router logits (gemma.py:77-80; the tie rule of route_finish: value
// descending, then index ascending, NaN highest).  Both forms leave the
// top_k experts in rank order: P.uexp (the unique experts, which is all the
// weight loads need), P.slot_e, P.sel_key and P.sel_es, and P.U = top_k.
// The softmax waits until the weight loads are in flight (d1_weights).
//
// Up to kRankKeys experts (d1_rank_count, d1_rank_pick): every wave loads the
// router row (lane l: experts l and l + 64) and forms each expert's composite
// key (key << 10 | (1023 - expert): a higher value, then the lower index, is
// larger; padding experts past E get key 0, below every real key).  Wave w
// broadcasts its 16 keys j = 16w .. 16w+15 (readlane) and counts, for all 128
// keys, how many of its 16 are larger; after a barrier thread i < 128 adds the
// 8 waves' counts, the rank of key i, and writes expert i at its rank when
// that is below top_k.
//
// More experts (d1_select, d1_rank_radix; wave 0): a radix select finds the
// top_k-th largest key T, two bits per step (three candidate prefixes counted
// at once with ballots and popcounts), first over the high 16 bits of the
// keys and, only when that leaves a tie at the boundary, over the low 16; the
// selection is every key above T and the lowest-index keys equal to T, which
// top_k steps over the selected keys then rank.
struct RankKeys {
  unsigned long long c[2];  // composite keys of experts lane, lane + 64
  float es[2];              // their expert scales
};

__device__ __forceinline__ void d1_rank_count(const D1Args& a, D1Pro& P, const RouteIn<2>& r, RankKeys& k) {
  const int lane = threadIdx.x & (kWave - 1), wave = uniform(threadIdx.x >> 6);
  const bool bf = a.logits_dtype == GI_DTYPE_BF16;
#pragma unroll
  for (int v = 0; v < 2; ++v) {
    const int e = lane + v * kWave;
    const float f = __uint_as_float(bf ? r.raw[v] << 16 : r.raw[v]);
    const uint32_t key = e < a.E ? orderable_key(f) : 0u;  // a real key is never 0
    k.c[v] = ((unsigned long long)key << 10) | (unsigned long long)(1023 - e);
    k.es[v] = a.expert_scale ? __uint_as_float(r.es[v]) : 1.f;
  }
  // keys j = 16w + jj: lane (16w + jj) % 64 of c[w / 4]; those 16 lanes put
  // them in the wave's own LDS row, and every lane reads the row back (same
  // wave: ordered without a barrier; broadcast reads, all issued at once)
  const unsigned long long src = wave < 4 ? k.c[0] : k.c[1];
  const int l0 = (wave & 3) * 16;
  if (lane >= l0 && lane < l0 + 16) P.rkeys[wave][lane - l0] = src;
  lds_fence();
  unsigned long long cj[16];
#pragma unroll
  for (int jj = 0; jj < 16; jj += 2) {
    const uint4 v = *(const uint4*)&P.rkeys[wave][jj];
    cj[jj] = ((unsigned long long)v.y << 32) | v.x;
    cj[jj + 1] = ((unsigned long long)v.w << 32) | v.z;
  }
  int n0 = 0, n1 = 0;
#pragma unroll
  for (int jj = 0; jj < 16; ++jj) {
    n0 += cj[jj] > k.c[0] ? 1 : 0;
    n1 += cj[jj] > k.c[1] ? 1 : 0;
  }
  P.rpart[wave][lane] = n0;
  P.rpart[wave][kWave + lane] = n1;
}

// Threads i < 128 (waves 0 and 1: key i is c[i / 64] of lane i % 64), after
// the barrier that published P.rpart.
__device__ __forceinline__ void d1_rank_pick(const D1Args& a, D1Pro& P, const RankKeys& k) {
  const int i = threadIdx.x;
  int rank = 0;
#pragma unroll
  for (int w = 0; w < kW; ++w) rank += P.rpart[w][i];
  const int v = i >> 6;
  const unsigned long long ci = v ? k.c[1] : k.c[0];
  if (i < a.E && rank < a.top_k) {
    P.uexp[rank] = i;
    P.slot_e[rank] = i;
    P.sel_key[rank] = (uint32_t)(ci >> 10);
    P.sel_es[rank] = v ? k.es[1] : k.es[0];
  }
}

template <int VPL>
__device__ __forceinline__ int count_ge(const uint32_t (&key)[VPL], uint32_t t) {
  int c = 0;
#pragma unroll
  for (int v = 0; v < VPL; ++v) c += __popcll(__ballot(key[v] >= t));
  return c;
}

template <int VPL>
__device__ __forceinline__ void d1_select(const D1Args& a, D1Pro& P, const RouteIn<VPL>& r) {
  const int lane = threadIdx.x & (kWave - 1);
  const bool bf = a.logits_dtype == GI_DTYPE_BF16;
  const int K = a.top_k;
  uint32_t key[VPL];
#pragma unroll
  for (int v = 0; v < VPL; ++v) {
    const float f = __uint_as_float(bf ? r.raw[v] << 16 : r.raw[v]);
    key[v] = lane + v * kWave < a.E ? orderable_key(f) : 0u;  // a real key is never 0
  }
  GI_STAMP(16);
  // T: the largest value with at least K keys >= T, two bits at a time
  uint32_t T = 0u;
  int lo_bit = 16;
  for (int bit = 30;; bit -= 2) {
    const uint32_t c1 = T | (1u << bit), c2 = T | (2u << bit), c3 = T | (3u << bit);
    const int n1 = count_ge(key, c1), n2 = count_ge(key, c2), n3 = count_ge(key, c3);
    T = n3 >= K ? c3 : n2 >= K ? c2 : n1 >= K ? c1 : T;
    if (bit == lo_bit) {
      // the high bits are decided: stop if no key below T shares them (no tie
      // to break), else go on through the low 16 bits
      if (lo_bit == 16 && count_ge(key, T) != K) lo_bit = 0;
      else break;
    }
  }
  // the selection: keys above T, then keys equal to T in index order; in
  // ascending id order, with each one's key and expert scale
  int n_gt = 0;
#pragma unroll
  for (int v = 0; v < VPL; ++v) n_gt += __popcll(__ballot(key[v] > T));
  int need = K - n_gt;
  const unsigned long long below = (1ull << lane) - 1ull;
  int pos_base = 0;
#pragma unroll
  for (int v = 0; v < VPL; ++v) {
    const unsigned long long eq = __ballot(key[v] == T);
    const bool take = key[v] > T || (key[v] == T && __popcll(eq & below) < need);
    need -= min(need, __popcll(eq));
    const unsigned long long m = __ballot(take);
    if (take) {
      const int pos = pos_base + __popcll(m & below);
      P.uexp[pos] = lane + v * kWave;
      P.id_key[pos] = key[v];
      P.id_es[pos] = a.expert_scale ? __uint_as_float(r.es[v]) : 1.f;
    }
    pos_base += __popcll(m);
  }
  if (lane == 0) P.U = K;
  GI_STAMP(17);
}

// Wave 0, after d1_select: the selection (in id order) ranked by key; a lower
// place in the id order is a lower index.
__device__ __forceinline__ void d1_rank_radix(const D1Args& a, D1Pro& P) {
  const int lane = threadIdx.x & (kWave - 1);
  const int K = a.top_k;
  lds_fence();
  const int j = lane < K ? lane : 0;
  const uint32_t kj = P.id_key[j];
  const int ej = P.uexp[j];
  const float esj = P.id_es[j];
  int rank = 0;
  for (int i = 0; i < K; ++i) {
    const uint32_t ki = (uint32_t)__builtin_amdgcn_readlane((int)kj, i);
    rank += (ki > kj) + (ki == kj && i < lane);
  }
  if (lane < K) {  // every lane has read P.uexp above (one wave, program order)
    P.uexp[rank] = ej;
    P.slot_e[rank] = ej;
    P.sel_key[rank] = kj;
    P.sel_es[rank] = esj;
  }
}

// Wave 0, while the weight loads are in flight: route_softmax over the
// selection in rank order (the arithmetic of route_finish); each weight,
// rounded to bf16, is the weight of the unique expert at the same place
// (P.uw) and is kept for the routing report (P.slot_w).
__device__ __forceinline__ void d1_weights(const D1Args& a, D1Pro& P) {
  const int lane = threadIdx.x & (kWave - 1);
  const int K = a.top_k;
  const int rr = lane < K ? lane : 0;
  route_softmax(a, lane, P.slot_e[rr], P.sel_key[rr], P.sel_es[rr], P.slot_e, P.slot_w);
  lds_fence();
  if (lane < K) {
    const float w = round_to_bf16(P.slot_w[lane]);
    P.slot_w[lane] = w;  // reported by workgroup 0 at the end
    P.uw[lane] = w;
  }
  GI_STAMP(19);
}

// Wave 0, the caller's ids: the slots' experts and weights, then the
// unique experts; a slot whose expert an earlier slot has is merged into that
// one (weights added in slot order), invalid ids are dropped.  The weights are
// rounded to bf16 (the reference casts them to the activation dtype,
// marlin.cu:634-636).  The unique experts are in the order of their first
// slot: for ids from a sorted top-k (gemma.py:77-80) that is the rank order
// of the router-logits form, so both forms split the work alike.
template <int VPL, bool F16>
__device__ __forceinline__ void d1_route_ids(const D1Args& a, D1Pro& P, const D1In<VPL>& in) {
  const int lane = threadIdx.x & (kWave - 1);
  const int S = a.top_k;
  if (lane < S) {
    int e = (int)in.id_lo;
    if (a.idx_is64) {
      const long long v = (long long)(((unsigned long long)in.id_hi << 32) | in.id_lo);
      e = (v < -2147483647LL || v > 2147483647LL) ? -1 : (int)v;
    }
    P.slot_e[lane] = (e >= 0 && e < a.E) ? e : -1;
    const float wv = a.w_dtype == GI_DTYPE_FP32   ? __uint_as_float(in.wb)
                     : a.w_dtype == GI_DTYPE_FP16 ? fp16_to_f32((uint16_t)in.wb)
                                                  : bf16_to_f32(in.wb);
    P.slot_w[lane] = round_to_act<F16>(wv);
  }
  lds_fence();
  const int e = lane < S ? P.slot_e[lane] : -1;
  // same-expert slots, from LDS (broadcast reads, independent of each other)
  float ws = 0.f;
  bool first = true;
  for (int j0 = 0; j0 < S; j0 += 8) {
    int ej[8];
    float wj[8];
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      const int j = min(j0 + m, kSlots - 1);
      ej[m] = P.slot_e[j];
      wj[m] = P.slot_w[j];
    }
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      if (j0 + m < S && e >= 0 && ej[m] == e) {
        ws += wj[m];
        if (j0 + m < lane) first = false;
      }
    }
  }
  const bool keep = lane < S && e >= 0 && first;
  const unsigned long long bal = __ballot(keep);
  const int u = __popcll(bal & ((1ull << lane) - 1ull));
  if (keep && u < kMaxU) {
    P.uexp[u] = e;
    P.uw[u] = ws;
  }
  if (lane == 0) P.U = __popcll(bal);
}

// Share `slot` of `nslots` of what the previous launch wrote into the other
// parity's buffers (16-byte stores by all threads; the footprint is in the
// epoch word ew, stores past it fall outside the buffer resources).
__device__ __forceinline__ void clear_prev(const D1Args& a, unsigned long long ew, int parity, int slot,
                                           int nslots) {
  const uint32_t act_b = moe_state::epoch_act_units(ew) * moe_state::kUnit;
  const uint32_t part_b = moe_state::epoch_part_units(ew) * moe_state::kUnit;
  const u32x4_t z = {0u, 0u, 0u, 0u};
  const __amdgpu_buffer_rsrc_t ra = buffer_rsrc(a.act + (size_t)(parity ^ 1) * kActParity, act_b);
  const __amdgpu_buffer_rsrc_t rp = buffer_rsrc(a.part + (size_t)(parity ^ 1) * kPartParity, part_b);
  const int na = (int)(act_b / 16), np = (int)(part_b / 16);
  const int pa = (na + nslots - 1) / nslots, pp = (np + nslots - 1) / nslots;
  for (int i = (int)threadIdx.x; i < pa; i += kT)
    __builtin_amdgcn_raw_buffer_store_b128(z, ra, (uint32_t)(slot * pa + i) * 16u, 0, kCpolAgent);
  for (int i = (int)threadIdx.x; i < pp; i += kT)
    __builtin_amdgcn_raw_buffer_store_b128(z, rp, (uint32_t)(slot * pp + i) * 16u, 0, kCpolAgent);
}

// The start of every workgroup: the routing inputs go out first (wave 0),
// then the epoch word and x, which do not depend on the routing (x stays in
// registers, thread c holding 16-byte chunk c, until the workgroup knows its
// role).  Ends with the routing in LDS (P.U, P.uexp; from router logits also
// the selection in rank order) after the last barrier.
template <int VPL, bool F16>
__device__ __forceinline__ void d1_start(const D1Args& a, D1Pro& P, u32x4_t* xv_out, int* parity_out) {
  const int tid = threadIdx.x, wave = uniform(tid >> 6);
  constexpr bool kRank = VPL * kWave <= kRankKeys;
  D1In<VPL> in;
  if (wave == 0 || (kRank && a.logits)) d1_issue<VPL>(a, in);  // from logits, every wave ranks
  const u32x2_t ev = __builtin_amdgcn_raw_buffer_load_b64(buffer_rsrc(a.epochs, (uint32_t)kEpochSlots * 8u),
                                                          blockIdx.x * 8u, 0, kCpolAgent);
  const __amdgpu_buffer_rsrc_t rx = buffer_rsrc(a.x, (uint32_t)a.H * 2u);
  *xv_out = __builtin_amdgcn_raw_buffer_load_b128(rx, tid < kMaxH / 8 ? (uint32_t)tid * 16u : kOob, 0, 0);
  RankKeys rk;
  if constexpr (kRank) {
    if (a.logits) {
#ifdef GI_TIMELINE
      __builtin_amdgcn_s_waitcnt(0x0F72);  // vmcnt(2): the routing inputs (the epoch word and x are younger)
      GI_STAMP(10);
#endif
      d1_rank_count(a, P, in.r, rk);
      GI_STAMP(16);
    }
  }
  if (wave == 0) {
#ifdef GI_TIMELINE
    if (!(kRank && a.logits)) {
      __builtin_amdgcn_s_waitcnt(0x0F72);
      GI_STAMP(10);
    }
#endif
    if (a.logits) {
      if constexpr (!kRank) {
        d1_select<VPL>(a, P, in.r);
        d1_rank_radix(a, P);
      } else if (tid == 0) {
        P.U = a.top_k;
      }
    } else {
      d1_route_ids<VPL, F16>(a, P, in);
    }
    GI_STAMP(11);
    if (tid == 0) {
      P.bad = 0;
      P.epoch = ((unsigned long long)ev.y << 32) | ev.x;
    }
  }
  lds_barrier();
  if constexpr (kRank) {
    if (a.logits) {
      if (tid < kRankKeys) d1_rank_pick(a, P, rk);
      GI_STAMP(17);
      lds_barrier();
    }
  }
  *parity_out = (int)((moe_state::epoch_count(P.epoch) + 1ull) & 1ull);
}

// ---------------------------------------------------------------------------
// items: gate/up on the matrix cores, activation, folded down products
// ---------------------------------------------------------------------------
struct ItemRegs {
  uint2 s[kGuSc];   // this lane's 4 columns' scales in the wave's groups
  uint4 w[kKbw];    // this lane's words: packed rows 4kb + lq of the wave's k blocks
  uint4 fw;         // folded down word: 4 columns x 8 rows
  uint2 fs;         // its scales
  uint32_t old;     // folded unit `item` (item < n_left, accumulating calls): previous output bits (t < 32)
};

__device__ __forceinline__ void item_load(const D1Args& a, int e, int it, int c, int Kv8, int n_whole, int n_left,
                                          ItemRegs& r) {
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = uniform(tid >> 6);
  {
    // folded unit n_whole + it, summed by this item (it < n_left)
    const __amdgpu_buffer_rsrc_t ro = buffer_rsrc(a.out, a.overwrite ? 0u : (uint32_t)a.H * 2u);
    const uint32_t off = (tid < 32 && it < n_left) ? (uint32_t)(32 * (n_whole + it) + tid) * 2u : kOob;
    r.old = __builtin_amdgcn_raw_buffer_load_b16(ro, off, 0, 0);
  }
  const int lq = lane >> 4, lr = lane & 15;
  const int twoI = 2 * a.I;
  const int col = (lr < 8 ? 0 : a.I) + 32 * c + 4 * (lr & 7);
  const int kb0 = wave * kKbw;
  const int g0 = kb0 >> a.gsh;
  const int nsc = ((kb0 + kKbw - 1) >> a.gsh) - g0 + 1;
  const __amdgpu_buffer_rsrc_t rs = buffer_rsrc(a.gu_scales + (size_t)e * (a.gus_bytes / 2), a.gus_bytes);
  const __amdgpu_buffer_rsrc_t rw = buffer_rsrc(a.gu_packed + (size_t)e * (a.gu_bytes / 4), a.gu_bytes);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int j = 0; j < kGuSc; ++j) {
    const int g = g0 + j;
    const uint32_t off = (j < nsc && g < a.Ggu) ? (uint32_t)((g * twoI + col) * 2) : kOob;
    const u32x2_t v = __builtin_amdgcn_raw_buffer_load_b64(rs, off, 0, 0);
    r.s[j] = make_uint2(v.x, v.y);
  }
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int j = 0; j < kKbw; ++j) {
    const int row = 4 * (kb0 + j) + lq;
    const uint32_t off = row < Kv8 ? (uint32_t)((row * twoI + col) * 4) : kOob;
    const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(rw, off, 0, kCpolNt);
    r.w[j] = make_uint4(v.x, v.y, v.z, v.w);
  }
  __builtin_amdgcn_sched_barrier(0);
  // folded units: thread (pr, fq) loads columns 32 n_whole + 4 fq of down row 4c + pr
  const int n_fq = n_left * 8;
  const int pr = n_fq > 0 ? tid / n_fq : 4, fq = n_fq > 0 ? tid - pr * n_fq : 0;
  const int gd = c >> a.gsh;
  const __amdgpu_buffer_rsrc_t rd = buffer_rsrc(a.d_packed + (size_t)e * (a.dn_bytes / 4), a.dn_bytes);
  const __amdgpu_buffer_rsrc_t rds = buffer_rsrc(a.d_scales + (size_t)e * (a.dsc_bytes / 2), a.dsc_bytes);
  const int fcol = 32 * n_whole + 4 * fq;
  const uint32_t woff = pr < 4 ? (uint32_t)(((4 * c + pr) * a.H + fcol) * 4) : kOob;
  const uint32_t soff = (pr == 0 && gd < a.Gd) ? (uint32_t)((gd * a.H + fcol) * 2) : kOob;
  const u32x4_t fv = __builtin_amdgcn_raw_buffer_load_b128(rd, woff, 0, kCpolNt);
  const u32x2_t sv = __builtin_amdgcn_raw_buffer_load_b64(rds, soff, 0, 0);
  r.fw = make_uint4(fv.x, fv.y, fv.z, fv.w);
  r.fs = make_uint2(sv.x, sv.y);
  __builtin_amdgcn_sched_barrier(0);
}

// The gate/up products of one wave's kKbw k blocks, whose first k block sits
// at phase PH of its scale group (group size 32 << GSH): y[i] (column quad
// lr's column i; lanes lr >= 8 hold up columns) = sum over groups of
// scale * (the group's products + its -24 * sum of x).  A group's first
// product starts from zero.
template <int GSH, int PH, bool F16>
__device__ __forceinline__ void item_products(const ItemRegs& r, const uint4* arow, float kbv, uint32_t mq,
                                              uint32_t mc, float (&y)[4]) {
  constexpr int kPg = 1 << GSH;
  const f32x4_t zf = {0.f, 0.f, 0.f, 0.f};
  f32x4_t D[4];
  float bacc = 0.f;
#pragma unroll
  for (int j = 0; j < kKbw; ++j) {
    const bool gstart = j == 0 || (PH + j) % kPg == 0;
    const uint4 A = arow[4 * j];
    const uint4 w = opaque(r.w[j]);
#ifdef GI_TIMELINE
    if (j == 0 || j == kKbw - 1) {
      asm volatile("" ::"v"(w.x), "v"(w.w));
      if (j == 0) GI_STAMP(20);
      else GI_STAMP(21);
    }
#endif
    D[0] = mfma_bf16(A, q4_operand_fast(w.x, mq, mc), gstart ? zf : D[0]);
    D[1] = mfma_bf16(A, q4_operand_fast(w.y, mq, mc), gstart ? zf : D[1]);
    D[2] = mfma_bf16(A, q4_operand_fast(w.z, mq, mc), gstart ? zf : D[2]);
    D[3] = mfma_bf16(A, q4_operand_fast(w.w, mq, mc), gstart ? zf : D[3]);
    bacc = (gstart ? 0.f : bacc) + __int_as_float(__builtin_amdgcn_readlane(__float_as_int(kbv), 4 * j));
    if ((PH + j + 1) % kPg == 0 || j == kKbw - 1) {  // a scale group ends
      const uint2 s2 = opaque(r.s[(PH + j) / kPg]);  // opaque: the variants' epilogues stay apart
      const float sc[4] = {sc_lo<F16>(s2.x), sc_hi<F16>(s2.x), sc_lo<F16>(s2.y), sc_hi<F16>(s2.y)};
#pragma unroll
      for (int i = 0; i < 4; ++i) y[i] += sc[i] * ((F16 ? D[i][0] + D[i][1] : D[i][0]) + bacc);
    }
  }
}

template <int GSH, bool F16>
__device__ __forceinline__ void item_run(const D1Args& a, const D1Pro& P, ItemLds<F16>& L, int it, int u, int c,
                                         int n_left, char* act, char* part, const ItemRegs& r) {
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = uniform(tid >> 6);
  const int lq = lane >> 4, lr = lane & 15;
  const int gsh = gsh_of<GSH>(a);
  const int kb0 = wave * kKbw;
  const int g0 = kb0 >> gsh;
  const int kbpg_m1 = (1 << gsh) - 1;
  // -24 * each of the wave's k blocks' sum of x: lane 4j holds k block kb0 + j's
  float kbv = P.cb[min(4 * kb0 + lane, kMaxH / 8 - 1)];
  kbv = lane < 4 * kKbw ? kbv : 0.f;
  kbv += dpp_f32<0xB1>(kbv);  // quad_perm [1,0,3,2]
  kbv += dpp_f32<0x4E>(kbv);  // quad_perm [2,3,0,1]
  const uint32_t mq = q4_magic();
  const uint32_t mc = q4_high_bits();
  // A row 0 is the token (lanes lr == 0 read x), rows 1-15 are zero (the
  // other lanes read the zero block at the same offsets): no select per k block
  // (fp16: row 1 is x's lo part)
  const uint4* arow = lr == 0 ? L.xs + 4 * kb0 + lq : (F16 && lr == 1) ? L.xs_lo + 4 * kb0 + lq : L.xz + lq;
  float y[4] = {0.f, 0.f, 0.f, 0.f};
  if constexpr (GSH > 0) {
    // the wave's first k block sits at phase kb0 % (k blocks per group) of
    // its group: with the phase a compile-time value, every group end, group
    // start and scale register of the loop is known to the compiler
    constexpr int kPh = 1 << GSH;
    const int ph = kb0 & (kPh - 1);
    if (ph == 0) item_products<GSH, 0, F16>(r, arow, kbv, mq, mc, y);
    else if (kPh > 1 && ph == 1) item_products<GSH, (kPh > 1 ? 1 : 0), F16>(r, arow, kbv, mq, mc, y);
    else if (kPh > 2 && ph == 2) item_products<GSH, (kPh > 2 ? 2 : 0), F16>(r, arow, kbv, mq, mc, y);
    else if (kPh > 3 && ph == 3) item_products<GSH, (kPh > 3 ? 3 : 0), F16>(r, arow, kbv, mq, mc, y);
    else if (kPh > 4 && ph == 4) item_products<GSH, (kPh > 4 ? 4 : 0), F16>(r, arow, kbv, mq, mc, y);
    else if (kPh > 5 && ph == 5) item_products<GSH, (kPh > 5 ? 5 : 0), F16>(r, arow, kbv, mq, mc, y);
    else if (kPh > 6 && ph == 6) item_products<GSH, (kPh > 6 ? 6 : 0), F16>(r, arow, kbv, mq, mc, y);
    else item_products<GSH, (kPh > 7 ? 7 : 0), F16>(r, arow, kbv, mq, mc, y);
  } else {
    const f32x4_t zf = {0.f, 0.f, 0.f, 0.f};
    f32x4_t D[4] = {zf, zf, zf, zf};
    float bacc = 0.f;
#pragma unroll
    for (int j = 0; j < kKbw; ++j) {
      const int kb = kb0 + j;
      const uint4 A = arow[4 * j];
      const uint4 w = opaque(r.w[j]);
      D[0] = mfma_bf16(A, q4_operand_fast(w.x, mq, mc), D[0]);
      D[1] = mfma_bf16(A, q4_operand_fast(w.y, mq, mc), D[1]);
      D[2] = mfma_bf16(A, q4_operand_fast(w.z, mq, mc), D[2]);
      D[3] = mfma_bf16(A, q4_operand_fast(w.w, mq, mc), D[3]);
      bacc += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(kbv), 4 * j));
      if (((kb + 1) & kbpg_m1) == 0 || j == kKbw - 1) {  // a scale group ends
        const int gi = (kb >> gsh) - g0;
        uint2 s2 = opaque(r.s[0]);
#pragma unroll
        for (int q = 1; q < kGuSc; ++q)
          if (gi == q) s2 = opaque(r.s[q]);
        const float sc[4] = {sc_lo<F16>(s2.x), sc_hi<F16>(s2.x), sc_lo<F16>(s2.y), sc_hi<F16>(s2.y)};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          y[i] += sc[i] * ((F16 ? D[i][0] + D[i][1] : D[i][0]) + bacc);
          D[i] = zf;
        }
        bacc = 0.f;
      }
    }
  }
  if (lq == 0) L.red[wave][lr] = make_float4(y[0], y[1], y[2], y[3]);
  lds_barrier();
  GI_STAMP(4);
  const int Iv = min(a.I, a.Gd << (a.gsh + 5));  // activations past the last down group are dropped
  if (tid < 32) {
    float g = 0.f, up = 0.f;
#pragma unroll
    for (int w2 = 0; w2 < kW; ++w2) {
      const float* rg = (const float*)&L.red[w2][tid >> 2];
      const float* ru = (const float*)&L.red[w2][8 + (tid >> 2)];
      g += rg[tid & 3];
      up += ru[tid & 3];
    }
    const float av = (32 * c + tid < Iv) ? gelu_tanh(g) * up : 0.f;
    const uint16_t bits = act_signal_bits<F16>(av);  // rounded to the activation dtype, canonical NaN
    ((uint16_t*)L.sa)[(tid & ~7) + mfma_k_pos(tid & 7)] = bits;
  }
  lds_barrier();
  // publish: 16 bytes per 8 activations, inverted; the data is the signal
  if (tid < 4) {
    const uint4 v = L.sa[tid];
    u32x4_t vv;
    vv.x = ~v.x;
    vv.y = ~v.y;
    vv.z = ~v.z;
    vv.w = ~v.w;
    __builtin_amdgcn_raw_buffer_store_b128(vv, buffer_rsrc(act, kActParity),
                                           (uint32_t)((u * a.I + 32 * c + 8 * tid) * 2), 0, kCpolAgent);
  }
  GI_STAMP(5);
  if (n_left == 0) return;
  // folded units: thread (pr, fq): its word times activation chunk pr
  const int n_fq = n_left * 8;
  const int pr = tid / n_fq, fq = tid - pr * n_fq;
  if (pr < 4) {
    const uint4 A = L.sa[pr];
    float s[4];
    const uint32_t wv[4] = {r.fw.x, r.fw.y, r.fw.z, r.fw.w};
    if constexpr (F16) {
      uint4 Ah, Al;
      f16_split(A, Ah, Al);
      const float bias = q4_bias(Ah) + q4_bias(Al);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const Q4Pairs q = unpack_q4(wv[i], mq);
        s[i] = dot_chunk(Al, q, dot_chunk(Ah, q, bias));
      }
    } else {
      const float bias = q4_bias(A);
#pragma unroll
      for (int i = 0; i < 4; ++i) s[i] = dot_chunk(A, unpack_q4(wv[i], mq), bias);
    }
    L.fr[pr][fq] = make_float4(s[0], s[1], s[2], s[3]);
  }
  lds_barrier();
  if (tid < n_fq) {
    const float wu = P.uw[u];
    const float4 f0 = L.fr[0][tid], f1 = L.fr[1][tid], f2 = L.fr[2][tid], f3 = L.fr[3][tid];
    const float v0 = ((f0.x + f1.x) + f2.x) + f3.x, v1 = ((f0.y + f1.y) + f2.y) + f3.y;
    const float v2 = ((f0.z + f1.z) + f2.z) + f3.z, v3 = ((f0.w + f1.w) + f2.w) + f3.w;
    u32x4_t o;
    o.x = f32_signal_bits((wu * sc_lo<F16>(r.fs.x)) * v0);
    o.y = f32_signal_bits((wu * sc_hi<F16>(r.fs.x)) * v1);
    o.z = f32_signal_bits((wu * sc_lo<F16>(r.fs.y)) * v2);
    o.w = f32_signal_bits((wu * sc_hi<F16>(r.fs.y)) * v3);
    __builtin_amdgcn_raw_buffer_store_b128(o, buffer_rsrc(part, kPartParity),
                                           (uint32_t)((it * n_fq * 4 + 4 * tid) * 4), 0, kCpolAgent);
  }
  GI_STAMP(6);
}

// ---------------------------------------------------------------------------
// units: down products of 32 output columns over every expert
// ---------------------------------------------------------------------------
// Wave w holds expert w (U <= kW): step s covers its k blocks 2s (lanes
// lr < 8, A row 0) and 2s + 1 (lanes lr >= 8, A row 1); lane (lq, lr) loads
// the 4 columns 32d + 4(lr & 7) of packed row 4kb + lq.  NS = ceil(Tk / 2).
template <int NS>
struct UnitRegs {
  uint4 w[NS];
  uint4 sc;      // one down-scale chunk (staged into LDS)
  uint32_t old;  // previous output bits of this unit (accumulating calls, t < 32)
};

template <int NS>
__device__ __forceinline__ void unit_load(const D1Args& a, const D1Pro& P, int d, int U, int n_whole, int n_left,
                                          UnitRegs<NS>& r) {
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = uniform(tid >> 6);
  const int lq = lane >> 4, lr = lane & 15;
  const __amdgpu_buffer_rsrc_t ro = buffer_rsrc(a.out, a.overwrite ? 0u : (uint32_t)a.H * 2u);
  {
    const uint32_t off = tid < 32 ? (uint32_t)(32 * d + tid) * 2u : kOob;
    r.old = __builtin_amdgcn_raw_buffer_load_b16(ro, off, 0, 0);
  }
  // down scales of the unit's columns: chunk ch = (u * Gd + g) * 4 + q holds columns 8q .. 8q+7
  {
    const int ch = tid, ug = ch >> 2, q = ch & 3;
    const int u = ug / a.Gd, g = ug - u * a.Gd;
    const int e = P.uexp[min(u, kMaxU - 1)];
    const uint32_t off = ch < U * a.Gd * 4 ? (uint32_t)((g * a.H + 32 * d + 8 * q) * 2) + (uint32_t)e * a.dsc_bytes
                                           : kOob;
    const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(buffer_rsrc(a.d_scales, a.dsc_total), off, 0, 0);
    r.sc = make_uint4(v.x, v.y, v.z, v.w);
  }
  // the wave's expert: one buffer resource (empty for waves past U)
  const int e = uniform(P.uexp[min(wave, kMaxU - 1)]);
  const __amdgpu_buffer_rsrc_t rw =
      buffer_rsrc(a.d_packed + (size_t)(wave < U ? e : 0) * (a.dn_bytes / 4), wave < U ? a.dn_bytes : 0u);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const int kb = 2 * s + (lr >> 3);
    const uint32_t off = kb < a.Tk ? (uint32_t)(((4 * kb + lq) * a.H + 32 * d + 4 * (lr & 7)) * 4) : kOob;
    const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(rw, off, 0, kCpolNt);
    r.w[s] = make_uint4(v.x, v.y, v.z, v.w);
  }
  __builtin_amdgcn_sched_barrier(0);
}

// One wave polls the n chunks (16 bytes each, lane + 64j) of `src` into dst
// (all of them present: no 16-bit half zero), inverted back, with chunk
// lane + 64j's -24 * sum of its 8 values in bias[j] (bf16; the fp16 products
// on q - 8 operands need none).  Bounded: on timeout the status word and host
// flag are set, *bad is set and the wave goes on.
template <int CPT, bool F16>
__device__ __forceinline__ void poll_chunks(const D1Args& a, const __amdgpu_buffer_rsrc_t src, uint4* dst,
                                            float (&bias)[CPT], int n, int* bad) {
  const int lane = threadIdx.x & (kWave - 1);
  uint32_t pending = 0u;
#pragma unroll
  for (int j = 0; j < CPT; ++j) {
    bias[j] = 0.f;
    if (lane + j * kWave < n) pending |= 1u << j;
  }
  int spins = 0;
  while (true) {
    u32x4_t v[CPT];
#pragma unroll
    for (int j = 0; j < CPT; ++j)
      v[j] = __builtin_amdgcn_raw_buffer_load_b128(src, ((pending >> j) & 1u) ? (uint32_t)(lane + j * kWave) * 16u : kOob,
                                                   0, kCpolAgent);
#pragma unroll
    for (int j = 0; j < CPT; ++j) {
      if (((pending >> j) & 1u) && chunk_ready(v[j])) {
        const uint4 x = make_uint4(~v[j].x, ~v[j].y, ~v[j].z, ~v[j].w);
        dst[lane + j * kWave] = x;
        if constexpr (!F16) bias[j] = q4_bias(x);
        pending &= ~(1u << j);
      }
    }
    if (__ballot(pending != 0u) == 0ull) break;
    if (++spins >= a.spin_limit) {
      if (lane == 0) {
        report_timeout(a.status, a.host_flag);
        *bad = 1;
      }
      break;
    }
    __builtin_amdgcn_s_sleep(2);
    asm volatile("" ::: "memory");
  }
}

// Loads of the pending chunks of a folded unit's partial sums: item st + 64j,
// columns 32d + 4cq .. +3 (16 bytes; offsets of chunks not pending read nothing).
__device__ __forceinline__ void folded_poll(const __amdgpu_buffer_rsrc_t rp, int st, int d, int cq, int stride,
                                            uint32_t pending, u32x4_t (&v)[4]) {
#pragma unroll
  for (int j = 0; j < 4; ++j)
    v[j] = __builtin_amdgcn_raw_buffer_load_b128(
        rp, ((pending >> j) & 1u) ? (uint32_t)(((st + 64 * j) * stride + 32 * d + 4 * cq) * 4) : kOob, 0, kCpolAgent);
}

// The products of one scale group, finished: y += scale * (the group's sum +
// its -24 * sum of activations); lanes lr < 8 take A row 0 (k block 2s),
// lanes lr >= 8 row 1 (k block 2s + 1).
// (fp16: the same rows, fp16 products on q - 8 operands, bacc zero)
template <bool F16>
__device__ __forceinline__ void group_epilogue(float (&y)[4], const f32x4_t (&D)[4], uint2 s2, float bacc, int h) {
  const float sc[4] = {sc_lo<F16>(s2.x), sc_hi<F16>(s2.x), sc_lo<F16>(s2.y), sc_hi<F16>(s2.y)};
#pragma unroll
  for (int i = 0; i < 4; ++i) y[i] += sc[i] * ((h ? D[i][1] : D[i][0]) + bacc);
}

template <int NS, int GSH, bool F16>
__device__ __forceinline__ void unit_run(const D1Args& a, D1Pro& P, UnitLds<F16>& L, int d, int U, const char* act,
                                         const UnitRegs<NS>& r, int parity, int cslot, int nslots) {
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = uniform(tid >> 6);
  const int lq = lane >> 4, lr = lane & 15, h = lr >> 3;
  const int Tk = a.Tk, cps = a.I >> 3;
  int* bad = &P.bad;
  if (tid < U * a.Gd * 4) L.dsc[tid] = r.sc;
  // the words as matrix-core operands, while the activations are on their way
  // (fp16: exact fp16 q - 8, for fp16 products with no offset term)
  const uint32_t mq = q4_magic_t<F16>();
  const uint32_t mc = q4_high_bits();
  uint4 B[NS][4];
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const uint4 w = r.w[s];
    B[s][0] = q4_operand_fast_t<F16>(w.x, mq, mc);
    B[s][1] = q4_operand_fast_t<F16>(w.y, mq, mc);
    B[s][2] = q4_operand_fast_t<F16>(w.z, mq, mc);
    B[s][3] = q4_operand_fast_t<F16>(w.w, mq, mc);
    // here, not next to the products: the unpacking overlaps the wait
#pragma unroll
    for (int i = 0; i < 4; ++i) asm volatile("" : "+v"(B[s][i].x), "+v"(B[s][i].y), "+v"(B[s][i].z), "+v"(B[s][i].w));
  }
  GI_STAMP(3);
  // the previous launch's footprint (clearing workgroups): the stores go out
  // while the activations are computed elsewhere
  if (cslot >= 0) {
    clear_prev(a, P.epoch, parity, cslot, nslots);
    GI_STAMP(15);
  }
  lds_barrier();  // the down scales staged by every wave
  const f32x4_t zf = {0.f, 0.f, 0.f, 0.f};
  const uint4 z4 = make_uint4(0u, 0u, 0u, 0u);
  const int u = wave;
  const int uc = min(u, kMaxU - 1);
  const int gsh = gsh_of<GSH>(a);
  const int gpb_m1 = (1 << gsh) - 1;  // k blocks per scale group - 1 (odd: groups hold whole steps)
  float y[4] = {0.f, 0.f, 0.f, 0.f};
  if (u < U) {
    // wave u waits for expert u's activations only (its products start as
    // soon as they are there), with each chunk's -24 * sum
    float cb[2];
    poll_chunks<2, F16>(a, buffer_rsrc(act + (size_t)u * a.I * 2, (uint32_t)(a.I * 2)), L.sact + u * cps, cb, cps,
                        bad);
    GI_STAMP(4);
    GI_STAMP_BY(20, (U - 1) * kWave);
    // -24 * the sum of k block kb's activations: k block kb is chunks 4kb ..
    // 4kb+3, held by lanes 4(kb % 16) .. +3 in cb[kb / 16]; summed over each
    // quad of lanes in registers ((c0 + c1) + (c2 + c3) in every lane of it),
    // read with readlane per step (fp16: none)
    float kq[2] = {0.f, 0.f};
    if constexpr (!F16) {
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const float v = cb[j] + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(cb[j]), 0xB1, 0xF, 0xF,
                                                                            false));  // quad_perm [1,0,3,2]
        kq[j] = v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF,
                                                                false));  // quad_perm [2,3,0,1]
      }
    }
    // A rows 0, 1: k blocks 2s, 2s+1 (lanes lr < 2), read three steps ahead
    const int rowoff = uc * cps + lq;
    const int kbo = lr & 1;
    const uint4* srow = L.sact;
    constexpr int kArows = 2;
    constexpr int kAhead = 3;
    uint4 an[kAhead];
#pragma unroll
    for (int s = 0; s < kAhead; ++s) an[s] = srow[rowoff + min(4 * (2 * s + kbo), cps - 4)];
    // two accumulator sets, alternating by scale group: a group's scale is
    // applied after the next group's products are issued, so that the
    // epilogue does not wait for the matrix cores (the sets are named, not
    // indexed, so that they stay in registers when the group size is a
    // run-time value)
    // each step's offset sum for this lane's k block (2s + h), read before the steps
    float kb_off[NS];
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      kb_off[s] = 0.f;
      if constexpr (!F16) {
        const int k0 = 2 * s, k1 = 2 * s + 1;
        const float b0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(kq[(k0 >> 4) & 1]), 4 * (k0 & 15)));
        const float b1 =
            k1 < Tk ? __int_as_float(__builtin_amdgcn_readlane(__float_as_int(kq[(k1 >> 4) & 1]), 4 * (k1 & 15)))
                    : 0.f;
        kb_off[s] = h ? b1 : b0;
      }
    }
    f32x4_t D0[4], D1[4];
    uint2 s20 = make_uint2(0u, 0u), s21 = make_uint2(0u, 0u);
    float bacc0 = 0.f, bacc1 = 0.f;
    auto step = [&](int s, const uint4& A, bool gstart, bool epi, int g, f32x4_t(&Dc)[4], uint2& s2c, float& bc,
                    const f32x4_t(&Dp)[4], uint2 s2p, float bp) {
      if (gstart) {
        const int gg = min(g, a.Gd - 1);
        s2c = *(const uint2*)((const uint16_t*)&L.dsc[(uc * a.Gd + gg) * 4] + 4 * (lr & 7));
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) Dc[i] = mfma_act<F16>(A, B[s][i], gstart ? zf : Dc[i]);
      if constexpr (!F16) bc = (gstart ? 0.f : bc) + kb_off[s];
      if (epi) group_epilogue<F16>(y, Dp, s2p, bp, h);
    };
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const int kba = 2 * s + kbo;
      const uint4 A = (lr < kArows && kba < Tk) ? an[s % kAhead] : z4;
      if (s + kAhead < NS) an[s % kAhead] = srow[rowoff + min(4 * (kba + 2 * kAhead), cps - 4)];
      const int g = (2 * s) >> gsh;
      const bool gstart = ((2 * s) & gpb_m1) == 0;
      const bool epi = gstart && g > 0;
      if ((g & 1) == 0) step(s, A, gstart, epi, g, D0, s20, bacc0, D1, s21, bacc1);
      else step(s, A, gstart, epi, g, D1, s21, bacc1, D0, s20, bacc0);
    }
    GI_STAMP(21);
    if ((((2 * (NS - 1)) >> gsh) & 1) == 0) group_epilogue<F16>(y, D0, s20, bacc0, h);
    else group_epilogue<F16>(y, D1, s21, bacc1, h);
#ifdef GI_TIMELINE
    asm volatile("" ::"v"(y[0]), "v"(y[1]), "v"(y[2]), "v"(y[3]));
#endif
    GI_STAMP(22);
  }
  const float wu = u < U ? P.uw[uc] : 0.f;
  if (lq == 0) L.red[wave][lr] = make_float4(wu * y[0], wu * y[1], wu * y[2], wu * y[3]);
  lds_barrier();
  GI_STAMP(5);
  if (tid < 32) {
    float sacc = 0.f;
#pragma unroll
    for (int w2 = 0; w2 < kW; ++w2) {
      sacc += ((const float*)&L.red[w2][tid >> 2])[tid & 3];
      sacc += ((const float*)&L.red[w2][8 + (tid >> 2)])[tid & 3];
    }
    if (!a.overwrite) sacc += act_to_f32<F16>(r.old & 0xffffu);
    if (P.bad) sacc = __uint_as_float(0x7fc00000u);  // never a wrong finite value
    a.out[32 * d + tid] = f32_to_act<F16>(sacc);
  }
  GI_STAMP(6);
}

// Folded unit n_whole + f (item f < n_left, after its own work): the items'
// partial sums of its 32 columns, 64 item streams (items st, st + 64, ...) x
// 8 column quads, polled with a bounded wait and added in a fixed order: each
// thread's items in order, then the wave's 8 streams (xor 8, 16, 32), then
// the 8 waves in order; one bf16 rounding (plus the previous output).
template <bool F16>
__device__ __forceinline__ void folded_reduce(const D1Args& a, D1Pro& P, float4 (&rr)[kW][8], int f, int n_items,
                                              int n_whole, int n_left, const char* part, uint32_t old) {
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = uniform(tid >> 6);
  const int fcq = tid & 7, fst = tid >> 3;
  const int fstride = n_left * 32;  // floats per item
  const __amdgpu_buffer_rsrc_t frp = buffer_rsrc(part, (uint32_t)(n_items * fstride * 4));
  uint32_t fpend = 0u;
#pragma unroll
  for (int j = 0; j < 4; ++j)
    if (fst + 64 * j < n_items) fpend |= 1u << j;
  u32x4_t fv[4];
  float4 got[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) got[j] = make_float4(0.f, 0.f, 0.f, 0.f);
  int spins = 0;
  while (true) {
    folded_poll(frp, fst, f, fcq, fstride, fpend, fv);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (((fpend >> j) & 1u) && fv[j].x != 0u && fv[j].y != 0u && fv[j].z != 0u && fv[j].w != 0u) {
        got[j] = make_float4(__uint_as_float(~fv[j].x), __uint_as_float(~fv[j].y), __uint_as_float(~fv[j].z),
                             __uint_as_float(~fv[j].w));
        fpend &= ~(1u << j);
      }
    }
    if (__ballot(fpend != 0u) == 0ull) break;
    if (++spins >= a.spin_limit) {
      if (lane == 0) {
        report_timeout(a.status, a.host_flag);
        P.bad = 1;
      }
      break;
    }
    __builtin_amdgcn_s_sleep(2);
    asm volatile("" ::: "memory");
  }
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    if (fst + 64 * j < n_items) {
      acc.x += got[j].x;
      acc.y += got[j].y;
      acc.z += got[j].z;
      acc.w += got[j].w;
    }
  }
#pragma unroll
  for (int off = 8; off < kWave; off <<= 1) {
    acc.x += __shfl_xor(acc.x, off, kWave);
    acc.y += __shfl_xor(acc.y, off, kWave);
    acc.z += __shfl_xor(acc.z, off, kWave);
    acc.w += __shfl_xor(acc.w, off, kWave);
  }
  if (lane < 8) rr[wave][lane] = acc;
  lds_barrier();
  if (tid < 32) {
    float sacc = 0.f;
#pragma unroll
    for (int w2 = 0; w2 < kW; ++w2) sacc += ((const float*)&rr[w2][tid >> 2])[tid & 3];
    if (!a.overwrite) sacc += act_to_f32<F16>(old & 0xffffu);
    if (P.bad) sacc = __uint_as_float(0x7fc00000u);
    a.out[32 * (n_whole + f) + tid] = f32_to_act<F16>(sacc);
  }
  GI_STAMP(7);
}

// ---------------------------------------------------------------------------
// kernel
// ---------------------------------------------------------------------------
template <int NS, int GSH, bool F16>
__global__ __launch_bounds__(kT) void moe_decode1_kernel(D1Args a) {
  __shared__ D1Pro P;
  __shared__ D1Lds<F16> L;
#ifdef GI_TIMELINE
  tl_init();
#endif
  GI_STAMP(0);
  int parity = 0;
  u32x4_t xv;
  if (a.E <= 2 * kWave) d1_start<2, F16>(a, P, &xv, &parity);
  else if (a.E <= 4 * kWave) d1_start<4, F16>(a, P, &xv, &parity);
  else if (a.E <= 8 * kWave) d1_start<8, F16>(a, P, &xv, &parity);
  else d1_start<kRouteMaxExperts / kWave, F16>(a, P, &xv, &parity);
  GI_STAMP(1);
  const int tid = threadIdx.x;
  const int b = blockIdx.x, G = gridDim.x;
  const int U = uniform(P.U);
  char* act = a.act + (size_t)parity * kActParity;
  char* part = a.part + (size_t)parity * kPartParity;
  const d1::Split sp = d1::split(G, U, a.Tk, a.units);
  const int n_items = sp.n_items, n_whole = sp.n_whole, n_left = sp.n_left;
  const int Kv8 = min(a.H >> 3, a.Ggu << (a.gsh + 2));  // packed rows inside the gate/up scale groups
  // the workgroups that clear the previous launch's footprint: the idle ones
  // if there are any, else the units (they wait for the activations), else all
  const int n_idle = G - n_items - n_whole;
  const int c0 = n_idle > 0 ? n_items + n_whole : (n_whole > 0 ? n_items : 0);
  const int nc = n_idle > 0 ? n_idle : (n_whole > 0 ? n_whole : G);
  const int cslot = (b >= c0 && b < c0 + nc) ? b - c0 : -1;
#ifdef GI_TIMELINE
  tl_value(29, 2ull);
  tl_value(30, b < n_items ? 1ull : (b - n_items < n_whole ? 2ull : 0ull));
  tl_value(31, (unsigned long long)(b < n_items ? b : b - n_items));
#endif
  if (U == 0) {
    if (a.overwrite && b == 0)
      for (int i = tid; i < a.H; i += kT) a.out[i] = 0;  // a layer call owns out
    if (cslot >= 0) clear_prev(a, P.epoch, parity, cslot, nc);
  } else if (b < n_items) {
    const int u = b / a.Tk, c = b - u * a.Tk;
    ItemRegs r;
    item_load(a, uniform(P.uexp[u]), b, c, Kv8, n_whole, n_left, r);
    GI_STAMP(2);
    // x in LDS in the matrix-core k order, with each chunk's -24 * sum
    if (tid < kMaxH / 8) {
      const uint4 v = make_uint4(xv.x, xv.y, xv.z, xv.w);
      const uint4 z = make_uint4(0u, 0u, 0u, 0u);
      if constexpr (F16) {
        uint4 vh, vl;
        f16_split(v, vh, vl);
        L.it.xs[tid] = tid < Kv8 ? mfma_k_order(vh) : z;
        L.it.xs_lo[tid] = tid < Kv8 ? mfma_k_order(vl) : z;
        P.cb[tid] = tid < Kv8 ? q4_bias(vh) + q4_bias(vl) : 0.f;
      } else {
        L.it.xs[tid] = tid < Kv8 ? mfma_k_order(v) : z;
        P.cb[tid] = tid < Kv8 ? q4_bias(v) : 0.f;
      }
    } else if (tid < kMaxH / 8 + 4 * kKbw) {
      L.it.xz[tid - kMaxH / 8] = make_uint4(0u, 0u, 0u, 0u);
    }
    GI_STAMP_BY(14, kWave);
    if (a.logits && tid < kWave) d1_weights(a, P);
    lds_barrier();
    item_run<GSH, F16>(a, P, L.it, b, u, c, n_left, act, part, r);
    if (b < n_left) folded_reduce<F16>(a, P, L.it.rr, b, n_items, n_whole, n_left, part, r.old);
    if (cslot >= 0) clear_prev(a, P.epoch, parity, cslot, nc);
  } else if (b - n_items < n_whole) {
    const int d = b - n_items;
    UnitRegs<NS> r;
    // The units' words are needed only after the activation exchange: issued
    // right after the routing they would share the HBM with the items' words,
    // whose products are on the critical path.  Hold them back for about the
    // time the items' bytes take (a bounded wait on the constant clock).
    {
      const uint32_t item_bytes = 32u * (uint32_t)a.H + 128u * (uint32_t)a.Ggu;
      const unsigned long long hold = (unsigned long long)n_items * item_bytes / kUnitHoldBytesPerTick;
      const unsigned long long t0 = __builtin_amdgcn_s_memrealtime();
      while (__builtin_amdgcn_s_memrealtime() - t0 < hold) __builtin_amdgcn_s_sleep(4);
    }
    unit_load<NS>(a, P, d, U, n_whole, n_left, r);
    GI_STAMP(2);
    if (a.logits && tid < kWave) d1_weights(a, P);  // read after the unit's next barrier
    unit_run<NS, GSH, F16>(a, P, L.un, d, U, act, r, parity, cslot, nc);
  } else if (cslot >= 0) {
    clear_prev(a, P.epoch, parity, cslot, nc);
  }
  // the end: routing report (workgroup 0), the next epoch word with this launch's footprint
  if (b == 0 && a.logits && tid < a.top_k) {
    if (a.out_idx) a.out_idx[tid] = P.slot_e[tid];
    if (a.out_w) a.out_w[tid] = f32_to_bf16(P.slot_w[tid]);
  }
  if (tid == 0) {
    const unsigned long long ep = moe_state::epoch_count(P.epoch) + 1ull;
    const uint32_t au = moe_state::bytes_to_units((size_t)U * a.I * 2);
    const uint32_t pu = moe_state::bytes_to_units((size_t)n_items * n_left * 32 * 4);
    const unsigned long long wv = moe_state::epoch_word(ep, au, pu);
    for (int j = b; j < kEpochSlots; j += G)
      __hip_atomic_store(a.epochs + j, wv, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  GI_STAMP(9);
#ifdef GI_TIMELINE
  tl_flush(a.timeline);
#endif
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
int log2_exact(int v) {
  int s = 0;
  while ((1 << s) < v) ++s;
  return (1 << s) == v ? s : -1;
}

// Unit steps per wave (two k blocks each) for Tk = I / 32: the instantiated
// count at or above ceil(Tk / 2); steps past Tk read nothing.
// The Gemma shape (Tk = 22) also has variants with the group size fixed at
// compile time (64 and 128).
constexpr int kStepCounts[] = {2, 4, 6, 8, 11, 12};
constexpr int kNumSteps = (int)(sizeof(kStepCounts) / sizeof(kStepCounts[0]));
constexpr int kNumVariants = kNumSteps + 2;
int variant_for(int Tk, int gsh) {
  for (int i = 0; i < kNumSteps; ++i)
    if (2 * kStepCounts[i] >= Tk) {
      if (kStepCounts[i] == 11 && gsh == 1) return kNumSteps;
      if (kStepCounts[i] == 11 && gsh == 2) return kNumSteps + 1;
      return i;
    }
  return -1;
}
template <bool F16>
const void* kernel_for_t(int v) {
  switch (v) {
    case 0: return (const void*)moe_decode1_kernel<2, 0, F16>;
    case 1: return (const void*)moe_decode1_kernel<4, 0, F16>;
    case 2: return (const void*)moe_decode1_kernel<6, 0, F16>;
    case 3: return (const void*)moe_decode1_kernel<8, 0, F16>;
    case 4: return (const void*)moe_decode1_kernel<11, 0, F16>;
    case 5: return (const void*)moe_decode1_kernel<12, 0, F16>;
    case 6: return (const void*)moe_decode1_kernel<11, 1, F16>;
    default: return (const void*)moe_decode1_kernel<11, 2, F16>;
  }
}
// variants [0, kNumVariants): bf16 activations; [kNumVariants, 2 kNumVariants): fp16
const void* kernel_for(int v) {
  return v < kNumVariants ? kernel_for_t<false>(v) : kernel_for_t<true>(v - kNumVariants);
}

// Every workgroup of a launch (one per CU) must be resident at once: the
// occupancy calculator must put one on every CU (cached per device and variant).
std::mutex g_occ_mu;
int g_occ[64][2 * kNumVariants];  // 0 unknown, 1 resident, -1 not

bool resident_everywhere(int v) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return false;
  std::lock_guard<std::mutex> lk(g_occ_mu);
  if (g_occ[dev][v] == 0) {
    int n = 0;
    const hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kernel_for(v), kT, 0);
    if (e != hipSuccess) (void)hipGetLastError();
    g_occ[dev][v] = (e == hipSuccess && n >= 1) ? 1 : -1;
  }
  return g_occ[dev][v] == 1;
}

int grid_for() {
  const int cus = device_cu_count();
  return cus < kEpochSlots ? cus : kEpochSlots;
}

}  // namespace

bool moe_decode1_supported(const MoeHostArgs& h) {
  if (h.M != 1) return false;
  if (h.H % 32 || h.H > kMaxH || h.I % 32 || h.I > 32 * kMaxTk) return false;
  if (h.gs % 32 || log2_exact(h.gs / 32) < 1) return false;  // a group spans whole k blocks, at least 2
  if (h.Gd > kMaxGd || h.Ggu < 1 || h.Gd < 1) return false;
  if (h.top_k < 1 || h.top_k > kSlots || h.E > kRouteMaxExperts) return false;
  if (h.logits && h.top_k > h.E) return false;
  if ((((uintptr_t)h.gu_scales) | ((uintptr_t)h.d_scales) | ((uintptr_t)h.x)) % 16) return false;
  // whole tensors addressed with 32-bit buffer offsets
  if ((long long)h.E * (h.H / 8) * 2 * h.I * 4 >= (1LL << 32)) return false;
  if ((long long)h.E * (h.I / 8) * h.H * 4 >= (1LL << 32)) return false;
  if ((long long)h.E * h.Gd * h.H * 2 >= (1LL << 32)) return false;
  if ((long long)h.E * h.Ggu * 2 * h.I * 2 >= (1LL << 32)) return false;
  const int G = grid_for();
  const int Tk = h.I / 32, units = h.H / 32;
  const int umax = h.top_k < h.E ? h.top_k : h.E;
  const int v0 = variant_for(Tk, log2_exact(h.gs / 32));
  if (v0 < 0 || umax > kMaxU || !d1::split_ok(G, umax, Tk, units, kMaxLeft)) return false;
  // bf16, or fp16 from caller ids (the layer-from-logits entry is bf16 only)
  if (h.x_dtype != GI_DTYPE_BF16 && !(h.x_dtype == GI_DTYPE_FP16 && !h.logits)) return false;
  const int v = v0 + (h.x_dtype == GI_DTYPE_FP16 ? kNumVariants : 0);
  if (umax * h.Gd * 4 > kT) return false;  // down-scale staging: one chunk per thread
  // the split at the most unique experts (fewer experts only shrink the folded part)
  const d1::Split sp = d1::split(G, umax, Tk, units);
  if ((size_t)sp.n_items * sp.n_left * 32 * 4 > kPartParity) return false;
  if ((size_t)umax * h.I * 2 > kActParity) return false;
  return resident_everywhere(v);
}

int launch_moe_decode1(const MoeHostArgs& h, void* state, int* status) {
  D1Args k{};
  k.x = (const uint16_t*)h.x;
  k.gu_packed = h.gu_packed;
  k.gu_scales = (const uint16_t*)h.gu_scales;
  k.d_packed = h.d_packed;
  k.d_scales = (const uint16_t*)h.d_scales;
  k.idx = h.idx;
  k.w = h.w;
  k.logits = h.logits;
  k.expert_scale = h.expert_scale;
  k.out_idx = h.out_idx;
  k.out_w = (uint16_t*)h.out_w;
  k.out = (uint16_t*)h.out;
  k.epochs = (unsigned long long*)state;
  k.act = (char*)state + moe_state::act_offset();
  k.part = (char*)state + moe_state::part_offset();
  k.status = status;
  k.host_flag = device_error_flag(!h.no_alloc, h.stream);
  k.timeline = decode_timeline_slot();
  k.gu_bytes = (uint32_t)((h.H / 8) * 2 * h.I * 4);
  k.gus_bytes = (uint32_t)(h.Ggu * 2 * h.I * 2);
  k.dn_bytes = (uint32_t)((h.I / 8) * h.H * 4);
  k.dsc_bytes = (uint32_t)(h.Gd * h.H * 2);
  k.dn_total = (uint32_t)((size_t)h.E * k.dn_bytes);
  k.dsc_total = (uint32_t)((size_t)h.E * k.dsc_bytes);
  k.idx_is64 = h.idx_is64;
  k.w_dtype = h.w_dtype;
  k.logits_dtype = h.logits_dtype;
  k.H = h.H;
  k.I = h.I;
  k.E = h.E;
  k.top_k = h.top_k;
  k.Ggu = h.Ggu;
  k.Gd = h.Gd;
  k.gsh = log2_exact(h.gs / 32);
  k.Tk = h.I / 32;
  k.units = h.H / 32;
  k.overwrite = h.overwrite;
  k.spin_limit = h.spin_limit > 0 ? h.spin_limit : kDefaultSpin;
  void* args[] = {(void*)&k};
  const hipError_t e =
      hipLaunchKernel(kernel_for(variant_for(k.Tk, k.gsh) + (h.x_dtype == GI_DTYPE_FP16 ? kNumVariants : 0)),
                      dim3(grid_for()), dim3(kT), args, 0, h.stream);
  if (e != hipSuccess) return hip_fail(e, "fused MoE one-token decode launch");
  return GI_OK;
}

}  // namespace gi
