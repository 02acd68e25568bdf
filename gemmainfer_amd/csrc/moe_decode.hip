// Token-Union W4A16 fused MoE for decode and speculative verify on gfx950:
// at most 8 tokens (64 slots) per launch, one launch per layer, no grid-wide
// barrier, no partial sums in memory.
//
// Reference behaviour restated (paths relative to the GemmaInfer repo):
//   routing        gemmainfer/models/gemma.py:77-80
//   dedup          csrc/marlin.cu:285-335 (gate_up) / :453-505 (down)
//   gate_up + GELU csrc/marlin.cu:337-426
//   down + combine csrc/marlin.cu:507-586
//
// A launch has G workgroups of 512 threads, one per CU, all resident.  Every
// workgroup routes the tokens (layer mode) or reads the routing, and builds
// the Token-Union tables in LDS: the unique experts in ascending id order
// (a bitmap of the selected ids and prefix popcounts), each expert's token
// mask, and the activation rows in expert order (expert u's tokens, in token
// order, occupy rows epos[u] .. epos[u+1]).  The number U of unique experts
// then picks the split of the grid into two roles from a table the host
// computed for every U (the split that balances the weight bytes per CU):
//
//   gate/up  workgroups [0, n_gu).  Item (u, c) is unique expert u times the
//            32 intermediate columns [32c, 32c+32).  The item's gate and up
//            words (64 columns over the whole hidden size) are issued at once
//            as fixed-count 16-byte loads, two items ahead, and multiplied on
//            the matrix cores against every token's x, which sits in LDS
//            (one more product against a constant operand gives the offset
//            term of the int4 decoding).  The waves' sums are reduced in LDS,
//            then gelu_tanh(gate)*up is rounded to bf16 (where the reference
//            stores its activation, marlin.cu:421-423) and written to the
//            exchange buffer at the rows of the tokens routed to u.
//   down     workgroups [n_gu, n_gu + n_dn).  One or two units of 32 output
//            columns.  Each wave owns a contiguous range of the (expert,
//            32-k block) pairs, issues their down words at once and keeps
//            them in registers, then all 512 threads poll the exchange
//            buffer and copy its rows into LDS.  The products run on the
//            matrix cores (rows = tokens), are scaled per group and routing
//            weight into per-token fp32 sums, reduced over the waves in a
//            fixed order, and out is written (or added to) once, in bf16.
//
// Deterministic: every sum has a fixed order, whatever the timing.  Slots of
// one token with the same expert (possible only with caller-given ids) are
// one row whose weight is the sum of theirs, in slot order.
//
// Exchange: activations are stored bit-inverted, 16 bytes at a time, into one
// of two buffers chosen by the parity of the launch epoch.  A stored 16-bit
// value is never zero (the one bf16 pattern that would invert to zero, a NaN
// with every bit set, is stored as the canonical NaN), so an all-zero value
// means "not written yet": the reader polls the data itself, one round trip,
// no flag to order against it, and a chunk with any zero half-word is simply
// read again.  Each launch's down workgroups clear the other parity's buffer
// for the next launch (the workspace starts zero-filled).
//
// Launch epochs (moe_state.h): the workspace holds kEpochSlots 64-bit epoch
// words, all equal.  Workgroup b reads word b at launch start, adds one to
// its count, and stores the result to every word j with j % G == b, so all
// words advance by one per launch whatever the grid size (the one-token
// kernel of moe_decode1.hip shares the words and the exchange buffers).  No
// contended atomics are used anywhere:
// on this part a returning atomic on one address costs microseconds when 256
// workgroups issue it.
//
// fp16 activations (template parameter F16; x, scales and out in fp16, the
// routing caller-given): the same kernel with fp16 products.  The int4 codes
// are unpacked exactly to fp16 q - 8 (the bytes of the bf16 16 + q operands
// under a 0x58 high byte are the half 144 + q; a packed fp16 add of -152), so
// the offset products and the offset sums drop out, and the activation, the
// routing weights and out are rounded to fp16 where the bf16 kernel rounds to
// bf16.  Everything else (tables, exchange, partial sums) is shared: the
// exchange and the LDS hold 16-bit values of either type.
//
// Code shape: the hot loops are straight-line with register indices fixed at
// compile time, per-expert values are read from registers with readlane (no
// LDS round trip before a weight load), no integer division in a loop (group
// sizes are powers of two), and one buffer resource per tensor with a scalar
// per-expert offset.

#include <mutex>

#include "../../include/gemmainfer_amd.h"
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

constexpr int kThreads = 512;
constexpr int kWaves = kThreads / kWave;
constexpr int kRows = 8;              // tokens per launch (matrix-core rows used)
constexpr int kSlots = 64;            // slots per launch
constexpr int kCols = 32;             // intermediate columns per item == down k block
constexpr int kUnitCols = 32;         // output columns of a down unit
constexpr int kDefaultSpin = 1 << 20;
constexpr int kCpolNt = 2;            // non-temporal: weights are read once
constexpr int kMaxItems = 9;          // gate/up items per workgroup and launch
constexpr int kDownKpw = 3;           // down k blocks per wave: Tk <= 24 (I <= 768)
constexpr int kDownPreMfma = 4;       // matrix-core path: blocks unpacked before the activations arrive
constexpr int kMaxI = kCols * kDownKpw * kWaves;  // 768
static_assert(kActParity == (size_t)kSlots * kMaxI * 2, "activation exchange buffer size");
constexpr int kScaleLoads = 4;        // 16-byte down-scale chunks per thread (2048 per workgroup)
constexpr int kMaxStage = 12;         // exchange chunks per thread: 64 rows of I/8 <= 96 chunks
constexpr uint32_t kOob = 0xFFFFFFF0u;  // buffer offset past any resource: the load returns zeros


// A value every lane of the wave holds (read from LDS, so the compiler cannot
// tell): made scalar, so that buffer offsets built from it need no per-lane
// loop and loop control stays on the scalar unit.
__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

__host__ __device__ constexpr size_t align16(size_t v) { return (v + 15) & ~(size_t)15; }

// Orders LDS accesses of this wave before the next instruction (no vmcnt wait).
__device__ __forceinline__ void lds_fence() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// Phase stamps of the timeline build (moe_timeline.h).  Slots: 0 start,
// 1 routing and tables, 2 x in LDS, 3 weight loads issued, 4 gate/up items
// done, 5 activations staged, 6 down products, 7 wave sums, 8 output /
// partial sums, 9 end; 29 kernel id (1), 30 and 31 the workgroup's gate/up
// item and down block counts.

struct DecArgs {
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
  uint16_t* act;               // [2][kSlots][I] (parity stride kActParity bytes): rows in expert
                               // order, inverted bf16 (fp16), matrix-core k order
  float* part;                 // [2][units][kPartSlots][kRows][32] partial sums, inverted bits
  int* status;
  int* host_flag;              // host-visible error flag of the device (may be null)
  unsigned long long* timeline;  // [G][kStamps] per-workgroup stamps (timeline builds only; else null)
  uint32_t gu_bytes, gus_bytes, dn_bytes;  // one expert's packed gate/up, its scales, packed down
  uint32_t gu_total, gus_total, dn_total;  // whole tensors (buffer resource sizes)
  uint32_t dsc_total;                      // down scales tensor
  int idx_is64, w_dtype, logits_dtype;
  int M, H, I, E, top_k, Ggu, Gd, S;
  int gsh;      // group_size = 32 << gsh
  int Tk;       // I / 32: items per expert, k blocks of the down projection
  int units;    // H / 32 column units of the down projection
  int overwrite, spin_limit;
};

struct DecPrologue {
  int slot_e[kSlots];
  float slot_w[kSlots];
  uint32_t bm[32];                 // bitmap of the selected expert ids (E <= 1024)
  uint32_t tm[kSlots];             // token mask of unique expert u
  int uexp[kSlots];                // expert id of unique expert u
  int epos[kSlots + 1];            // expert u's rows are [epos[u], epos[u+1])
  __attribute__((aligned(8))) int8_t rowpos[kSlots][kRows];  // row of (u, token), -1 if none
  __attribute__((aligned(16))) float roww[kSlots][kRows];    // routing weight of (u, token), 0 if none
  int n_unique;
  int bad;  // a bounded wait of this workgroup gave up: its outputs are written as NaN
};

// ---------------------------------------------------------------------------
// prologue: routing, Token-Union tables
// ---------------------------------------------------------------------------
// Inclusive prefix sum over the wave: shifts inside each 16-lane row, then
// the row totals broadcast into the rows above (DPP, no LDS round trip).
__device__ __forceinline__ int wave_scan_incl(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xF, 0xF, false);  // row_shr:1
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xF, 0xF, false);  // row_shr:2
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, false);  // row_shr:4
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xF, 0xF, false);  // row_shr:8
  v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xA, 0xF, false);  // row_bcast:15 into rows 1, 3
  v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xC, 0xF, false);  // row_bcast:31 into rows 2, 3
  return v;
}

// Loads of the routing inputs, issued before anything else: with router
// logits, wave w takes token min(w, M - 1)'s row; otherwise lane s of wave 0
// takes slot s's expert id and weight (zeros past S: the resource ends there).
template <int VPL>
struct DecIn {
  RouteIn<VPL> r;
  uint32_t id_lo, id_hi, wb;
};
template <int VPL>
__device__ __forceinline__ void dec_issue(const DecArgs& a, DecIn<VPL>& in) {
  const int lane = threadIdx.x & (kWave - 1), wave = uniform(threadIdx.x >> 6);
  in.id_lo = in.id_hi = in.wb = 0u;
  if (a.logits) {
    route_issue<VPL>(a, min(wave, a.M - 1), lane, in.r);
  } else if (wave == 0) {
    if (a.idx_is64) {
      const u32x2_t v = __builtin_amdgcn_raw_buffer_load_b64(buffer_rsrc(a.idx, (uint32_t)a.S * 8u), lane * 8u, 0, 0);
      in.id_lo = v.x;
      in.id_hi = v.y;
    } else {
      in.id_lo = __builtin_amdgcn_raw_buffer_load_b32(buffer_rsrc(a.idx, (uint32_t)a.S * 4u), lane * 4u, 0, 0);
    }
    if (a.w_dtype == GI_DTYPE_FP32)
      in.wb = __builtin_amdgcn_raw_buffer_load_b32(buffer_rsrc(a.w, (uint32_t)a.S * 4u), lane * 4u, 0, 0);
    else
      in.wb = __builtin_amdgcn_raw_buffer_load_b16(buffer_rsrc(a.w, (uint32_t)a.S * 2u), lane * 2u, 0, 0);
  }
}

template <int VPL, bool F16>
__device__ __forceinline__ void dec_prologue(const DecArgs& a, DecPrologue& P, const DecIn<VPL>& in) {
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = uniform(tid >> 6);
  const int S = a.S;
  if (tid < 32) P.bm[tid] = 0u;
  if (tid == 0) P.bad = 0;
  if (tid < kSlots) P.tm[tid] = 0u;
  (&P.rowpos[0][0])[tid] = -1;  // kSlots * kRows == kThreads entries
  (&P.roww[0][0])[tid] = 0.f;
  if (a.logits) {
    if (wave < a.M) route_finish<VPL>(a, lane, in.r, P.slot_e + wave * a.top_k, P.slot_w + wave * a.top_k);
  } else if (wave == 0 && lane < S) {
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
  GI_STAMP(15);
  lds_barrier();
  GI_STAMP(16);
  if (wave == 0) {
    int e = lane < S ? P.slot_e[lane] : -1;
    float w = lane < S ? P.slot_w[lane] : 0.f;
    const int t = lane / a.top_k;
    if (a.logits) {
      w = round_to_act<F16>(w);
      if (lane < S) P.slot_w[lane] = w;  // reported by workgroup 0 at the end
    } else {
      // a token's slots with one expert: the first keeps the sum of their
      // weights (in slot order), the others are dropped
      const int t0 = t * a.top_k;
      float ws = 0.f;
      bool first = true;
      for (int k2 = 0; k2 < a.top_k; ++k2) {
        const int j = min(t0 + k2, kWave - 1);
        const int ej = __shfl(e, j, kWave);
        const float wj = __shfl(w, j, kWave);
        if (t0 + k2 < S && e >= 0 && ej == e) {
          ws += wj;
          if (t0 + k2 < lane) first = false;
        }
      }
      w = ws;
      if (!first) e = -1;
    }
    // unique experts in ascending id order
    if (e >= 0) __hip_atomic_fetch_or(&P.bm[e >> 5], 1u << (e & 31), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    lds_fence();
    const uint32_t word = lane < 32 ? P.bm[lane] : 0u;
    const int cnt = __popc(word);
    const int incl = wave_scan_incl(cnt);
    const int U = __builtin_amdgcn_readlane(incl, kWave - 1);
    const int wi = max(e, 0) >> 5;
    const int base = __shfl(incl - cnt, wi, kWave);
    const uint32_t bw = (uint32_t)__shfl((int)word, wi, kWave);
    const int u = e >= 0 ? base + __popc(bw & ((1u << (e & 31)) - 1u)) : -1;
    if (u >= 0) {
      __hip_atomic_fetch_or(&P.tm[u], 1u << t, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      P.uexp[u] = e;
      P.roww[u][t] = w;
    }
    lds_fence();
    // rows in expert order, tokens ascending within an expert
    const uint32_t tmu = lane < U ? P.tm[lane] : 0u;
    const int c2 = __popc(tmu);
    const int inc2 = wave_scan_incl(c2);
    const int total = __builtin_amdgcn_readlane(inc2, kWave - 1);
    const int ep0 = inc2 - c2;
    if (lane < U) {
      P.epos[lane] = ep0;
      uint32_t lo = 0u, hi = 0u;
#pragma unroll
      for (int t2 = 0; t2 < kRows; ++t2) {
        const int r = ((tmu >> t2) & 1u) ? ep0 + __popc(tmu & ((1u << t2) - 1u)) : -1;
        if (t2 < 4) lo |= ((uint32_t)r & 0xffu) << (8 * t2);
        else hi |= ((uint32_t)r & 0xffu) << (8 * (t2 - 4));
      }
      *(uint2*)&P.rowpos[lane][0] = make_uint2(lo, hi);
    }
    if (lane == 0) {
      P.epos[U] = total;
      P.n_unique = U;
    }
    GI_STAMP(17);
  }
  lds_barrier();
}

// Launch epoch (see the header).
__device__ __forceinline__ u32x2_t load_epoch(const DecArgs& a) {
  return __builtin_amdgcn_raw_buffer_load_b64(buffer_rsrc(a.epochs, (uint32_t)kEpochSlots * 8u), blockIdx.x * 8u, 0,
                                              kCpolAgent);
}
// The next epoch word: this kernel clears the whole other parity at its end
// and may write all of its own, so its footprint is both whole buffers.
__device__ __forceinline__ void advance_epoch(const DecArgs& a, unsigned long long ep) {
  const unsigned long long wv = moe_state::epoch_word(ep, moe_state::kActUnitsAll, moe_state::kPartUnitsAll);
  for (int j = blockIdx.x; j < kEpochSlots; j += gridDim.x)
    __hip_atomic_store(a.epochs + j, wv, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------------------
// gate/up role
// ---------------------------------------------------------------------------
template <int KBW>
struct GuShape {
  static constexpr int KPM = 4 * kWaves * KBW;  // packed rows of x staged (>= H/8)
};

// Scale groups a wave's k blocks can span: KBW = 11 k blocks of 32 meet at
// most ceil(10 / 2) + 1 = 6 groups of 64 and 4 groups of 128 or more.  A
// fixed count of loads per item keeps every wait count exact; the loads past
// the wave's own group count read past the resource (zeros, no access).
constexpr int kGuScales = 6;

// One item in flight: this lane's words and the scales of the (at most six)
// groups its wave's k blocks fall in.
template <int KBW>
struct GuBuf {
  uint2 s[kGuScales];
  uint4 w[KBW];
};

// The item's words of this lane (16 bytes = 4 adjacent columns, gate for
// lanes 0-7 of each 16, up for 8-15) at packed rows 4kb + lq of this wave's
// k blocks, and their group scales; scales first, so the first group end
// does not wait for the words.  Past the last item the resource is empty:
// the same loads return zeros without touching memory, and the number of
// loads in flight (with it every wait count) is the same on every path.
// Rows past H/8 read the next expert's words (or zeros past the tensor),
// which meet x = 0.
template <int KBW>
__device__ __forceinline__ void gu_load(const DecArgs& a, int uexp_v, int item, int n_items, GuBuf<KBW>& b) {
  const int lane = threadIdx.x & (kWave - 1), wave = uniform(threadIdx.x >> 6);
  const int lq = lane >> 4, lr = lane & 15;
  const int twoI = 2 * a.I;
  const bool real = item < n_items;
  const int u = real ? item / a.Tk : 0, c = real ? item - u * a.Tk : 0;
  const int e = __builtin_amdgcn_readlane(uexp_v, u);
  const int col = (lr < 8 ? 0 : a.I) + kCols * c + 4 * (lr & 7);
  const int kb0 = wave * KBW;
  const int g0 = kb0 >> a.gsh;
  const int nsc = ((kb0 + KBW - 1) >> a.gsh) - g0 + 1;  // groups this wave's k blocks meet
  const __amdgpu_buffer_rsrc_t rs = buffer_rsrc(a.gu_scales, real ? a.gus_total : 0u);
  const __amdgpu_buffer_rsrc_t rw = buffer_rsrc(a.gu_packed, real ? a.gu_total : 0u);
  const int so_s = real ? e * (int)a.gus_bytes : 0, so_w = real ? e * (int)a.gu_bytes : 0;
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int j = 0; j < kGuScales; ++j) {
    const int g = min(g0 + j, a.Ggu - 1);
    const uint32_t off = j < nsc ? (uint32_t)((g * twoI + col) * 2) : kOob;
    const u32x2_t v = __builtin_amdgcn_raw_buffer_load_b64(rs, off, so_s, 0);
    b.s[j] = make_uint2(v.x, v.y);
  }
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int j = 0; j < KBW; ++j) {
    const uint32_t row = 4 * (kb0 + j) + lq;
    const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(rw, (row * twoI + col) * 4, so_w, kCpolNt);
    b.w[j] = make_uint4(v.x, v.y, v.z, v.w);
  }
  __builtin_amdgcn_sched_barrier(0);
}

struct GuLds {
  uint4* xs;       // [kRows][KPM] x in k order (rows >= M and past the scale groups are zero)
  float4* red;     // [kWaves][M][16] per-wave gate/up sums, 64 task columns
  uint16_t* sact;  // [M][32] one item's activations in k order
};
template <int KBW>
__host__ __device__ constexpr size_t gu_lds_bytes() {
  return (size_t)kRows * GuShape<KBW>::KPM * 16 + (size_t)kWaves * kRows * 16 * 16 + (size_t)kRows * kCols * 2;
}

// The gate/up products of one wave's KBW k blocks: y[i][jj] (token row
// 4lq + jj, task column 4lr + i) = sum over scale groups of scale * (the
// group's products + its -24 * sum of x, from one more product against a
// constant operand).  Generic form: the group size is a run-time value.
template <int KBW, bool F16>
__device__ __forceinline__ void gu_products(const DecArgs& a, const GuBuf<KBW>& b, const uint4* xrow, int kb0,
                                            float (&y)[4][4]) {
  const int kbpg_m1 = (1 << a.gsh) - 1;  // k blocks per scale group - 1
  const uint32_t mq = q4_magic_t<F16>();
  const f32x4_t zf = {0.f, 0.f, 0.f, 0.f};
  const uint4 bc = make_uint4(kQ4BiasPair, kQ4BiasPair, kQ4BiasPair, kQ4BiasPair);
  f32x4_t D[4] = {zf, zf, zf, zf};
  f32x4_t Db = zf;
#pragma unroll
  for (int j = 0; j < KBW; ++j) {
    const int kb = kb0 + j;
    const uint4 A = xrow[4 * kb];
    const uint4 w = opaque(b.w[j]);
    D[0] = mfma_act<F16>(A, q4_operand_t<F16>(w.x, mq), D[0]);
    D[1] = mfma_act<F16>(A, q4_operand_t<F16>(w.y, mq), D[1]);
    D[2] = mfma_act<F16>(A, q4_operand_t<F16>(w.z, mq), D[2]);
    D[3] = mfma_act<F16>(A, q4_operand_t<F16>(w.w, mq), D[3]);
    if constexpr (!F16) Db = mfma_bf16(A, bc, Db);  // -24 * sum of each row's x over the k block
    if (((kb + 1) & kbpg_m1) == 0 || j == KBW - 1) {  // a scale group ends here
      const int gi = min(kb >> a.gsh, a.Ggu - 1) - min(kb0 >> a.gsh, a.Ggu - 1);
      uint2 s2 = opaque(b.s[0]);
#pragma unroll
      for (int q = 1; q < kGuScales; ++q)
        if (gi == q) s2 = opaque(b.s[q]);
      const float sc[4] = {sc_lo<F16>(s2.x), sc_hi<F16>(s2.x), sc_lo<F16>(s2.y), sc_hi<F16>(s2.y)};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) y[i][jj] += sc[i] * (F16 ? D[i][jj] : D[i][jj] + Db[jj]);
        D[i] = zf;
      }
      Db = zf;
    }
  }
}

// The same with the group size 32 << GSH and the phase PH of the wave's first
// k block within its group fixed at compile time: every group start and end
// and the scale register of each group are known to the compiler, and a
// group's first products start from zero.  The scales of groups past the
// scale tensor were loaded as zeros.
template <int KBW, bool F16, int GSH, int PH>
__device__ __forceinline__ void gu_products_ph(const GuBuf<KBW>& b, const uint4* xrow, int kb0, float (&y)[4][4]) {
  constexpr int kPg = 1 << GSH;
  const uint32_t mq = q4_magic_t<F16>();
  const f32x4_t zf = {0.f, 0.f, 0.f, 0.f};
  const uint4 bc = make_uint4(kQ4BiasPair, kQ4BiasPair, kQ4BiasPair, kQ4BiasPair);
  f32x4_t D[4], Db;
#pragma unroll
  for (int j = 0; j < KBW; ++j) {
    const bool gstart = j == 0 || (PH + j) % kPg == 0;
    const uint4 A = xrow[4 * (kb0 + j)];
    const uint4 w = opaque(b.w[j]);
    D[0] = mfma_act<F16>(A, q4_operand_t<F16>(w.x, mq), gstart ? zf : D[0]);
    D[1] = mfma_act<F16>(A, q4_operand_t<F16>(w.y, mq), gstart ? zf : D[1]);
    D[2] = mfma_act<F16>(A, q4_operand_t<F16>(w.z, mq), gstart ? zf : D[2]);
    D[3] = mfma_act<F16>(A, q4_operand_t<F16>(w.w, mq), gstart ? zf : D[3]);
    if constexpr (!F16) Db = mfma_bf16(A, bc, gstart ? zf : Db);
    if ((PH + j + 1) % kPg == 0 || j == KBW - 1) {  // a scale group ends
      const uint2 s2 = opaque(b.s[(PH + j) / kPg]);
      const float sc[4] = {sc_lo<F16>(s2.x), sc_hi<F16>(s2.x), sc_lo<F16>(s2.y), sc_hi<F16>(s2.y)};
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) y[i][jj] += sc[i] * (F16 ? D[i][jj] : D[i][jj] + Db[jj]);
    }
  }
}

// One item: gate/up product, cross-wave reduction, activation, exchange.
// PHASED: the group sizes 64 and 128 take the phase-specialized products.
template <int KBW, bool F16, bool PHASED = false>
__device__ __forceinline__ void gu_item(const DecArgs& a, const DecPrologue& P, int item, const GuBuf<KBW>& b,
                                        const GuLds& L, uint16_t* act) {
  constexpr int KPM = GuShape<KBW>::KPM;
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = uniform(tid >> 6);
  const int lq = lane >> 4, lr = lane & 15;
  const int u = item / a.Tk, c = item - u * a.Tk;
  const int kb0 = wave * KBW;
  float y[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i) y[i][0] = y[i][1] = y[i][2] = y[i][3] = 0.f;
  // rows 8-15 of the product repeat rows 0-7 (never used); x rows >= M are zero
  const uint4* xrow = L.xs + (lr & 7) * KPM + lq;
#ifdef GI_TIMELINE
  {  // arrival of this item's first and last k block's words (wave 0's view)
    const int k = item == (int)blockIdx.x ? 0 : 2;
    asm volatile("" ::"v"(b.w[0].x));
    GI_STAMP(10 + k);
    asm volatile("" ::"v"(b.w[KBW - 1].x));
    GI_STAMP(11 + k);
  }
#endif
  if constexpr (PHASED) {
    if (a.gsh == 2) {
      const int ph = kb0 & 3;
      if (ph == 0) gu_products_ph<KBW, F16, 2, 0>(b, xrow, kb0, y);
      else if (ph == 1) gu_products_ph<KBW, F16, 2, 1>(b, xrow, kb0, y);
      else if (ph == 2) gu_products_ph<KBW, F16, 2, 2>(b, xrow, kb0, y);
      else gu_products_ph<KBW, F16, 2, 3>(b, xrow, kb0, y);
    } else if (a.gsh == 1) {
      if ((kb0 & 1) == 0) gu_products_ph<KBW, F16, 1, 0>(b, xrow, kb0, y);
      else gu_products_ph<KBW, F16, 1, 1>(b, xrow, kb0, y);
    } else {
      gu_products<KBW, F16>(a, b, xrow, kb0, y);
    }
  } else {
    gu_products<KBW, F16>(a, b, xrow, kb0, y);
  }
  // per-wave sums of token rows 4lq+jj, task columns 4lr..4lr+3
#pragma unroll
  for (int jj = 0; jj < 4; ++jj) {
    const int row = 4 * lq + jj;
    if (row < a.M) L.red[(wave * a.M + row) * 16 + lr] = make_float4(y[0][jj], y[1][jj], y[2][jj], y[3][jj]);
  }
  lds_barrier();
  const int Iv = min(a.I, a.Gd << (a.gsh + 5));  // activations past the last down group are dropped
  if (tid < a.M * kCols) {
    const int t = tid >> 5, ci = tid & 31;
    float g = 0.f, up = 0.f;
#pragma unroll
    for (int w2 = 0; w2 < kWaves; ++w2) {
      const float* r = (const float*)(L.red + (w2 * a.M + t) * 16);
      g += r[ci];
      up += r[32 + ci];
    }
    const float av = (kCols * c + ci < Iv) ? round_to_act<F16>(gelu_tanh(g) * up) : 0.f;
    const uint16_t bits = act_signal_bits<F16>(av);  // canonical NaN: no stored zero (see header)
    L.sact[t * kCols + (ci & ~7) + mfma_k_pos(ci & 7)] = bits;
  }
  lds_barrier();
  // publish: 16 bytes per (token, 8 columns), inverted; the data is the signal
  if (tid < a.M * 4) {
    const int t = tid >> 2, q = tid & 3;
    const int row = P.rowpos[u][t];
    if (row >= 0) {
      const uint4 v = ((const uint4*)L.sact)[t * 4 + q];
      u32x4_t vv;
      vv.x = ~v.x;
      vv.y = ~v.y;
      vv.z = ~v.z;
      vv.w = ~v.w;
      __builtin_amdgcn_raw_buffer_store_b128(vv, buffer_rsrc(act, kActParity),
                                             (uint32_t)((row * a.I + kCols * c + 8 * q) * 2), 0, kCpolAgent);
    }
  }
}

// x rows of every token, loaded by the kernel before the routing (they do not
// depend on it) so that their latency overlaps the router logits'; rows >= M
// fall outside the resource and read as zero.
template <int KBW>
struct XRegs {
  static constexpr int XPT = (kRows * GuShape<KBW>::KPM + kThreads - 1) / kThreads;
  uint4 v[XPT];
};
template <int KBW>
__device__ __forceinline__ void load_x(const DecArgs& a, XRegs<KBW>& x) {
  constexpr int KPM = GuShape<KBW>::KPM;
  const __amdgpu_buffer_rsrc_t rx = buffer_rsrc(a.x, (uint32_t)a.M * a.H * 2);
#pragma unroll
  for (int i = 0; i < XRegs<KBW>::XPT; ++i) {
    const int id = threadIdx.x + i * kThreads, n = id / KPM, r = id - n * KPM;
    const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(rx, (uint32_t)((n * a.H + 8 * r) * 2), 0, 0);
    x.v[i] = make_uint4(v.x, v.y, v.z, v.w);
  }
}

// Items it0 + K*stride, ... of this workgroup: item K from buffer `cur`, which
// is then reloaded with item K+2 while item K+1 runs from `nxt`.  Template
// recursion instead of a loop: a register array carried around a loop is
// copied at the loop header, which waits for every load in flight.
template <int KBW, bool F16, int K>
__device__ __forceinline__ void gu_items(const DecArgs& a, const DecPrologue& P, const GuLds& L, int uexp_v,
                                         int it0, int stride, int n_items, GuBuf<KBW>& cur, GuBuf<KBW>& nxt,
                                         uint16_t* act) {
  if constexpr (K < kMaxItems) {
    const int item = it0 + K * stride;
    if (item >= n_items) return;
    gu_item<KBW, F16>(a, P, item, cur, L, act);
    gu_load<KBW>(a, uexp_v, item + 2 * stride, n_items, cur);
    gu_items<KBW, F16, K + 1>(a, P, L, uexp_v, it0, stride, n_items, nxt, cur, act);
  }
}

// x of every token into LDS in the matrix-core k order (rows >= M and
// packed rows past the gate/up scale groups are zero: the reference drops
// them).
template <int KBW>
__device__ __forceinline__ void stage_x(const DecArgs& a, const GuLds& L, const XRegs<KBW>& xr) {
  constexpr int KPM = GuShape<KBW>::KPM;
  constexpr int XPT = XRegs<KBW>::XPT;
  const int tid = threadIdx.x;
  const int Kv = min(a.H >> 3, a.Ggu << (a.gsh + 2));
#pragma unroll
  for (int i = 0; i < XPT; ++i) {
    const int id = tid + i * kThreads;
    if (id < kRows * KPM) {
      const int r = id % KPM;
      const uint4 v = mfma_k_order(xr.v[i]);
      L.xs[id] = r < Kv ? v : make_uint4(0u, 0u, 0u, 0u);
    }
  }
  lds_barrier();
  GI_STAMP(2);
}

// ---------------------------------------------------------------------------
// down projection: blocks (unit d, unique expert u), b = d * U + u
// ---------------------------------------------------------------------------
constexpr int kMaxUnits = 88;          // H <= 2816
constexpr int kPartSlots = 8;          // workgroups sharing one unit
static_assert(kPartParity == (size_t)kMaxUnits * kPartSlots * kRows * kUnitCols * 4, "partial buffer size");

// Workgroup w owns blocks [blk_lo(w), blk_lo(w + 1)); the workgroup holding
// block b is the largest w with blk_lo(w) <= b.
// (products stay below 2^31: w, G <= 1024, NB <= 88 * 64)
__host__ __device__ inline int blk_lo(int w, int NB, int G) { return w * NB / G; }
__host__ __device__ inline int blk_owner(int b, int NB, int G) { return ((b + 1) * G - 1) / NB; }

struct DnLds {
  uint4* sact;    // [S + 1][I/8] activation chunks (plain bf16 or fp16, k order); row S is zero
  float* abias;   // [S + 1][I/8] -24 * sum of each chunk's 8 values
  uint32_t* dsc;  // [block of the workgroup][Gd][16] scale pairs (bf16 or fp16) of each lane's two columns
  float* red;     // [2][kWaves][kRows][32] per-wave output sums (aliases sact once it is consumed)
  float* pbuf;    // [kPartSlots][kRows][32] partial sums of a unit's other workgroups (after red)
};

// LDS layout of the down phase.  The down scales sit past both the gate/up
// phase's LDS (gu bytes) and the down phase's data: they are staged before
// the weight loads go out.
struct DnLayout {
  size_t abias, dsc, total;
};
// nbmax: the most down blocks one workgroup owns (blk_lo spacing, rounded up).
__host__ __device__ inline int dn_max_blocks(int units, int U, int G) { return (units * U + G - 1) / G; }
__host__ __device__ inline DnLayout dn_layout(int S, int I, int Gd, size_t gu, int nbmax) {
  const size_t rows = (size_t)S + 1;
  size_t sact = align16(rows * I * 2);
  const size_t red = (size_t)2 * kWaves * kRows * 32 * 4 + (size_t)kPartSlots * kRows * 32 * 4;
  if (sact < red) sact = red;
  DnLayout l;
  l.abias = sact;
  l.dsc = l.abias + align16(rows * (I / 8) * 4);
  if (l.dsc < gu) l.dsc = align16(gu);
  l.total = l.dsc + align16((size_t)nbmax * Gd * 64);
  return l;
}

// Every 16-bit half non-zero.
__device__ __forceinline__ bool chunk_ready(const uint4 v) {
  const uint32_t a0 = min(v.x & 0xffffu, v.x >> 16), a1 = min(v.y & 0xffffu, v.y >> 16);
  const uint32_t a2 = min(v.z & 0xffffu, v.z >> 16), a3 = min(v.w & 0xffffu, v.w >> 16);
  return min(min(a0, a1), min(a2, a3)) != 0u;
}

// sum of the 8 values of a staged chunk (in matrix-core k order) times 16+q,
// for one unpacked word: A.x holds (x0, x4), A.y (x2, x6), A.z (x1, x5), A.w
// (x3, x7), the order of unpack_q4's pairs.
template <bool F16>
__device__ __forceinline__ float dot_chunk(const uint4 A, const Q4Pairs& q, float c) {
  c = fdot2_act<F16>(A.x, q.p0, c);
  c = fdot2_act<F16>(A.y, q.p1, c);
  c = fdot2_act<F16>(A.z, q.p2, c);
  return fdot2_act<F16>(A.w, q.p3, c);
}

// The workgroup's down blocks and the wave's k blocks: wave w takes blocks
// [kb_lo(w), kb_lo(w + 1)) of the 32-k blocks, kb_lo(w) = w * Tk / 8 (at most
// KPW), of every block of the workgroup.
struct DnPlan {
  int blo, nb;  // first block of the batch, blocks held in registers (<= BPW)
  int d_a;      // unit of the batch's first block
  int n0;       // blocks of unit d_a
  int e_off;    // blocks of the workgroup before the batch (scales are indexed from the workgroup's first)
  int kbw0, nkb;
};

// Down words of the workgroup's blocks: lane (lq, lr) loads the 8 bytes of
// columns 32d + 2lr, 32d + 2lr + 1 at packed row 4kb + lq for the wave's k
// blocks.  A fixed number of loads (blocks past nb or k blocks past nkb read
// an offset past the resource: zeros, no memory access), so that the wait
// counts of the gate/up loads issued before them stay exact.
template <int BPW>
__device__ __forceinline__ void dn_load(const DecArgs& a, int uexp_v, int U, const DnPlan& dp,
                                        uint2 (&dw)[BPW][kDownKpw]) {
  const int lane = threadIdx.x & (kWave - 1), lq = lane >> 4, lr = lane & 15;
  const __amdgpu_buffer_rsrc_t rs = buffer_rsrc(a.d_packed, a.dn_total);
  const uint32_t vbase = ((uint32_t)(4 * dp.kbw0 + lq) * a.H) * 4 + (uint32_t)(2 * lr) * 4;
  const uint32_t vstep = (uint32_t)a.H * 16;  // 4 packed rows
  int d = dp.d_a, u = dp.blo - dp.d_a * U;
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int e = 0; e < BPW; ++e) {
    const bool real = e < dp.nb;
    const int ex = __builtin_amdgcn_readlane(uexp_v, min(u, kSlots - 1));
    const int so = real ? ex * (int)a.dn_bytes : 0;
#pragma unroll
    for (int j = 0; j < kDownKpw; ++j) {
      const uint32_t off = real && j < dp.nkb ? vbase + j * vstep + (uint32_t)(kUnitCols * d) * 4 : kOob;
      const u32x2_t v = __builtin_amdgcn_raw_buffer_load_b64(rs, off, so, kCpolNt);
      dw[e][j] = make_uint2(v.x, v.y);
    }
    if (++u == U) {
      u = 0;
      ++d;
    }
  }
  __builtin_amdgcn_sched_barrier(0);
}

// Per-block inputs: the chunk index of each token's activation at the wave's
// first k block (the zero row for tokens not routed to the expert), the
// routing weights, and the scale pairs of the (at most two) groups the
// wave's k blocks fall in.
template <int NT>
struct DnBlock {
  uint32_t ci[NT];
  float wt[NT];
  uint32_t s1, s2;
};
template <int NT, bool MFMA>
__device__ __forceinline__ DnBlock<NT> dn_block(const DecArgs& a, const DecPrologue& P, const DnLds& L,
                                                int epos_v, int tm_v, int u, int e, bool valid, int kbw0, int g1,
                                                int g2) {
  const int lane = threadIdx.x & (kWave - 1), lq = lane >> 4, lr = lane & 15;
  const int cps = a.I >> 3;
  const int uc = min(u, kSlots - 1);
  const int ep = __builtin_amdgcn_readlane(epos_v, uc);
  const uint32_t tmk = valid ? (uint32_t)__builtin_amdgcn_readlane(tm_v, uc) : 0u;
  DnBlock<NT> x;
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    // matrix cores: A row lr is token lr (rows >= M are zero); VALU: token t
    const int tok = MFMA ? (lr & 7) : t;
    const bool ok = (!MFMA || lr < a.M) && ((tmk >> tok) & 1u);
    const int row = ok ? ep + __popc(tmk & ((1u << tok) - 1u)) : a.S;
    x.ci[t] = (uint32_t)(row * cps + 4 * kbw0 + lq);
    x.wt[t] = valid ? P.roww[uc][t] : 0.f;
  }
  x.s1 = L.dsc[(e * a.Gd + g1) * 16 + lr];
  x.s2 = L.dsc[(e * a.Gd + g2) * 16 + lr];  // e counts from the workgroup's first block
  return x;
}

// The VALU path's per-block inputs in the form the products use (scales as
// floats), built for a whole batch before the activations arrive.
template <int NT>
struct DnBlockF {
  uint32_t ci[NT];
  float wt[NT];
  float s[4];  // first group (columns 2lr, 2lr+1), second group
};
template <int BPW, int NT, bool F16>
__device__ __forceinline__ void dn_blocks_valu(const DecArgs& a, const DecPrologue& P, const DnLds& L, int epos_v,
                                               int tm_v, int U, const DnPlan& dp, DnBlockF<NT> (&xb)[BPW]) {
  const int g1 = min(dp.kbw0 >> a.gsh, a.Gd - 1), g2 = min((dp.kbw0 + kDownKpw - 1) >> a.gsh, a.Gd - 1);
  const int u_base = dp.blo - dp.d_a * U;
#pragma unroll
  for (int e = 0; e < BPW; ++e) {
    int u = u_base + e;
    if (u >= U) u -= U;
    const DnBlock<NT> x = dn_block<NT, false>(a, P, L, epos_v, tm_v, u, dp.e_off + e, e < dp.nb, dp.kbw0, g1, g2);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      xb[e].ci[t] = x.ci[t];
      xb[e].wt[t] = x.wt[t];
    }
    xb[e].s[0] = sc_lo<F16>(x.s1);
    xb[e].s[1] = sc_hi<F16>(x.s1);
    xb[e].s[2] = sc_lo<F16>(x.s2);
    xb[e].s[3] = sc_hi<F16>(x.s2);
  }
}

// Chunk j of a wave's k blocks (the zero row past the wave's count unless
// every wave has KPW blocks).
template <bool FULL>
__device__ __forceinline__ uint32_t dn_chunk(uint32_t ci, int j, int nkb, uint32_t zc) {
  if constexpr (FULL) return ci + 4 * j;
  else return j < nkb ? ci + 4 * j : zc;
}


// A down word (columns 2lr, 2lr+1) as the products take it: packed (unpacked
// where it is used) or already unpacked into bf16 pairs 16 + q.
struct DnQ {
  Q4Pairs q[2];
};
template <bool F16>
__device__ __forceinline__ void dn_unpack(const uint2 w, uint32_t mq, Q4Pairs (&q)[2]) {
  q[0] = unpack_q4_t<F16>(w.x, mq);
  q[1] = unpack_q4_t<F16>(w.y, mq);
}
template <bool F16>
__device__ __forceinline__ void dn_unpack(const DnQ& w, uint32_t, Q4Pairs (&q)[2]) {
  q[0] = w.q[0];
  q[1] = w.q[1];
}
// The words of the first NPRE blocks already unpacked, the others packed.
template <int BPW, int NPRE>
struct DnMix {
  const uint2 (&raw)[BPW][kDownKpw];
  const DnQ (&pre)[NPRE][kDownKpw];
};
// word (block e, k block j) of either source; e is a constant once the block
// loops are unrolled, so the choice costs nothing
template <bool F16, int B>
__device__ __forceinline__ void dn_word(const uint2 (&dw)[B][kDownKpw], int e, int j, uint32_t mq, Q4Pairs (&q)[2]) {
  dn_unpack<F16>(dw[e][j], mq, q);
}
template <bool F16, int B>
__device__ __forceinline__ void dn_word(const DnQ (&dw)[B][kDownKpw], int e, int j, uint32_t mq, Q4Pairs (&q)[2]) {
  dn_unpack<F16>(dw[e][j], mq, q);
}
template <bool F16, int B, int NPRE>
__device__ __forceinline__ void dn_word(const DnMix<B, NPRE>& dw, int e, int j, uint32_t mq, Q4Pairs (&q)[2]) {
  if (e < NPRE) dn_unpack<F16>(dw.pre[e < NPRE ? e : 0][j], mq, q);
  else dn_unpack<F16>(dw.raw[e][j], mq, q);
}

// One or two tokens: dot products on the VALU, for blocks [e0, e1) of the
// workgroup (all of one unit).  Lane (lq, lr) takes columns 2lr, 2lr+1 at
// packed row 4kb + lq, i.e. one 8-value chunk of each token's activation
// row; the chunk's -24 offset sum comes precomputed from LDS.  Each k block
// and token has its own dot chain; the first SPLIT of a wave's k blocks
// belong to one scale group, the rest to the next.  The four lq lanes are
// added at the end.
template <int BPW, int NT, int SPLIT, bool FULL, bool F16, class W>
__device__ __forceinline__ void dn_valu(const DecArgs& a, const DnLds& L, const DnPlan& dp, int e_lo, int e_hi,
                                        const W& dw, const DnBlockF<NT> (&xb)[BPW], float (&acc)[NT][2]) {
  constexpr int KPW = kDownKpw;
  const int cps = a.I >> 3;
  const uint32_t mq = q4_magic_t<F16>();
  const uint32_t zc = (uint32_t)(a.S * cps);  // the zero row
#pragma unroll
  for (int e = 0; e < BPW; ++e) {
    if (e >= e_lo && e < e_hi) {
      const DnBlockF<NT>& x = xb[e];
      float d[KPW][NT][2];
#pragma unroll
      for (int j = 0; j < KPW; ++j) {
        Q4Pairs q[2];
        dn_word<F16>(dw, e, j, mq, q);
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          const uint32_t ci = dn_chunk<FULL>(x.ci[t], j, dp.nkb, zc);
          const uint4 A = L.sact[ci];
          const float b = F16 ? 0.f : L.abias[ci];  // fp16: q - 8 operands, no offset
#pragma unroll
          for (int h = 0; h < 2; ++h) d[j][t][h] = dot_chunk<F16>(A, q[h], b);
        }
      }
#pragma unroll
      for (int t = 0; t < NT; ++t) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          // segment sums: k block 0 is always in the first group, block
          // KPW-1 in the second unless SPLIT == KPW
          float v1 = d[0][t][h], v2 = d[KPW - 1][t][h];
#pragma unroll
          for (int j = 1; j < KPW - 1; ++j) (j < SPLIT ? v1 : v2) += d[j][t][h];
          if constexpr (SPLIT == KPW) v1 += v2;
          float v = x.s[h] * v1;
          if constexpr (SPLIT < KPW) v += x.s[2 + h] * v2;
          acc[t][h] += x.wt[t] * v;
        }
      }
    }
  }
}

// Three tokens or more: matrix-core products, A rows = tokens (row lr is
// token lr's chunk when lr < M and the token is routed to the expert, else
// the zero row), B = the unpacked words (columns 2lr + h), one more product
// with a constant -24 operand for the int4 offset, accumulated per scale
// group (the first SPLIT of the wave's k blocks, then the rest) and scaled
// by the group scale and routing weight into acc[h] (rows 4lq + jj).
template <int BPW, int SPLIT, bool FULL, bool F16, class W>
__device__ __forceinline__ void dn_mfma(const DecArgs& a, const DecPrologue& P, const DnLds& L, int epos_v,
                                        int tm_v, int U, const DnPlan& dp, int e_lo, int e_hi,
                                        const W& dw, f32x4_t (&acc)[2]) {
  constexpr int KPW = kDownKpw;
  const int lane = threadIdx.x & (kWave - 1), lq = lane >> 4;
  const int cps = a.I >> 3;
  const uint32_t mq = q4_magic_t<F16>();
  const f32x4_t zf = {0.f, 0.f, 0.f, 0.f};
  const uint4 bc = make_uint4(kQ4BiasPair, kQ4BiasPair, kQ4BiasPair, kQ4BiasPair);
  const int g1 = min(dp.kbw0 >> a.gsh, a.Gd - 1), g2 = min((dp.kbw0 + KPW - 1) >> a.gsh, a.Gd - 1);
  const uint32_t zc = (uint32_t)(a.S * cps);
  const int u_base = dp.blo - dp.d_a * U;
#pragma unroll
  for (int e = 0; e < BPW; ++e) {
    if (e >= e_lo && e < e_hi) {
      int u = u_base + e;
      if (u >= U) u -= U;
      const DnBlock<1> x = dn_block<1, true>(a, P, L, epos_v, tm_v, u, dp.e_off + e, true, dp.kbw0, g1, g2);
      const float4 wr = *(const float4*)&P.roww[u][4 * (lq & 1)];
      const float wv[4] = {wr.x, wr.y, wr.z, wr.w};
      f32x4_t D[2][2], Db[2];
#pragma unroll
      for (int sgi = 0; sgi < 2; ++sgi) {
        Db[sgi] = zf;
        D[sgi][0] = zf;
        D[sgi][1] = zf;
      }
#pragma unroll
      for (int j = 0; j < KPW; ++j) {
        const int sgi = j < SPLIT ? 0 : 1;
        const uint4 A = L.sact[dn_chunk<FULL>(x.ci[0], j, dp.nkb, zc)];
        Q4Pairs q[2];
        dn_word<F16>(dw, e, j, mq, q);
        D[sgi][0] = mfma_act<F16>(A, make_uint4(q[0].p0, q[0].p1, q[0].p2, q[0].p3), D[sgi][0]);
        D[sgi][1] = mfma_act<F16>(A, make_uint4(q[1].p0, q[1].p1, q[1].p2, q[1].p3), D[sgi][1]);
        if constexpr (!F16) Db[sgi] = mfma_bf16(A, bc, Db[sgi]);
      }
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const float sa = h ? sc_hi<F16>(x.s1) : sc_lo<F16>(x.s1);
        const float sb = h ? sc_hi<F16>(x.s2) : sc_lo<F16>(x.s2);
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          float v = sa * (F16 ? D[0][h][jj] : D[0][h][jj] + Db[0][jj]);
          if constexpr (SPLIT < KPW) v += sb * (F16 ? D[1][h][jj] : D[1][h][jj] + Db[1][jj]);
          acc[h][jj] += wv[jj] * v;
        }
      }
    }
  }
}

// Blocks [e_lo, e_hi) with the wave's variant: k blocks in its first scale
// group (1, 2 or all KPW; a group has at least KPW blocks) and whether the
// wave has all KPW k blocks.
template <int BPW, int MODE, bool F16, int SPLIT, class W>
__device__ __forceinline__ void dn_run_split(const DecArgs& a, const DecPrologue& P, const DnLds& L, int epos_v,
                                             int tm_v, int U, const DnPlan& dp, int e_lo, int e_hi, const W& dw,
                                             const DnBlockF<(MODE > 0 ? MODE : 1)> (&xb)[BPW],
                                             float (&accv)[MODE > 0 ? MODE : 1][2], f32x4_t (&accm)[2]) {
  constexpr int NT = MODE > 0 ? MODE : 1;
  if (dp.nkb == kDownKpw) {
    if constexpr (MODE > 0) dn_valu<BPW, NT, SPLIT, true, F16>(a, L, dp, e_lo, e_hi, dw, xb, accv);
    else dn_mfma<BPW, SPLIT, true, F16>(a, P, L, epos_v, tm_v, U, dp, e_lo, e_hi, dw, accm);
  } else {
    if constexpr (MODE > 0) dn_valu<BPW, NT, SPLIT, false, F16>(a, L, dp, e_lo, e_hi, dw, xb, accv);
    else dn_mfma<BPW, SPLIT, false, F16>(a, P, L, epos_v, tm_v, U, dp, e_lo, e_hi, dw, accm);
  }
}
template <int BPW, int MODE, bool F16, class W>
__device__ __forceinline__ void dn_run(const DecArgs& a, const DecPrologue& P, const DnLds& L, int epos_v, int tm_v,
                                       int U, const DnPlan& dp, int e_lo, int e_hi, const W& dw,
                                       const DnBlockF<(MODE > 0 ? MODE : 1)> (&xb)[BPW],
                                       float (&accv)[MODE > 0 ? MODE : 1][2], f32x4_t (&accm)[2]) {
  const int split = min(kDownKpw, (1 << a.gsh) - (dp.kbw0 & ((1 << a.gsh) - 1)));
  if (split == 1) dn_run_split<BPW, MODE, F16, 1>(a, P, L, epos_v, tm_v, U, dp, e_lo, e_hi, dw, xb, accv, accm);
  else if (split == 2) dn_run_split<BPW, MODE, F16, 2>(a, P, L, epos_v, tm_v, U, dp, e_lo, e_hi, dw, xb, accv, accm);
  else dn_run_split<BPW, MODE, F16, kDownKpw>(a, P, L, epos_v, tm_v, U, dp, e_lo, e_hi, dw, xb, accv, accm);
}

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// All 512 threads copy exchange rows into LDS: chunks g = base + tid + 512j
// of the rows [r0, r1) (less the rows [x0, x1), which no block of the
// workgroup reads), written straight into LDS at their own index (a wave's
// 64 lanes fill 1 KB in lane order, no registers held).  A chunk is complete
// when no 16-bit half is zero, and is then inverted in place and its offset
// sum stored.  Each wave repeats its incomplete chunks until none is left
// (bounded: on timeout the status word is flagged and the wave goes on, so
// the launch always ends).
template <int CPT, bool BIAS>
__device__ __forceinline__ void stage_acts(const DecArgs& a, const DnLds& L, const uint16_t* act, int c0, int c1,
                                           int x0, int x1, int* bad) {
  const int tid = threadIdx.x, wave = uniform(tid >> 6);
  const __amdgpu_buffer_rsrc_t rs = buffer_rsrc(act, kActParity);
  uint32_t pending = 0u;
#pragma unroll
  for (int j = 0; j < CPT; ++j) {
    const int g = c0 + tid + j * kThreads;
    if (g < c1 && (g < x0 || g >= x1)) pending |= 1u << j;
  }
  int spins = 0;
  while (true) {
#pragma unroll
    for (int j = 0; j < CPT; ++j) {
      if ((pending >> j) & 1u)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_ptr_t)(L.sact + c0 + j * kThreads + wave * kWave), 16,
                                                 (uint32_t)(c0 + tid + j * kThreads) * 16u, 0, 0, kCpolAgent);
    }
    wait_vmem();
    asm volatile("" ::: "memory");
#pragma unroll
    for (int j = 0; j < CPT; ++j) {
      if ((pending >> j) & 1u) {
        const int g = c0 + tid + j * kThreads;
        const uint4 v = L.sact[g];
        if (chunk_ready(v)) {
          const uint4 x = make_uint4(~v.x, ~v.y, ~v.z, ~v.w);
          L.sact[g] = x;
          if constexpr (BIAS) L.abias[g] = q4_bias(x);
          pending &= ~(1u << j);
        }
      }
    }
    if (__ballot(pending != 0u) == 0ull) break;
    if (++spins >= a.spin_limit) {
      if ((threadIdx.x & (kWave - 1)) == 0) {
        report_timeout(a.status, a.host_flag);
        *bad = 1;
      }
      break;
    }
    __builtin_amdgcn_s_sleep(2);
    asm volatile("" ::: "memory");  // the next poll reads memory again
  }
}

// Down scales of the workgroup's blocks (all batches), straight into LDS: chunk ch =
// (e * Gd + g) * 4 + q holds bf16 columns 8q .. 8q+7 of block e's unit for
// group g, so that lane lr's pair (columns 2lr, 2lr+1) is u32 word
// (e * Gd + g) * 16 + lr.  Complete once the wave has waited for its loads.
__device__ __forceinline__ void dsc_load(const DecArgs& a, uint32_t* dsc, int uexp_v, int U, int blo, int nb) {
  const int tid = threadIdx.x, wave = uniform(tid >> 6);
  const int n = nb * a.Gd * 4;
  const __amdgpu_buffer_rsrc_t rs = buffer_rsrc(a.d_scales, a.dsc_total);
  // quotients from float reciprocals: the operands are below 2^13, so the
  // rounding error of (n + 0.5) * (1/m) is far from the next integer
  const float inv_gd = 1.0f / (float)a.Gd, inv_u = 1.0f / (float)U;
  int ex[kScaleLoads];
  uint32_t off[kScaleLoads];
  // the expert ids of all chunks first (one LDS round trip for all of them)
#pragma unroll
  for (int j = 0; j < kScaleLoads; ++j) {
    const int ch = tid + j * kThreads;
    const int eg = ch >> 2, q = ch & 3;
    const int e = (int)(((float)eg + 0.5f) * inv_gd), g = eg - e * a.Gd;
    const int b = blo + e;
    const int d = (int)(((float)b + 0.5f) * inv_u), u = b - d * U;
    ex[j] = __shfl(uexp_v, min(u, kSlots - 1), kWave);
    off[j] = (uint32_t)((g * a.H + kUnitCols * d + 8 * q) * 2);
  }
#pragma unroll
  for (int j = 0; j < kScaleLoads; ++j) {
    const int ch = tid + j * kThreads;
    const uint32_t o = off[j] + (uint32_t)ex[j] * (uint32_t)(a.Gd * a.H * 2);
    if (ch < n)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_ptr_t)((uint4*)dsc + j * kThreads + wave * kWave), 16,
                                               o, 0, 0, 0);
  }
}

// Share `part` of `parts` of a buffer of `bytes`, cleared.
__device__ __forceinline__ void clear_share(void* buf, size_t bytes, int part, int parts) {
  const int nch = (int)(bytes / 16);
  const int per = (nch + parts - 1) / parts;
  const __amdgpu_buffer_rsrc_t nx = buffer_rsrc(buf, (uint32_t)bytes);
  const u32x4_t z = {0u, 0u, 0u, 0u};
  for (int i = threadIdx.x; i < per; i += kThreads) {
    const int ch = part * per + i;
    if (ch < nch) __builtin_amdgcn_raw_buffer_store_b128(z, nx, (uint32_t)ch * 16u, 0, kCpolAgent);
  }
}

__device__ __forceinline__ uint32_t f32_signal_bits(float v) {
  uint32_t b = __float_as_uint(v);
  if ((b & 0x7fffffffu) > 0x7f800000u) b = 0x7fc00000u;  // canonical NaN: no stored zero
  return ~b;
}

// The down phase of one workgroup: stage the activation rows its blocks
// read, the products, the sums over the waves, then per unit either the
// output (a unit held whole, or the unit's first workgroup once the others'
// partial sums are in) or this workgroup's partial sum for the first one.
template <int BPW, int MODE, int CPT, bool PRE, bool F16>
__device__ __forceinline__ void down_phase(const DecArgs& a, const DecPrologue& P, char* lds, const DnLayout& ly,
                                           int U, int uexp_v, const uint16_t* act, float* part, int blo, int bhi,
                                           DnPlan dp, const uint2 (&dw0)[BPW][kDownKpw]) {
  constexpr int NT = MODE > 0 ? MODE : 1;
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = uniform(tid >> 6);
  const int lq = lane >> 4, lr = lane & 15;
  const int cps = a.I >> 3;
  const int G = gridDim.x, NB = a.units * U;
  DnLds L;
  L.sact = (uint4*)lds;
  L.red = (float*)lds;
  L.pbuf = L.red + 2 * kWaves * kRows * 32;
  L.abias = (float*)(lds + ly.abias);
  L.dsc = (uint32_t*)(lds + ly.dsc);
  const int epos_v = P.epos[lane];
  const int tm_v = (int)P.tm[lane];
  const int nb_all = bhi - blo, d_first = blo / U;
  const int n_units = (bhi - 1) / U > d_first ? 2 : 1;  // at most two: a workgroup has at most U blocks
  // previous output of the writer thread's (token, column) of each unit when
  // accumulating: the 4-byte word holding it, loaded by every thread (no
  // memory access past the resource), so that no wait is placed here
  const bool writer = tid < a.M * kUnitCols;
  const int wt = tid >> 5, wc = tid & 31;
  const __amdgpu_buffer_rsrc_t ro = buffer_rsrc(a.out, a.overwrite ? 0u : (uint32_t)a.M * a.H * 2u);
  uint32_t old[2];
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    const int d = min(d_first + p, a.units - 1);
    const uint32_t off = writer ? (uint32_t)(wt * a.H + kUnitCols * d + (wc & ~1)) * 2u : kOob;
    old[p] = __builtin_amdgcn_raw_buffer_load_b32(ro, off, 0, 0);
  }
  lds_barrier();  // the gate/up phase's LDS is free
  // the zero row (absent tokens and missing k blocks read it)
  if (tid < cps) {
    L.sact[a.S * cps + tid] = make_uint4(0u, 0u, 0u, 0u);
    L.abias[a.S * cps + tid] = 0.f;
  }
  // rows of the experts the blocks read: expert u_a.. of the first unit, and
  // 0..u_b of the second
  const int u_a = blo - d_first * U;
  int c0, c1, x0 = 0, x1 = 0;
  if (n_units == 1) {
    c0 = P.epos[u_a] * cps;
    c1 = P.epos[u_a + nb_all] * cps;
  } else {
    const int u_b = bhi - 1 - (d_first + 1) * U;
    c0 = 0;
    c1 = P.epos[U] * cps;
    if (u_b + 1 < u_a) {
      x0 = P.epos[u_b + 1] * cps;
      x1 = P.epos[u_a] * cps;
    }
  }
  c0 = uniform(c0);
  c1 = uniform(c1);
  x0 = uniform(x0);
  x1 = uniform(x1);
  // the first batch's words unpacked while the activations are on their way,
  // where the registers allow: every block with one token and few blocks,
  // the first kDownPreMfma blocks on the matrix-core path
#ifdef GI_TIMELINE
  asm volatile("" ::"v"(dw0[BPW - 1][kDownKpw - 1].x));
  GI_STAMP(14);  // the first batch's down words landed (wave 0's view)
#endif
  constexpr int NPRE = PRE ? BPW : (MODE == 0 ? (BPW < kDownPreMfma ? BPW : kDownPreMfma) : 0);
  DnQ dq[NPRE > 0 ? NPRE : 1][kDownKpw];
  if constexpr (NPRE > 0) {
    const uint32_t mq = q4_magic_t<F16>();
#pragma unroll
    for (int e = 0; e < NPRE; ++e)
#pragma unroll
      for (int j = 0; j < kDownKpw; ++j) {
        dn_unpack<F16>(dw0[e][j], mq, dq[e][j].q);
        // here, not next to the products: the unpacking overlaps the wait
#pragma unroll
        for (int h = 0; h < 2; ++h)
          asm volatile("" : "+v"(dq[e][j].q[h].p0), "+v"(dq[e][j].q[h].p1), "+v"(dq[e][j].q[h].p2),
                       "+v"(dq[e][j].q[h].p3));
      }
  }
  // batch 0: the words loaded with the gate/up items; on the VALU path its
  // per-block inputs are built before the wait as well
  dp.blo = blo;
  dp.e_off = 0;
  dp.nb = min(nb_all, BPW);
  dp.d_a = d_first;
  dp.n0 = min(dp.nb, (d_first + 1) * U - blo);
  DnBlockF<NT> xb[BPW];
  if constexpr (MODE > 0) dn_blocks_valu<BPW, NT, F16>(a, P, L, epos_v, tm_v, U, dp, xb);
  int* bad = const_cast<int*>(&P.bad);
  stage_acts<CPT, (MODE > 0 && !F16)>(a, L, act, c0, c1, x0, x1, bad);  // waits for every load of the wave
  lds_barrier();
  GI_STAMP(5);

  float accv[2][NT][2];
  f32x4_t accm[2][2];
  const f32x4_t zf = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int p = 0; p < 2; ++p)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      accm[p][h] = zf;
#pragma unroll
      for (int t = 0; t < NT; ++t) accv[p][t][h] = 0.f;
    }
  if constexpr (NPRE == BPW) {
    dn_run<BPW, MODE, F16>(a, P, L, epos_v, tm_v, U, dp, 0, dp.n0, dq, xb, accv[0], accm[0]);
    if (dp.nb > dp.n0) dn_run<BPW, MODE, F16>(a, P, L, epos_v, tm_v, U, dp, dp.n0, dp.nb, dq, xb, accv[1], accm[1]);
  } else if constexpr (NPRE > 0) {
    const DnMix<BPW, NPRE> mix{dw0, dq};
    dn_run<BPW, MODE, F16>(a, P, L, epos_v, tm_v, U, dp, 0, dp.n0, mix, xb, accv[0], accm[0]);
    if (dp.nb > dp.n0) dn_run<BPW, MODE, F16>(a, P, L, epos_v, tm_v, U, dp, dp.n0, dp.nb, mix, xb, accv[1], accm[1]);
  } else {
    dn_run<BPW, MODE, F16>(a, P, L, epos_v, tm_v, U, dp, 0, dp.n0, dw0, xb, accv[0], accm[0]);
    if (dp.nb > dp.n0) dn_run<BPW, MODE, F16>(a, P, L, epos_v, tm_v, U, dp, dp.n0, dp.nb, dw0, xb, accv[1], accm[1]);
  }
  // further batches (more blocks than the registers hold)
  for (int b0 = blo + BPW; b0 < bhi; b0 += BPW) {
    dp.blo = b0;
    dp.e_off = b0 - blo;
    dp.nb = min(bhi - b0, BPW);
    dp.d_a = b0 / U;
    dp.n0 = max(0, min(dp.nb, (d_first + 1) * U - b0));
    uint2 dw[BPW][kDownKpw];
    dn_load<BPW>(a, uexp_v, U, dp, dw);
    if constexpr (MODE > 0) dn_blocks_valu<BPW, NT, F16>(a, P, L, epos_v, tm_v, U, dp, xb);
    if (dp.n0 > 0) dn_run<BPW, MODE, F16>(a, P, L, epos_v, tm_v, U, dp, 0, dp.n0, dw, xb, accv[0], accm[0]);
    if (dp.nb > dp.n0) dn_run<BPW, MODE, F16>(a, P, L, epos_v, tm_v, U, dp, dp.n0, dp.nb, dw, xb, accv[1], accm[1]);
  }
  // sums over the waves, fixed order (the per-wave sums alias the staged rows)
  lds_barrier();
  GI_STAMP(6);
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    float* red = L.red + (size_t)p * kWaves * kRows * 32;
    if constexpr (MODE > 0) {
#pragma unroll
      for (int t = 0; t < NT; ++t) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          float v = accv[p][t][h];
          v += __shfl_xor(v, 16, kWave);
          v += __shfl_xor(v, 32, kWave);
          if (lq == 0 && t < a.M) red[(wave * kRows + t) * 32 + 2 * lr + h] = v;
        }
      }
    } else {
      if (lq < 2) {
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          const int row = 4 * lq + jj;
          if (row < a.M) {
            red[(wave * kRows + row) * 32 + 2 * lr] = accm[p][0][jj];
            red[(wave * kRows + row) * 32 + 2 * lr + 1] = accm[p][1][jj];
          }
        }
      }
    }
  }
  lds_barrier();
  GI_STAMP(7);
  for (int p = 0; p < n_units; ++p) {
    const int d = d_first + p;
    const int wf = blk_owner(d * U, NB, G), wl = blk_owner(d * U + U - 1, NB, G);
    const int ns = wl - wf + 1, slot = (int)blockIdx.x - wf;
    float s = 0.f;
    if (writer) {
      const float* red = L.red + (size_t)p * kWaves * kRows * 32;
#pragma unroll
      for (int w2 = 0; w2 < kWaves; ++w2) s += red[(w2 * kRows + wt) * 32 + wc];
    }
    const __amdgpu_buffer_rsrc_t pr = buffer_rsrc(part, kPartParity);
    if (slot > 0) {
      // a partial sum for the unit's first workgroup: 16 bytes per (token, 4 columns)
      if (writer) L.pbuf[wt * 32 + wc] = P.bad ? __uint_as_float(0x7fc00000u) : s;
      lds_barrier();
      if (tid < a.M * 8) {
        const int t = tid >> 3, q = tid & 7;
        const float4 v = *(const float4*)&L.pbuf[t * 32 + 4 * q];
        u32x4_t vv;
        vv.x = f32_signal_bits(v.x);
        vv.y = f32_signal_bits(v.y);
        vv.z = f32_signal_bits(v.z);
        vv.w = f32_signal_bits(v.w);
        __builtin_amdgcn_raw_buffer_store_b128(
            vv, pr, (uint32_t)((((d * kPartSlots + slot) * kRows + t) * kUnitCols + 4 * q) * 4), 0, kCpolAgent);
      }
      lds_barrier();
      continue;
    }
    if (ns > 1) {
      // the unit's first workgroup: the others' partial sums, polled
      const int nch = (ns - 1) * a.M * 8;
      if (tid < nch) {
        const int sl = 1 + tid / (a.M * 8), r = tid - (sl - 1) * a.M * 8;
        const int t = r >> 3, q = r & 7;
        const uint32_t off = (uint32_t)((((d * kPartSlots + sl) * kRows + t) * kUnitCols + 4 * q) * 4);
        // with fewer blocks than workgroups some workgroups between the
        // unit's first and last hold none and publish nothing: a zero term
        const bool held = blk_lo(wf + sl, NB, G) < blk_lo(wf + sl + 1, NB, G);
        int spins = 0;
        u32x4_t v = {~0u, ~0u, ~0u, ~0u};  // inverted zeros
        while (held) {
          v = __builtin_amdgcn_raw_buffer_load_b128(pr, off, 0, kCpolAgent);
          if (v.x != 0u && v.y != 0u && v.z != 0u && v.w != 0u) break;
          if (++spins >= a.spin_limit) {
            report_timeout(a.status, a.host_flag);
            *bad = 1;
            break;
          }
          __builtin_amdgcn_s_sleep(2);
          asm volatile("" ::: "memory");
        }
        *(float4*)&L.pbuf[((sl - 1) * kRows + t) * 32 + 4 * q] =
            make_float4(__uint_as_float(~v.x), __uint_as_float(~v.y), __uint_as_float(~v.z), __uint_as_float(~v.w));
      }
      lds_barrier();
      if (writer)
        for (int sl = 1; sl < ns; ++sl) s += L.pbuf[((sl - 1) * kRows + wt) * 32 + wc];
      lds_barrier();
    }
    if (writer) {
      if (!a.overwrite) s += act_to_f32<F16>((old[p] >> (16 * (wc & 1))) & 0xffffu);
      if (P.bad) s = __uint_as_float(0x7fc00000u);  // never a wrong finite value
      a.out[(size_t)wt * a.H + kUnitCols * d + wc] = f32_to_act<F16>(s);
    }
  }
  GI_STAMP(8);
}

// The workgroup's gate/up items (it0, it0 + G, ...) and the issue of its down
// words: the items' words go out first, then the down words, so that every
// wait of the gate/up products has an exact count.  The down words are
// needed only after the activation exchange: NI = 1 issues them after its
// item's products, NI = 2 after its first item's products, so that the
// items' words (whose products are on the critical path) are served first.
// NI = 3 is the general path (two items in flight, the next one loaded as
// each finishes), which issues the down words after its items (registers: a
// rare case).
template <int KBW, int NI, int BPW, bool F16>
__device__ __forceinline__ void up_phase(const DecArgs& a, const DecPrologue& P, const GuLds& L, int U,
                                         int uexp_v, uint16_t* act, const DnPlan& dp, int n_items,
                                         uint2 (&dw)[BPW][kDownKpw]) {
  const int it0 = blockIdx.x, G = gridDim.x;
  GuBuf<KBW> b0, b1;
  gu_load<KBW>(a, uexp_v, it0, n_items, b0);
  if constexpr (NI >= 2) gu_load<KBW>(a, uexp_v, it0 + G, n_items, b1);
  GI_STAMP(3);
  if constexpr (NI == 1) {
    gu_item<KBW, F16, true>(a, P, it0, b0, L, act);
    dn_load<BPW>(a, uexp_v, U, dp, dw);
  } else if constexpr (NI == 2) {
    gu_item<KBW, F16, true>(a, P, it0, b0, L, act);
    dn_load<BPW>(a, uexp_v, U, dp, dw);
    gu_item<KBW, F16, true>(a, P, it0 + G, b1, L, act);
  } else {
    gu_items<KBW, F16, 0>(a, P, L, uexp_v, it0, G, n_items, b0, b1, act);
    dn_load<BPW>(a, uexp_v, U, dp, dw);
  }
  GI_STAMP(4);
}

// ---------------------------------------------------------------------------
// kernel
// ---------------------------------------------------------------------------
// The start of every workgroup: the routing inputs go out first, then the
// epoch word and x behind them (neither depends on the routing), then the
// routing and the Token-Union tables.  The epoch is read after the routing:
// a value needed in scalar registers is otherwise read right after its load,
// and the routing would wait for it.
template <int KBW, int VPL, bool F16>
__device__ __forceinline__ u32x2_t dec_start(const DecArgs& a, DecPrologue& P, XRegs<KBW>& xr) {
  DecIn<VPL> in;
  dec_issue<VPL>(a, in);
  u32x2_t ep = load_epoch(a);
  load_x<KBW>(a, xr);
  dec_prologue<VPL, F16>(a, P, in);
  asm volatile("" : "+v"(ep));
  return ep;
}

// The end of every workgroup: the stores that no part of this launch waits
// for, left to the end so that no wait of the launch counts them (a store
// counts in the same in-order counter as the loads): the next launch's epoch,
// this workgroup's share of the next launch's exchange buffers, and the
// routing report of workgroup 0.
__device__ __forceinline__ void dec_end(const DecArgs& a, const DecPrologue& P, unsigned long long ep,
                                        int parity) {
  const int b = blockIdx.x, G = gridDim.x;
  if (threadIdx.x == 0) advance_epoch(a, ep);
  clear_share(a.act + (size_t)(parity ^ 1) * (kActParity / 2), kActParity, b, G);
  clear_share(a.part + (size_t)(parity ^ 1) * (kPartParity / 4), kPartParity, b, G);
  if (b == 0 && a.logits && threadIdx.x < a.S) {
    if (a.out_idx) a.out_idx[threadIdx.x] = P.slot_e[threadIdx.x];
    if (a.out_w) a.out_w[threadIdx.x] = f32_to_bf16(P.slot_w[threadIdx.x]);
  }
}

template <int KBW, int MODE, int BPW, int CPT, bool F16>
__global__ __launch_bounds__(kThreads) void moe_decode_kernel(DecArgs a) {
  __shared__ DecPrologue P;
  extern __shared__ __attribute__((aligned(16))) char dyn_lds[];
#ifdef GI_TIMELINE
  tl_init();
#endif
  GI_STAMP(0);
  XRegs<KBW> xr;
  u32x2_t epr;
  if (a.E <= 2 * kWave) epr = dec_start<KBW, 2, F16>(a, P, xr);
  else if (a.E <= 4 * kWave) epr = dec_start<KBW, 4, F16>(a, P, xr);
  else epr = dec_start<KBW, kRouteMaxExperts / kWave, F16>(a, P, xr);
  const unsigned long long ep = moe_state::epoch_count(((unsigned long long)epr.y << 32) | epr.x) + 1ull;
  const int parity = (int)(ep & 1ull);
  uint16_t* act = a.act + (size_t)parity * (kActParity / 2);
  float* part = a.part + (size_t)parity * (kPartParity / 4);
  const int U = uniform(P.n_unique);
  const int b = blockIdx.x, G = gridDim.x;
  GI_STAMP(1);
  if (U == 0) {
    // no valid slot: a layer call still owns (overwrites) out
    if (a.overwrite)
      for (int i = b * kThreads + threadIdx.x; i < a.M * a.H; i += G * kThreads) a.out[i] = 0;
    dec_end(a, P, ep, parity);
    return;
  }
  const int uexp_v = P.uexp[threadIdx.x & (kWave - 1)];
  const int n_items = U * a.Tk;
  const int NB = a.units * U;
  const int n_my = b < n_items ? (n_items - b + G - 1) / G : 0;
  // down blocks of this workgroup, at most BPW at a time
  const int blo = blk_lo(b, NB, G), bhi = blk_lo(b + 1, NB, G);
  const int wave = uniform(threadIdx.x >> 6);
  GuLds L;
  constexpr int KPM = GuShape<KBW>::KPM;
  L.xs = (uint4*)dyn_lds;
  L.red = (float4*)(dyn_lds + (size_t)kRows * KPM * 16);
  L.sact = (uint16_t*)(L.red + kWaves * kRows * 16);
  GI_STAMP(18);
  // x into LDS first: its registers are free before the word buffers fill
  // (staged after the word loads are issued, it waited as long as the first
  // item's words: M=7 29.7 -> 30.0 us)
  if (n_my > 0) stage_x<KBW>(a, L, xr);
#ifdef GI_TIMELINE
  tl_value(29, 1ull);
  tl_value(30, (unsigned long long)n_my);
  tl_value(31, (unsigned long long)(bhi - blo));
#endif
  // the down scales of every block of the workgroup, ahead of the weights
  // (older than every weight load, they leave the weight waits exact)
  const DnLayout ly = dn_layout(a.S, a.I, a.Gd, gu_lds_bytes<KBW>(), dn_max_blocks(a.units, a.S, G));
  dsc_load(a, (uint32_t*)(dyn_lds + ly.dsc), uexp_v, U, blo, bhi - blo);
  DnPlan dp;
  dp.blo = blo;
  dp.e_off = 0;
  dp.nb = min(bhi - blo, BPW);
  dp.d_a = blo / U;
  dp.n0 = min(dp.nb, (dp.d_a + 1) * U - blo);
  dp.kbw0 = wave * a.Tk / kWaves;
  dp.nkb = (wave + 1) * a.Tk / kWaves - dp.kbw0;
  uint2 dw[BPW][kDownKpw];
  if (n_my == 0) dn_load<BPW>(a, uexp_v, U, dp, dw);
  else if (n_my == 1) up_phase<KBW, 1, BPW, F16>(a, P, L, U, uexp_v, act, dp, n_items, dw);
  else if (n_my == 2) up_phase<KBW, 2, BPW, F16>(a, P, L, U, uexp_v, act, dp, n_items, dw);
  else up_phase<KBW, 3, BPW, F16>(a, P, L, U, uexp_v, act, dp, n_items, dw);
  if (bhi > blo)
    down_phase<BPW, MODE, CPT, MODE == 1 && BPW <= 4, F16>(a, P, dyn_lds, ly, U, uexp_v, act, part, blo, bhi, dp, dw);
  dec_end(a, P, ep, parity);
#ifdef GI_TIMELINE
  GI_STAMP(9);
  tl_flush(a.timeline);
#endif
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
constexpr size_t kMaxDynLds = 160 * 1024 - 8 * 1024;  // room for the static prologue


int kbw_for(int H) { return H <= 512 ? 2 : 11; }

size_t lds_for(int kbw, int S, int I, int Gd, int units, int G) {
  const size_t g = kbw == 2 ? gu_lds_bytes<2>() : gu_lds_bytes<11>();
  return dn_layout(S, I, Gd, g, dn_max_blocks(units, S, G)).total;
}

// Residency of a kernel variant with `lds` bytes of dynamic LDS: the
// exchange between workgroups assumes that all workgroups of a launch (one
// per CU) run at the same time, so a variant is used only when the
// occupancy calculator puts at least one workgroup on every CU.  The
// dynamic-LDS limit is raised once per device and kernel first.  Results are
// cached per (device, kernel, LDS bytes).
struct ResEntry {
  int dev;
  const void* fn;
  size_t lds;
  int blocks;
};
constexpr int kResCache = 256;
std::mutex g_res_mu;
ResEntry g_res[kResCache];
int g_res_n = 0;

int blocks_per_cu(const void* fn, size_t lds, int* blocks) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  std::lock_guard<std::mutex> lk(g_res_mu);
  bool attr = false;
  for (int i = 0; i < g_res_n; ++i) {
    const ResEntry& r = g_res[i];
    if (r.dev == dev && r.fn == fn) {
      attr = true;
      if (r.lds == lds) {
        *blocks = r.blocks;
        return GI_OK;
      }
    }
  }
  if (!attr) {
    e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kMaxDynLds);
    if (e != hipSuccess) return hip_fail(e, "hipFuncSetAttribute(max dynamic LDS)");
  }
  int n = 0;
  e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, fn, kThreads, lds);
  if (e != hipSuccess) return hip_fail(e, "hipOccupancyMaxActiveBlocksPerMultiprocessor");
  if (g_res_n < kResCache) g_res[g_res_n++] = ResEntry{dev, fn, lds, n};
  *blocks = n;
  return GI_OK;
}

// Grid and variant of a launch of S slots: one workgroup per CU, fewer when
// the down units are few (at most kPartSlots workgroups share one unit), and
// enough that no workgroup gets more than kMaxItems gate/up items.
struct DecodePlan {
  int grid, bpw, cpt, mode;
};
bool decode_plan(int M, int S, int H, int I, int cus, DecodePlan& pl) {
  const int units = H / kUnitCols, tk = I / kCols;
  // U consecutive blocks meet at most ceil(G / units) + 1 workgroups
  int G = cus < kEpochSlots ? cus : kEpochSlots;
  if (G > (kPartSlots - 1) * units) G = (kPartSlots - 1) * units;
  if (G < 1 || ((long long)S * tk + G - 1) / G > kMaxItems) return false;
  if (G < units) return false;  // at most U blocks per workgroup (the scale staging holds S)
  pl.grid = G;
  pl.mode = M == 1 ? 1 : M == 2 ? 2 : 0;
  const int max_blocks = (units * S + G - 1) / G;
  pl.bpw = S <= kRows && max_blocks <= 4 ? 4 : 8;
  pl.cpt = S * (I / 8) <= 2 * kThreads ? 2 : kMaxStage;
  return true;
}

template <int KBW, bool F16>
const void* plan_kernel(const DecodePlan& pl) {
  if (pl.mode == 1 && pl.bpw == 4 && pl.cpt == 2) return (const void*)moe_decode_kernel<KBW, 1, 4, 2, F16>;
  if (pl.mode == 1) return (const void*)moe_decode_kernel<KBW, 1, 8, kMaxStage, F16>;
  if (pl.mode == 2) return (const void*)moe_decode_kernel<KBW, 2, 8, kMaxStage, F16>;
  return (const void*)moe_decode_kernel<KBW, 0, 8, kMaxStage, F16>;
}
// f16: fp16 activations, scales and out (fp16 products on q - 8 operands)
const void* decode_kernel(int kbw, const DecodePlan& pl, bool f16) {
  if (f16) return kbw == 2 ? plan_kernel<2, true>(pl) : plan_kernel<11, true>(pl);
  return kbw == 2 ? plan_kernel<2, false>(pl) : plan_kernel<11, false>(pl);
}

int log2_exact(int v) {
  int s = 0;
  while ((1 << s) < v) ++s;
  return (1 << s) == v ? s : -1;
}

}  // namespace

// Timeline builds: the caller's stamp buffer, used in slots of kEpochSlots
// workgroups x kStamps words, one slot per launch in rotation.
namespace {
std::mutex g_tl_mu;
unsigned long long* g_tl_buf = nullptr;
size_t g_tl_slots = 0, g_tl_next = 0;
}  // namespace

unsigned long long* decode_timeline_slot() {
  std::lock_guard<std::mutex> lk(g_tl_mu);
  if (!g_tl_buf || g_tl_slots == 0) return nullptr;
  unsigned long long* p = g_tl_buf + (g_tl_next % g_tl_slots) * (size_t)kEpochSlots * kStamps;
  ++g_tl_next;
  return p;
}

int set_decode_timeline(void* buf, size_t bytes) {
#ifdef GI_TIMELINE
  std::lock_guard<std::mutex> lk(g_tl_mu);
  g_tl_buf = (unsigned long long*)buf;
  g_tl_slots = buf ? bytes / ((size_t)kEpochSlots * kStamps * 8) : 0;
  g_tl_next = 0;
  return GI_OK;
#else
  (void)buf;
  (void)bytes;
  return fail(GI_ERR_UNSUPPORTED, "decode timeline: this library was built without the timeline option "
                                  "(python -m gemmainfer_amd.build --timeline builds libgemmainfer_amd_timeline.so)");
#endif
}

int moe_decode_rows_per_launch(int top_k) {
  if (top_k <= 0 || top_k > kSlots) return 0;
  const int r = kSlots / top_k;
  return r < kRows ? r : kRows;
}

bool moe_decode_supported(const MoeHostArgs& h) {
  // bf16 activations, or fp16 ones with caller-given routing
  if (h.x_dtype != GI_DTYPE_BF16 && !(h.x_dtype == GI_DTYPE_FP16 && !h.logits)) return false;
  if (h.H % 32 || h.I % 32 || h.H > kMaxUnits * kUnitCols || h.I > kMaxI) return false;
  if (h.gs % 32 || log2_exact(h.gs / 32) < 0) return false;
  // a scale group covers at least 2 k blocks: a wave's gate/up blocks span at
  // most six groups, its down blocks (at most three) at most two
  if (log2_exact(h.gs / 32) < 1) return false;
  if ((((uintptr_t)h.gu_scales) | ((uintptr_t)h.d_scales) | ((uintptr_t)h.out)) % 16) return false;
  if (h.top_k > kSlots || (h.logits && h.top_k > 64) || h.E > kRouteMaxExperts) return false;
  // whole tensors addressed with 32-bit buffer offsets
  if ((long long)h.E * (h.H / 8) * 2 * h.I * 4 >= (1LL << 32)) return false;
  if ((long long)h.E * (h.I / 8) * h.H * 4 >= (1LL << 32)) return false;
  if ((long long)h.E * h.Gd * h.H * 2 >= (1LL << 32)) return false;
  const int rows = moe_decode_rows_per_launch(h.top_k);
  if (rows < 1) return false;
  const int r1 = h.M < rows ? h.M : rows, S = r1 * h.top_k;
  DecodePlan pl;
  if (!decode_plan(r1, S, h.H, h.I, device_cu_count(), pl)) return false;
  if (pl.cpt > kMaxStage || S * (h.I / 8) > kMaxStage * kThreads) return false;
  // the down scales of a workgroup's blocks: at most kScaleLoads 16-byte chunks per thread
  if (dn_max_blocks(h.H / kUnitCols, S, pl.grid) * h.Gd * 4 > kScaleLoads * kThreads) return false;
  const size_t lds = lds_for(kbw_for(h.H), S, h.I, h.Gd, h.H / kUnitCols, pl.grid);
  if (lds > kMaxDynLds) return false;
  // every workgroup of the grid (one per CU) must be resident at once
  int blocks = 0;
  if (blocks_per_cu(decode_kernel(kbw_for(h.H), pl, h.x_dtype == GI_DTYPE_FP16), lds, &blocks) != GI_OK || blocks < 1)
    return false;
  return true;
}

size_t moe_decode_state_bytes() { return moe_state::state_bytes(); }

int launch_moe_decode(const MoeHostArgs& h, void* state, int* status) {
  const int rows_per = moe_decode_rows_per_launch(h.top_k);
  DecArgs k{};
  k.gu_packed = h.gu_packed;
  k.gu_scales = (const uint16_t*)h.gu_scales;
  k.d_packed = h.d_packed;
  k.d_scales = (const uint16_t*)h.d_scales;
  k.logits_dtype = h.logits_dtype;
  k.expert_scale = h.expert_scale;
  k.idx_is64 = h.idx_is64;
  k.w_dtype = h.w_dtype;
  k.H = h.H;
  k.I = h.I;
  k.E = h.E;
  k.top_k = h.top_k;
  k.gsh = log2_exact(h.gs / 32);
  k.Ggu = h.Ggu;
  k.Gd = h.Gd;
  k.Tk = h.I / kCols;
  k.units = h.H / kUnitCols;
  k.gu_bytes = (uint32_t)((h.H / 8) * 2 * h.I * 4);
  k.gus_bytes = (uint32_t)(h.Ggu * 2 * h.I * 2);
  k.dn_bytes = (uint32_t)((h.I / 8) * h.H * 4);
  k.gu_total = (uint32_t)((size_t)h.E * k.gu_bytes);
  k.gus_total = (uint32_t)((size_t)h.E * k.gus_bytes);
  k.dn_total = (uint32_t)((size_t)h.E * k.dn_bytes);
  k.dsc_total = (uint32_t)((size_t)h.E * h.Gd * h.H * 2);
  k.overwrite = h.overwrite;
  k.spin_limit = h.spin_limit > 0 ? h.spin_limit : kDefaultSpin;
  k.status = status;
  k.host_flag = device_error_flag(!h.no_alloc, h.stream);
  k.epochs = (unsigned long long*)state;
  k.act = (uint16_t*)((char*)state + moe_state::act_offset());
  k.part = (float*)((char*)state + moe_state::part_offset());

  const int kbw = kbw_for(h.H);
  const int cus = device_cu_count();
  const size_t idx_es = h.idx_is64 ? 8 : 4;
  const size_t w_es = h.w_dtype == GI_DTYPE_FP32 ? 4 : 2;
  for (int r0 = 0; r0 < h.M; r0 += rows_per) {
    const int rows = (h.M - r0) < rows_per ? (h.M - r0) : rows_per;
    k.M = rows;
    k.S = rows * h.top_k;
    DecodePlan pl;
    if (!decode_plan(rows, k.S, h.H, h.I, cus, pl)) return fail(GI_ERR_UNSUPPORTED, "fused MoE decode: no grid");
    k.x = (const uint16_t*)h.x + (size_t)r0 * h.H;
    k.out = (uint16_t*)h.out + (size_t)r0 * h.H;
    k.idx = h.idx ? (const char*)h.idx + (size_t)r0 * h.top_k * idx_es : nullptr;
    k.w = h.w ? (const char*)h.w + (size_t)r0 * h.top_k * w_es : nullptr;
    k.logits = h.logits ? (const char*)h.logits + (size_t)r0 * h.E * (h.logits_dtype == GI_DTYPE_FP32 ? 4 : 2)
                        : nullptr;
    k.out_idx = h.out_idx ? h.out_idx + (size_t)r0 * h.top_k : nullptr;
    k.out_w = h.out_w ? (uint16_t*)h.out_w + (size_t)r0 * h.top_k : nullptr;
    const size_t lds = lds_for(kbw, k.S, k.I, k.Gd, k.units, pl.grid);
    const void* fn = decode_kernel(kbw, pl, h.x_dtype == GI_DTYPE_FP16);
    int blocks = 0;
    int st = blocks_per_cu(fn, lds, &blocks);  // also raises the kernel's dynamic-LDS limit
    if (st != GI_OK) return st;
    if (blocks < 1) return fail(GI_ERR_UNSUPPORTED, "fused MoE decode: a workgroup does not fit on a CU");
    k.timeline = decode_timeline_slot();
    void* args[] = {(void*)&k};
    const hipError_t e = hipLaunchKernel(fn, dim3(pl.grid), dim3(kThreads), args, lds, h.stream);
    if (e != hipSuccess) return hip_fail(e, "fused MoE decode launch");
  }
  return GI_OK;
}

}  // namespace gi
