// Token-Union W4A16 fused MoE for small token counts (decode M=1, verify
// M<=8, any launch of up to 256 slots) on gfx950.
//
// Reference behaviour restated (paths relative to the GemmaInfer repo):
//   routing        gemmainfer/models/gemma.py:77-80
//   dedup          csrc/marlin.cu:285-335 (gate_up) / :453-505 (down)
//   gate_up + GELU csrc/marlin.cu:337-426
//   down + combine csrc/marlin.cu:507-586
//
// One launch per layer, ONE inter-workgroup synchronisation.
//
//   prologue  Every workgroup routes the tokens (layer mode: top-k + softmax
//             per token, one wave per token, DPP row reductions) and builds the
//             Token-Union alignment in LDS: the distinct valid expert ids in
//             first-occurrence slot order and each slot's unique index.
//   tasks     Task (u, c) owns intermediate columns [c*CG, (c+1)*CG) of unique
//             expert u.  It streams the matching gate and up columns over the
//             whole hidden dimension (registers, 16-byte non-temporal loads),
//             reduces them across lanes and waves, applies gelu_tanh(gate)*up
//             and rounds to bf16 (where the reference stores its activation),
//             then multiplies those CG activations by the CG/8 packed rows of
//             the down projection they meet -- across all H output columns --
//             whose words were streamed straight into LDS (global_load_lds)
//             at task start.  The activation never leaves the workgroup.
//             Result: an fp32 partial w[slot]*y for every slot of u, written
//             to part[slot][c][:] with coherent (sc1) stores.
//   barrier   One grid-wide arrival counter (all workgroups are resident: the
//             grid is sized from the occupancy calculator).
//   reduce    Every workgroup sums a slice of output columns over
//             (slot of the token, c) in a fixed order, adds it to out and
//             rounds once to bf16.  No float atomics; bitwise deterministic.
//
// Waits are bounded (spin_limit) and report GI_DEVICE_SPIN_TIMEOUT instead of
// hanging; the counters are reset by the last workgroup out.

#include <limits.h>

#include <mutex>

#include "../../include/gemmainfer_amd.h"
#include "gi_common.h"
#include "gi_internal.h"
#include "moe_shared.h"

namespace gi {

namespace {

using namespace moe;

constexpr int kMaxSlots = 256;
constexpr int kMaxExperts = 1024;
constexpr int kMaxWaves = 16;
constexpr int kDefaultSpin = 1 << 22;
constexpr int kCtrStride = 32;     // ints between counters (128 bytes: separate lines)
constexpr int kCtrSlots = 5;       // counter words (the last one: prefill arrivals)

typedef __attribute__((address_space(3))) void* lds_ptr_t;
typedef const __attribute__((address_space(1))) void* gbl_ptr_t;

struct Args {
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
  float* part;      // [S][Tg][H] fp32 partials
  uint32_t part_bytes;
  int* ctr;         // grid barrier: [0] launch epoch, [(1 + p) * kCtrStride] arrivals of parity p,
                    // [3 * kCtrStride] the last epoch whose barrier wait timed out
                    // ([4 * kCtrStride]: the prefill front launch's arrivals)
  int* status;
  int* host_flag;   // host-visible error flag of the device (may be null)
  int idx_is64, w_dtype, logits_dtype;
  int M, H, I, E, top_k, gs, Ggu, Gd, S, Tg;
  int overwrite, spin_limit;
  int qpw;          // reduction: output quads per workgroup pass (power of two)
};

// LDS of one task (static __shared__ arrays declared by the kernel).
template <int CG, int NT, int JGM, int CPR>
struct TaskLds {
  static constexpr int T = 16 * CG, W = T / 64, DR = CG / 8, KPM = 32 * JGM;
  uint4* xs;        // [NT][KPM] pair-permuted x words
  float* xb;        // [NT][KPM] -24 * sum of each x word
  float* red;       // [W][NT][2*CG] per-wave gate/up sums
  uint16_t* actp;   // [NT][DR][8] pair-permuted bf16 activations
  float* actb;      // [NT][DR] -24 * sum of each activation row
};

struct Prologue {
  int first_slot[kMaxExperts];
  int slot_e[kMaxSlots];
  int slot_u[kMaxSlots];      // unique index of each slot, -1 if skipped
  float slot_w[kMaxSlots];    // routing weight (bf16-rounded)
  int rank_of_slot[kMaxSlots];
  int uexp[kMaxSlots];        // expert id of each unique index
  int list[kMaxSlots];        // slots of the current task's expert, ascending (S > 64)
  int uoff[kMaxSlots + 1];    // S <= 64: slots of unique u are csr[uoff[u] .. uoff[u+1])
  int csr[kMaxSlots];
  int wave_cnt[kMaxWaves];
  int n_unique;
  int n_list;
};


// Token-Union alignment of up to 64 slots by one wave, without LDS atomics
// or barriers: lane s holds slot s's expert id; each round takes the lowest
// remaining slot, retires every slot routed to the same expert, and so
// enumerates the distinct ids in first-occurrence order (marlin.cu:298-319).
// Also writes the per-expert slot lists (CSR, slots ascending).
__device__ __forceinline__ void align_wave(const Args& a, Prologue& P, int lane) {
  const int e = lane < a.S ? P.slot_e[lane] : -1;
  unsigned long long rem = __ballot(e >= 0);
  int u = 0, run = 0, my_u = -1, my_pos = 0;
  while (rem) {
    const int s0 = __builtin_ctzll(rem);
    const int e0 = __builtin_amdgcn_readlane(e, s0);
    const unsigned long long m = __ballot(e == e0) & rem;
    if ((m >> lane) & 1ull) {
      my_u = u;
      my_pos = run + __popcll(m & ((1ull << lane) - 1ull));
    }
    if (lane == 0) {
      P.uexp[u] = e0;
      P.uoff[u] = run;
    }
    run += __popcll(m);
    rem &= ~m;
    ++u;
  }
  if (lane < a.S) {
    P.slot_u[lane] = my_u;
    if (my_u >= 0) P.csr[my_pos] = lane;
  }
  if (lane == 0) {
    P.uoff[u] = run;
    P.n_unique = u;
  }
}

// Routing (layer mode: one wave per token, gemma.py:77-80) or id/weight load,
// then the Token-Union alignment: the distinct valid ids in first-occurrence
// slot order (marlin.cu:298-319) and each slot's unique index.  All T threads.
template <int T>
__device__ void prologue(const Args& a, Prologue& P) {
  constexpr int W = T / kWave;
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid >> 6;
  const int S = a.S;
  if (a.logits) {
    for (int t = wave; t < a.M; t += W)
      route_token_any(a, t, lane, P.slot_e + t * a.top_k, P.slot_w + t * a.top_k);
  } else if (tid < S) {
    const int e = load_expert_id(a.idx, a.idx_is64, tid);
    P.slot_e[tid] = (e >= 0 && e < a.E) ? e : -1;
    P.slot_w[tid] = a.w ? load_weight_as_bf16(a.w, a.w_dtype, tid) : 0.f;
  }
  // A single routed token lives in wave 0, which can go on without a barrier.
  if (!(a.logits && a.M == 1)) __syncthreads();
  if (a.logits && tid < S) {
    const float wr = round_to_bf16(P.slot_w[tid]);
    P.slot_w[tid] = wr;
    if (blockIdx.x == 0) {
      if (a.out_idx) a.out_idx[tid] = P.slot_e[tid];
      if (a.out_w) a.out_w[tid] = f32_to_bf16(wr);
    }
  }
  if (S <= kWave) {
    if (wave == 0) align_wave(a, P, lane);
    __syncthreads();
    return;
  }
  for (int i = tid; i < a.E; i += T) P.first_slot[i] = INT_MAX;
  __syncthreads();
  int e = -1;
  if (tid < S) {
    e = P.slot_e[tid];
    if (e >= 0) atomicMin(&P.first_slot[e], tid);
  }
  __syncthreads();
  const bool is_first = tid < S && e >= 0 && P.first_slot[e] == tid;
  const unsigned long long bal = __ballot(is_first);
  const int below = __popcll(bal & ((1ull << lane) - 1ull));
  if (lane == 0) P.wave_cnt[wave] = __popcll(bal);
  __syncthreads();
  int base = 0, total = 0;
#pragma unroll
  for (int w = 0; w < W; ++w) {
    const int c = P.wave_cnt[w];
    base += (w < wave) ? c : 0;
    total += c;
  }
  if (is_first) {
    P.uexp[base + below] = e;
    P.rank_of_slot[tid] = base + below;
  }
  if (tid == 0) P.n_unique = total;
  __syncthreads();
  if (tid < S) P.slot_u[tid] = e >= 0 ? P.rank_of_slot[P.first_slot[e]] : -1;
  __syncthreads();
}

// Collect the slots (ascending) routed to unique expert u into P.list.
template <int T>
__device__ void gather_list(const Args& a, Prologue& P, int u) {
  constexpr int W = T / kWave;
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid >> 6;
  const bool mine = tid < a.S && P.slot_u[tid] == u;
  const unsigned long long bal = __ballot(mine);
  const int below = __popcll(bal & ((1ull << lane) - 1ull));
  __syncthreads();  // earlier readers of list / wave_cnt are done
  if (lane == 0) P.wave_cnt[wave] = __popcll(bal);
  __syncthreads();
  int base = 0, total = 0;
#pragma unroll
  for (int w = 0; w < W; ++w) {
    const int c = P.wave_cnt[w];
    base += (w < wave) ? c : 0;
    total += c;
  }
  if (mine) P.list[base + below] = tid;
  if (tid == 0) P.n_list = total;
  __syncthreads();
}

// ---------------------------------------------------------------------------
// task (u, c)
// ---------------------------------------------------------------------------
template <int N>
struct Count {
  static constexpr int value = N;
};
// f(Count<n>{}) for the runtime n in [1, NMAX]: one straight-line body per n.
template <int NMAX, typename F>
__device__ __forceinline__ void with_count(int n, F&& f) {
  if constexpr (NMAX > 1) {
    if (n >= NMAX) {
      f(Count<NMAX>{});
      return;
    }
    with_count<NMAX - 1>(n, f);
  } else {
    f(Count<1>{});
  }
}
template <int CG, int NT, int JGM, int CPR>
__device__ void run_task(const Args& a, Prologue& P, int u, int c, const TaskLds<CG, NT, JGM, CPR>& S) {
  constexpr int T = 16 * CG;      // threads
  constexpr int W = T / kWave;    // waves
  constexpr int L = CG / 2;       // lanes per packed row: CG/4 gate quads + CG/4 up quads
  constexpr int HALF = CG / 4;
  constexpr int DR = CG / 8;      // packed rows of the down projection this task meets
  constexpr int KPM = 32 * JGM;   // packed rows of x staged (>= H/8)
  constexpr int DQM = (CPR * kWave + T - 1) / T;  // output quads per thread in the down step
  constexpr int XPT = (NT * KPM + T - 1) / T;     // staged x words per thread (first chunk)
  // The per-lane offsets below are recomputed per task (a few integer ops)
  // rather than hoisted out of the task loop, where they would sit in
  // registers through the whole kernel.
  int tid = threadIdx.x;
  asm volatile("" : "+v"(tid));
  const int lane = tid & (kWave - 1);
  const int wave = tid >> 6;
  const int q = tid % L, rl = tid / L;  // rl in [0, 32): this lane's row within a 32-row step
  const bool is_up = q >= HALF;
  const int cq = is_up ? q - HALF : q;
  const int icol = c * CG + cq * 4;     // intermediate column of this lane's quad
  const bool col_ok = icol < a.I;
  const int e = P.uexp[u];
  const int Kp = a.H >> 3, Ip = a.I >> 3, twoI = 2 * a.I, rpg = a.gs >> 3, HQ = a.H >> 2;
  // Rows without a scale group are dropped (the reference sizes its loops by
  // the scale tensor, marlin.cu:128): x is staged as zero from row Kv on, and
  // activations from column Iv on, so no per-row mask is needed below.
  const int Kv = min(Kp, a.Ggu * rpg), Iv = min(a.I, a.Gd * a.gs);

  uint4* xs = S.xs;
  float* xb = S.xb;
  float* red = S.red;
  uint16_t* actp = S.actp;
  float* actb = S.actb;
  const __amdgpu_buffer_rsrc_t part = buffer_rsrc(a.part, a.part_bytes);

  // slots routed to expert u, ascending
  const int* list;
  int nmatch;
  if (a.S <= kWave) {
    list = P.csr + P.uoff[u];
    nmatch = P.uoff[u + 1] - P.uoff[u];
  } else {
    gather_list<T>(a, P, u);
    list = P.list;
    nmatch = P.n_list;
  }

  // Every load below is a plain register load, straight-line with a fixed
  // count per thread (addresses of unused lanes/rows are clamped, not
  // skipped), so the compiler's vmcnt waits are exact: staging x waits only
  // for the x words (issued first), row j of the gate/up sum only for the
  // loads up to row j, and the down step finds its words already in flight.
  // (Direct-to-LDS loads or stores pending here would turn every such wait
  // into a full drain: the wait-count pass treats mixed events as unordered.)
  // (1) x words of the first token chunk
  uint4 xr[XPT];
  {
    const int nch0 = min(NT, nmatch);
#pragma unroll
    for (int i = 0; i < XPT; ++i) {
      const int id = tid + i * T, n = id / KPM, r = id - n * KPM;
      const bool v = n < nch0 && r < Kv;
      const int tok = list[v ? n : 0] / a.top_k;
      xr[i] = *(const uint4*)(a.x + (size_t)tok * a.H + 8 * (v ? r : 0));
    }
  }
  const int icol_c = col_ok ? icol : 0;
  const int32_t* gp = a.gu_packed + (size_t)e * Kp * twoI + (is_up ? a.I : 0) + icol_c;
  const uint16_t* gsp = a.gu_scales + (size_t)e * a.Ggu * twoI + (is_up ? a.I : 0) + icol_c;
  const int g0 = (c * DR) / rpg, g1 = (c * DR + DR - 1) / rpg;
  const bool one_group = g0 == g1;
  const uint16_t* dsp = a.d_scales + (size_t)e * a.Gd * a.H;
  const int32_t* dp = a.d_packed + (size_t)e * Ip * a.H;
  uint4 wv[JGM];
  uint2 sg[JGM];
  uint2 sd[DQM];
  uint4 dw[DQM][DR];
  auto load_weights = [&]() {
    __builtin_amdgcn_sched_barrier(0);  // keep the issue order: x, gate/up, down scales, down words
    // (2) gate/up words of this lane's column quad, every 32nd row, and their scales
#pragma unroll
    for (int j = 0; j < JGM; ++j) {
      const int r = min(32 * j + rl, Kv - 1);
      wv[j] = load_nt_u4(gp + r * twoI);
      sg[j] = *(const uint2*)(gsp + (r / rpg) * twoI);
    }
    __builtin_amdgcn_sched_barrier(0);
    // (3) down scales of this thread's output quads (one group per task when
    //     gs is a multiple of CG; otherwise looked up per row in the down step)
#pragma unroll
    for (int m = 0; m < DQM; ++m) {
      const int hq = min(tid + m * T, HQ - 1);
      sd[m] = *(const uint2*)(dsp + min(g0, a.Gd - 1) * a.H + 4 * hq);
    }
    __builtin_amdgcn_sched_barrier(0);
    // (4) the packed down rows [c*DR, c*DR+DR) of expert e at this thread's
    //     output quads: the CG/8 rows the task's activations meet.
#pragma unroll
    for (int m = 0; m < DQM; ++m) {
      const int hq = min(tid + m * T, HQ - 1);
#pragma unroll
      for (int r = 0; r < DR; ++r) dw[m][r] = load_nt_u4(dp + min(c * DR + r, Ip - 1) * a.H + 4 * hq);
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  load_weights();
  const uint32_t mq = q4_magic();

  // One chunk of NC (1..NT) of the expert's slots, straight-line for each NC.
  // The first chunk is peeled out of the loop below, so that its waits stay
  // exact.
  auto chunk = [&](auto nc_tag, int c0, bool first) {
    constexpr int NC = decltype(nc_tag)::value;
    const int nch = NC;
    if (first) {
#pragma unroll
      for (int i = 0; i < XPT; ++i) {
        const int id = tid + i * T, n = id / KPM, r = id - n * KPM;
        if (n < NT) {
          const bool v = n < nch && r < Kv;
          const uint4 d = v ? xr[i] : make_uint4(0u, 0u, 0u, 0u);
          xs[n * KPM + r] = pair_permute(d);
          xb[n * KPM + r] = q4_bias(d);
        }
      }
    } else {
      for (int i = tid; i < NT * KPM; i += T) {
        const int n = i / KPM, r = i - n * KPM;
        uint4 d = make_uint4(0u, 0u, 0u, 0u);
        if (n < nch && r < Kv) {
          const int tok = list[c0 + n] / a.top_k;
          d = *(const uint4*)(a.x + (size_t)tok * a.H + 8 * r);
        }
        xs[n * KPM + r] = pair_permute(d);
        xb[n * KPM + r] = q4_bias(d);
      }
    }
    __syncthreads();

    // gate/up partial sums over this lane's rows, row by row as words arrive;
    // each word is unpacked once for every token of the chunk
    float acc[4][NC];
#pragma unroll
    for (int qq = 0; qq < 4; ++qq)
#pragma unroll
      for (int n = 0; n < NC; ++n) acc[qq][n] = 0.f;
#pragma unroll
    for (int j = 0; j < JGM; ++j) {
      const int r = 32 * j + rl;
      const uint2 s2 = opaque(sg[j]);
      const float sc[4] = {bf16lo(s2.x), bf16hi(s2.x), bf16lo(s2.y), bf16hi(s2.y)};
      const uint4 w = opaque(wv[j]);
      const Q4Pairs d[4] = {unpack_q4(w.x, mq), unpack_q4(w.y, mq), unpack_q4(w.z, mq),
                            unpack_q4(w.w, mq)};
#pragma unroll
      for (int n = 0; n < NC; ++n) {
        const uint4 xp = xs[n * KPM + r];
        const float b = xb[n * KPM + r];
#pragma unroll
        for (int qq = 0; qq < 4; ++qq) acc[qq][n] += sc[qq] * dot_unpacked(d[qq], xp, b);
      }
    }
    // lanes of one wave that share q hold different rows: reduce, then waves via LDS
#pragma unroll
    for (int qq = 0; qq < 4; ++qq)
#pragma unroll
      for (int n = 0; n < NC; ++n) acc[qq][n] = reduce_across_groups<L>(acc[qq][n]);
    if (lane < L) {
#pragma unroll
      for (int n = 0; n < NC; ++n)
#pragma unroll
        for (int qq = 0; qq < 4; ++qq)
          red[(wave * NT + n) * 2 * CG + (is_up ? CG : 0) + cq * 4 + qq] = acc[qq][n];
    }
    __syncthreads();

    // gelu_tanh(gate) * up, rounded to bf16 (where the reference stores its
    // activation, marlin.cu:421-423), pair-permuted per packed row, + bias
    if (tid < NC * CG) {
      const int n = tid / CG, ci = tid - n * CG;
      float g = 0.f, up = 0.f;
#pragma unroll
      for (int w2 = 0; w2 < W; ++w2) {
        g += red[(w2 * NT + n) * 2 * CG + ci];
        up += red[(w2 * NT + n) * 2 * CG + CG + ci];
      }
      const float av = (c * CG + ci < Iv) ? round_to_bf16(gelu_tanh(g) * up) : 0.f;
      float s8 = av;  // sum over the 8 activations of this packed row (8 adjacent lanes)
      s8 += __shfl_xor(s8, 1, kWave);
      s8 += __shfl_xor(s8, 2, kWave);
      s8 += __shfl_xor(s8, 4, kWave);
      const int r8 = ci >> 3, p = ci & 7;
      actp[(n * DR + r8) * 8 + 2 * (p & 3) + (p >> 2)] = f32_to_bf16(av);
      if (p == 0) actb[n * DR + r8] = -24.0f * s8;
    }
    __syncthreads();

    // down: y[h] = sum over the task's CG activations of act * w_down
    const uint4* actq = (const uint4*)actp;
#pragma unroll
    for (int m = 0; m < DQM; ++m) {
      const int hq = tid + m * T;
      if (hq >= HQ) continue;
      float y[NC][4];
#pragma unroll
      for (int n = 0; n < NC; ++n) y[n][0] = y[n][1] = y[n][2] = y[n][3] = 0.f;
#pragma unroll
      for (int r = 0; r < DR; ++r) {
        uint2 s2 = opaque(sd[m]);  // a value, so the select below stays a select of values
        if (!one_group) {
          const int g = min((c * DR + r) / rpg, a.Gd - 1);
          s2 = *(const uint2*)(dsp + g * a.H + 4 * hq);
        }
        const float sc[4] = {bf16lo(s2.x), bf16hi(s2.x), bf16lo(s2.y), bf16hi(s2.y)};
        const uint4 w = opaque(dw[m][r]);
        const Q4Pairs dq[4] = {unpack_q4(w.x, mq), unpack_q4(w.y, mq), unpack_q4(w.z, mq),
                               unpack_q4(w.w, mq)};
#pragma unroll
        for (int n = 0; n < NC; ++n) {
          const uint4 xp = actq[n * DR + r];
          const float b = actb[n * DR + r];
#pragma unroll
          for (int qq = 0; qq < 4; ++qq) y[n][qq] += sc[qq] * dot_unpacked(dq[qq], xp, b);
        }
      }
#pragma unroll
      for (int n = 0; n < NC; ++n) {
        const int slot = list[c0 + n];
        const float ws = P.slot_w[slot];
        const uint32_t off = (uint32_t)(((slot * a.Tg + c) * a.H + 4 * hq) * 4);
        st_coherent_f4(part, off, make_float4(y[n][0] * ws, y[n][1] * ws, y[n][2] * ws, y[n][3] * ws));
      }
    }
    __syncthreads();  // xs / red / act reused by the next chunk or task
  };
  with_count<NT>(min(NT, nmatch), [&](auto nc) { chunk(nc, 0, true); });
  for (int c0 = NT; c0 < nmatch; c0 += NT) {  // more slots than NT: reload the weights
    load_weights();
    with_count<NT>(min(NT, nmatch - c0), [&](auto nc) { chunk(nc, c0, false); });
  }
}

// ---------------------------------------------------------------------------
// reduction of the partials into out
// ---------------------------------------------------------------------------
template <int T>
__device__ void reduce_partials(const Args& a, const Prologue& P, float4* scratch, bool bad) {
  constexpr int W = T / kWave;
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid >> 6;
  const int HQ = a.H >> 2, total = a.M * HQ;
  const int qpw = a.qpw, stripes = T / qpw;
  const int qi = tid & (qpw - 1), st = tid / qpw;
  const int np = a.top_k * a.Tg;
  const __amdgpu_buffer_rsrc_t part = buffer_rsrc(a.part, a.part_bytes);
  for (int qb = blockIdx.x * qpw; qb < total; qb += gridDim.x * qpw) {
    const int quad = qb + qi;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    if (quad < total) {
      const int t = quad / HQ, hq = quad - t * HQ;
      // batches of four partials: addresses and validity first, then the
      // four loads in flight together (slots without an expert wrote nothing)
      for (int p0 = st; p0 < np; p0 += 4 * stripes) {
        float4 v[4];
        bool ok[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int p = min(p0 + i * stripes, np - 1);
          const int k = p / a.Tg, cc = p - k * a.Tg;
          const int s = t * a.top_k + k;
          ok[i] = p0 + i * stripes < np && P.slot_u[s] >= 0;
          v[i] = ld_coherent_f4(part, (uint32_t)(((s * a.Tg + cc) * a.H + 4 * hq) * 4));
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if (ok[i]) {
            acc.x += v[i].x;
            acc.y += v[i].y;
            acc.z += v[i].z;
            acc.w += v[i].w;
          }
        }
      }
    }
    // fixed-shape reduction over the stripes (deterministic order): lanes of
    // a wave that share qi first, then the waves through LDS
    for (int off = qpw; off < kWave; off <<= 1) {
      acc.x += __shfl_xor(acc.x, off, kWave);
      acc.y += __shfl_xor(acc.y, off, kWave);
      acc.z += __shfl_xor(acc.z, off, kWave);
      acc.w += __shfl_xor(acc.w, off, kWave);
    }
    const int per_wave = qpw < kWave ? qpw : kWave;  // distinct stripes' sums a wave holds
    if (lane < per_wave) scratch[wave * per_wave + lane] = acc;
    __syncthreads();
    if (tid < qpw && quad < total) {
      // quad qi was summed by waves qi / per_wave + k * (qpw / per_wave), in increasing order
      float4 sum = make_float4(0.f, 0.f, 0.f, 0.f);
      const int wstep = qpw / per_wave;  // waves between two holders of the same quad
      for (int w = qi / per_wave; w < W; w += wstep) {
        const float4 v = scratch[w * per_wave + (qi % per_wave)];
        sum.x += v.x;
        sum.y += v.y;
        sum.z += v.z;
        sum.w += v.w;
      }
      const int t = quad / HQ, hq = quad - t * HQ;
      uint2* o = (uint2*)(a.out + (size_t)t * a.H + 4 * hq);
      if (!a.overwrite) {
        const uint2 old = *o;
        sum.x += bf16lo(old.x);
        sum.y += bf16hi(old.x);
        sum.z += bf16lo(old.y);
        sum.w += bf16hi(old.y);
      }
      if (bad) sum = make_float4(__uint_as_float(0x7fc00000u), __uint_as_float(0x7fc00000u),
                                 __uint_as_float(0x7fc00000u), __uint_as_float(0x7fc00000u));
      *o = make_uint2((uint32_t)f32_to_bf16(sum.x) | ((uint32_t)f32_to_bf16(sum.y) << 16),
                      (uint32_t)f32_to_bf16(sum.z) | ((uint32_t)f32_to_bf16(sum.w) << 16));
    }
    __syncthreads();
  }
}

// Grid-wide barrier (every partial of every task is written), then the
// reduction of the partials into out.
template <int T>
__device__ __forceinline__ void finish_layer(const Args& a, const Prologue& P, int my_gen, float4* scratch) {
  const int tid = threadIdx.x;
  __shared__ int s_bad;  // the wait gave up: this workgroup's outputs are written as NaN
  if (tid == 0) s_bad = 0;
  // Grid-wide barrier (every partial of every task is written).  Launches
  // alternate between two arrival counters by the parity of the launch epoch
  // (read above, before this workgroup can arrive, so every workgroup of a
  // launch reads the same value).  Each workgroup adds one arrival; the last
  // one clears the other parity's counter (idle until the next launch) and
  // advances the epoch, which the others poll (a separate cache line, so the
  // polling does not queue behind the arrivals).
  wait_vmem();
  __syncthreads();
  if (tid == 0) {
    const int G = gridDim.x;
    int* cnt = a.ctr + (1 + (my_gen & 1)) * kCtrStride;
    if (atomic_add_relaxed(cnt, 1) == G - 1) {
      store_relaxed(a.ctr + (1 + ((my_gen + 1) & 1)) * kCtrStride, 0);
      store_relaxed(a.ctr, my_gen + 1);
    } else {
      // A waiter that gives up marks this launch's epoch so the others stop
      // waiting too; the mark names the epoch, so a later launch (another
      // epoch) is not cut short by it.
      int* gave_up = a.ctr + 3 * kCtrStride;
      int spins = 0;
      while (load_relaxed(a.ctr) == my_gen) {
        if (++spins >= a.spin_limit || load_relaxed(gave_up) == my_gen + 1) {
          store_relaxed(gave_up, my_gen + 1);
          report_timeout(a.status, a.host_flag);
          s_bad = 1;
          break;
        }
      }
    }
  }
  __syncthreads();
  reduce_partials<T>(a, P, scratch, s_bad != 0);
}

template <int CG, int NT, int JGM, int CPR>
__global__ __launch_bounds__(16 * CG) void fused_moe_kernel(Args a) {
  constexpr int T = 16 * CG;
  using Lds = TaskLds<CG, NT, JGM, CPR>;
  __shared__ Prologue P;
  __shared__ float4 s_scratch[T];
  __shared__ uint4 s_xs[NT * Lds::KPM];
  __shared__ float s_xb[NT * Lds::KPM];
  __shared__ float s_red[Lds::W * NT * 2 * CG];
  __shared__ __attribute__((aligned(16))) uint16_t s_actp[NT * Lds::DR * 8];
  __shared__ float s_actb[NT * Lds::DR];
  const Lds S{s_xs, s_xb, s_red, s_actp, s_actb};
  const int tid = threadIdx.x;
  // barrier generation of this launch (read before this workgroup can arrive)
  const int my_gen = tid == 0 ? load_relaxed(a.ctr) : 0;
  prologue<T>(a, P);
  const int ntask = P.n_unique * a.Tg;
  for (int t = blockIdx.x; t < ntask; t += gridDim.x)
    run_task<CG, NT, JGM, CPR>(a, P, t / a.Tg, t % a.Tg, S);

  finish_layer<T>(a, P, my_gen, s_scratch);
}

// Export of the alignment (gi_moe_align): one workgroup of 256 threads.
// ---------------------------------------------------------------------------
// Matrix-core task (group_size a multiple of 32; up to 8 resident tokens)
//
// Both projections run on v_mfma_f32_16x16x32_bf16, D[16x16] += A[16x32] *
// B[32x16], lane l holding A[l%16][8(l/16)..+8), B[8(l/16)..+8][l%16] and
// D[4(l/16)..+4][l%16].  B is the weights: one packed word per lane is
// exactly 8 consecutive k of one output column, unpacked to bf16 (16+q)
// pairs in the order (0,4)(2,6)(1,5)(3,7).  A is the activations of up to 16
// slots (rows), kept in LDS in that same k order.  A second product against a
// constant -24 matrix supplies -24*sum(a), so D + Db = sum a*(q-8) exactly
// as the fp32 accumulation of bf16 products; the group scale multiplies that
// when a scale group ends.  Per packed word this is 7 VALU (the unpack),
// whatever the number of tokens.
//
//   gate/up  wave w owns k blocks [w*KBW, (w+1)*KBW) (32 k each) for all 64
//            task columns: lane (lq = l/16, lr = l%16) loads the 16-byte word
//            quad of columns 4lr..4lr+3 (gate for lr < 8, up otherwise) at
//            packed row 4kb+lq; word i feeds MFMA i, whose column lr is task
//            column 4lr+i.  Partial sums per wave go through LDS.
//   act      gelu_tanh(gate)*up rounded to bf16 (marlin.cu:421-423).
//   down     one A operand for the task (the activations); wave w owns the
//            64-column output groups [w*DGW, (w+1)*DGW), one word quad per
//            lane and group, the scale of the task's (single) group.
// ---------------------------------------------------------------------------

constexpr int kMfmaThreads = 512;
constexpr int kMfmaWaves = kMfmaThreads / kWave;
constexpr int kResidentTokens = 8;   // x rows staged in LDS by the prologue
constexpr int kChunkRows = 16;       // slots per MFMA pass


template <int KBW, int DGW>
struct MfmaLds {
  static constexpr int KPM = 4 * KBW * kMfmaWaves;  // packed x rows staged (>= H/8)
  static constexpr int GW = KBW + 1;                // scale groups one wave's k blocks can touch
};

template <int KBW, int DGW>
__device__ void run_task_mfma(const Args& a, Prologue& P, int u, int c, const uint4* s_x, float4* s_red,
                              uint4* s_act, uint4* s_sc) {
  constexpr int KPM = MfmaLds<KBW, DGW>::KPM;
  constexpr int GW = MfmaLds<KBW, DGW>::GW;
  constexpr int SCT = (GW * 8 + kWave - 1) / kWave;  // scale chunks per lane
  static_assert(SCT <= 3, "three scale chunks per lane at most");
  constexpr int W = kMfmaWaves;
  int tid = threadIdx.x;
  asm volatile("" : "+v"(tid));  // per-task lane offsets, not hoisted out of the task loop
  const int lane = tid & (kWave - 1), wave = tid >> 6;
  const int lr = lane & 15, lq = lane >> 4;
  const int e = P.uexp[u];
  const int Kp = a.H >> 3, Ip = a.I >> 3, twoI = 2 * a.I;
  const int HG = (a.H + 63) >> 6;            // 64-column output groups
  const int KPG = a.gs >> 5;                 // 32-k blocks per scale group
  const int Iv = min(a.I, a.Gd * a.gs);      // activations past the last down group are dropped

  const int* list;
  int nmatch;
  if (a.S <= kWave) {
    list = P.csr + P.uoff[u];
    nmatch = P.uoff[u + 1] - P.uoff[u];
  } else {
    gather_list<kMfmaThreads>(a, P, u);
    list = P.list;
    nmatch = P.n_list;
  }

  // this lane's four task columns (gate for lr < 8, up otherwise)
  const int tcol = 4 * lr;
  const int icol = c * 32 + (tcol & 31);
  const bool col_ok = icol < a.I;
  const int gcol = (col_ok ? icol : 0) + (lr < 8 ? 0 : a.I);
  const int32_t* gp = a.gu_packed + (size_t)e * Kp * twoI + gcol;
  const int prow = min(c * 4 + lq, Ip - 1);  // this lane's packed down row
  const int gd = min((c * 32) / a.gs, a.Gd - 1);
  const int32_t* dp = a.d_packed + ((size_t)e * Ip + prow) * a.H;
  const uint16_t* dsp = a.d_scales + ((size_t)e * a.Gd + gd) * a.H;
  const int kb0 = wave * KBW;

  // The gate/up scale rows of the groups this wave's k blocks touch,
  // [group][64 task columns] bf16, go to the wave's own LDS slice (8 x 16
  // bytes per group: gate quarters, then up quarters); no workgroup barrier.
  const int wg0 = kb0 / KPG;  // first scale group of this wave
  const uint16_t* sc_base = a.gu_scales + (size_t)e * a.Ggu * twoI;
  uint4* w_sc = s_sc + wave * GW * 8;
  // (named values, not an array: a private array may be placed in LDS)
  uint4 scv0 = make_uint4(0u, 0u, 0u, 0u), scv1 = scv0, scv2 = scv0;
  auto sc_load = [&](int i) {
    const int id = lane + i * kWave, g = min(wg0 + (id >> 3), a.Ggu - 1), part = id & 7;
    return *(const uint4*)(sc_base + (size_t)g * twoI + (part < 4 ? 0 : a.I) + min(c * 32 + 8 * (part & 3), a.I - 8));
  };
  uint4 wv[KBW];
  uint4 dw[DGW];
  uint2 sdw[DGW];
  // Fixed-count register loads (clamped addresses): scales, gate/up, down,
  // in that order, so the compiler's vmcnt waits stay exact.
  auto load_weights = [&]() {
    __builtin_amdgcn_sched_barrier(0);
    scv0 = sc_load(0);
    if constexpr (SCT > 1) scv1 = sc_load(1);
    if constexpr (SCT > 2) scv2 = sc_load(2);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < KBW; ++j) {
      const int kb = kb0 + j;
      wv[j] = load_nt_u4(gp + min(4 * kb + lq, Kp - 1) * twoI);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int m = 0; m < DGW; ++m) {
      const int col = min((wave * DGW + m) * 64 + tcol, a.H - 4);
      dw[m] = load_nt_u4(dp + col);
      sdw[m] = *(const uint2*)(dsp + col);
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  load_weights();
  const uint32_t mq = q4_magic();
  const uint4 zero4 = make_uint4(0u, 0u, 0u, 0u);
  const uint4 bneg = make_uint4(kQ4BiasPair, kQ4BiasPair, kQ4BiasPair, kQ4BiasPair);
  const f32x4_t zf = {0.f, 0.f, 0.f, 0.f};

  for (int c0 = 0; c0 < nmatch; c0 += kChunkRows) {
    if (c0 > 0) load_weights();  // more than 16 slots: stream the weights again
    bool sc_staged = false;
    const int nc = min(kChunkRows, nmatch - c0);
    // A rows: row lr is slot list[c0 + lr]
    const int my_slot = lr < nc ? list[c0 + lr] : 0;
    const uint4* xrow = s_x + (size_t)(my_slot / a.top_k) * KPM;
    const bool a_ok = lr < nc;

    // ---- gate/up over this wave's k blocks
    f32x4_t D[4] = {zf, zf, zf, zf};
    f32x4_t Db = zf;
    float y[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i) y[i][0] = y[i][1] = y[i][2] = y[i][3] = 0.f;
    int next_end = (kb0 / KPG + 1) * KPG;  // first k block of the next scale group
#pragma unroll
    for (int j = 0; j < KBW; ++j) {
      const int kb = kb0 + j;
      const uint4 A = a_ok ? xrow[4 * kb + lq] : zero4;
      const uint4 w = opaque(wv[j]);
      D[0] = mfma_bf16(A, q4_operand(w.x, mq), D[0]);
      D[1] = mfma_bf16(A, q4_operand(w.y, mq), D[1]);
      D[2] = mfma_bf16(A, q4_operand(w.z, mq), D[2]);
      D[3] = mfma_bf16(A, q4_operand(w.w, mq), D[3]);
      Db = mfma_bf16(A, bneg, Db);
      if (kb + 1 == next_end || j == KBW - 1) {  // a scale group ends here
        if (!sc_staged) {  // first group end of the wave: its scale loads (issued first) are in
          if (lane < GW * 8) w_sc[lane] = scv0;  // (the wave's slice holds GW groups)
          if constexpr (SCT > 1) {
            if (lane + kWave < GW * 8) w_sc[lane + kWave] = scv1;
          }
          if constexpr (SCT > 2) {
            if (lane + 2 * kWave < GW * 8) w_sc[lane + 2 * kWave] = scv2;
          }
          sc_staged = true;
        }
        const uint2 s2 = ((const uint2*)(w_sc + (kb / KPG - wg0) * 8))[lr];  // task columns 4lr..4lr+3
        const float sc[4] = {bf16lo(s2.x), bf16hi(s2.x), bf16lo(s2.y), bf16hi(s2.y)};
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) y[i][jj] += sc[i] * (D[i][jj] + Db[jj]);
#pragma unroll
        for (int i = 0; i < 4; ++i) D[i] = zf;
        Db = zf;
        next_end += KPG;
      }
    }
    // per-wave partials: row 4lq+jj, task columns 4lr..4lr+3
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const int row = 4 * lq + jj;
      if (row < nc) s_red[(wave * kChunkRows + row) * 16 + lr] = make_float4(y[0][jj], y[1][jj], y[2][jj], y[3][jj]);
    }
    __syncthreads();

    // ---- activation: row n, intermediate column c*32 + ci
    if (tid < nc * 32) {
      const int n = tid >> 5, ci = tid & 31;
      float g = 0.f, up = 0.f;
#pragma unroll
      for (int w2 = 0; w2 < W; ++w2) {
        const float* rg = (const float*)(s_red + (w2 * kChunkRows + n) * 16);
        g += rg[ci];
        up += rg[32 + ci];
      }
      const float av = (c * 32 + ci < Iv) ? round_to_bf16(gelu_tanh(g) * up) : 0.f;
      ((uint16_t*)s_act)[(n * 4 + (ci >> 3)) * 8 + mfma_k_pos(ci & 7)] = f32_to_bf16(av);
    }
    __syncthreads();

    // ---- down over this wave's 64-column groups
    const uint4 Ad = a_ok ? s_act[lr * 4 + lq] : zero4;
    const f32x4_t Dbd = mfma_bf16(Ad, bneg, zf);
    int slot_r[4];
    float ws_r[4];
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const int row = 4 * lq + jj;
      slot_r[jj] = row < nc ? list[c0 + row] : -1;
      ws_r[jj] = row < nc ? P.slot_w[slot_r[jj]] : 0.f;
    }
    const __amdgpu_buffer_rsrc_t part = buffer_rsrc(a.part, a.part_bytes);
#pragma unroll
    for (int m = 0; m < DGW; ++m) {
      const int gc = wave * DGW + m;
      if (gc >= HG) break;
      const uint4 w = opaque(dw[m]);
      const f32x4_t D0 = mfma_bf16(Ad, q4_operand(w.x, mq), zf);
      const f32x4_t D1 = mfma_bf16(Ad, q4_operand(w.y, mq), zf);
      const f32x4_t D2 = mfma_bf16(Ad, q4_operand(w.z, mq), zf);
      const f32x4_t D3 = mfma_bf16(Ad, q4_operand(w.w, mq), zf);
      const uint2 s2 = opaque(sdw[m]);
      const float sc[4] = {bf16lo(s2.x), bf16hi(s2.x), bf16lo(s2.y), bf16hi(s2.y)};
      const int col = gc * 64 + tcol;
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        if (slot_r[jj] >= 0 && col < a.H) {
          const float wgt = ws_r[jj];
          const uint32_t off = (uint32_t)(((slot_r[jj] * a.Tg + c) * a.H + col) * 4);
          st_coherent_f4(part, off, make_float4(sc[0] * (D0[jj] + Dbd[jj]) * wgt, sc[1] * (D1[jj] + Dbd[jj]) * wgt,
                                                sc[2] * (D2[jj] + Dbd[jj]) * wgt, sc[3] * (D3[jj] + Dbd[jj]) * wgt));
        }
      }
    }
    __syncthreads();  // s_red / s_act reused by the next chunk or task
  }
}

template <int KBW, int DGW>
__global__ __launch_bounds__(kMfmaThreads) void fused_moe_mfma_kernel(Args a) {
  constexpr int T = kMfmaThreads;
  constexpr int KPM = MfmaLds<KBW, DGW>::KPM;
  constexpr int XPT = (kResidentTokens * KPM + T - 1) / T;
  __shared__ Prologue P;
  __shared__ float4 s_scratch[T];
  __shared__ uint4 s_x[kResidentTokens * KPM];
  __shared__ float4 s_red[kMfmaWaves * kChunkRows * 16];
  __shared__ uint4 s_act[kChunkRows * 4];
  __shared__ uint4 s_sc[kMfmaWaves * MfmaLds<KBW, DGW>::GW * 8];
  const int tid = threadIdx.x;
  // The launch's tokens' activations, loaded before routing so that their
  // latency overlaps the router logits' (x does not depend on the routing).
  const int Kp = a.H >> 3, Kv = min(Kp, a.Ggu * (a.gs >> 3));
  uint4 xr[XPT];
#pragma unroll
  for (int i = 0; i < XPT; ++i) {
    const int id = tid + i * T, n = id / KPM, r = id - n * KPM;
    const bool v = n < a.M && r < Kv;
    xr[i] = v ? *(const uint4*)(a.x + (size_t)n * a.H + 8 * r) : make_uint4(0u, 0u, 0u, 0u);
  }
  // barrier generation of this launch (read before this workgroup can arrive)
  const int my_gen = tid == 0 ? load_relaxed(a.ctr) : 0;
  prologue<T>(a, P);
#pragma unroll
  for (int i = 0; i < XPT; ++i) {
    const int id = tid + i * T;
    if (id < a.M * KPM) s_x[id] = mfma_k_order(xr[i]);
  }
  __syncthreads();
  const int ntask = P.n_unique * a.Tg;
  for (int t = blockIdx.x; t < ntask; t += gridDim.x)
    run_task_mfma<KBW, DGW>(a, P, t / a.Tg, t % a.Tg, s_x, s_red, s_act, s_sc);
  finish_layer<T>(a, P, my_gen, s_scratch);
}

__global__ __launch_bounds__(256) void moe_align_kernel(Args a, int32_t* uniq, int32_t* nuniq,
                                                         int32_t* s2u, int32_t* offsets,
                                                         int32_t* slots) {
  __shared__ Prologue P;
  prologue<256>(a, P);
  const int tid = threadIdx.x;
  const int U = P.n_unique;
  if (tid < U) uniq[tid] = P.uexp[tid];
  if (tid == 0) *nuniq = U;
  if (tid < a.S) s2u[tid] = P.slot_u[tid];
  // offsets[u + 1] = slots of unique experts 0..u (every thread one u, in parallel)
  if (tid == 0) offsets[0] = 0;
  for (int u = tid; u < U; u += 256) {
    int run = 0;
    for (int s = 0; s < a.S; ++s) {
      const int su = P.slot_u[s];
      run += (su >= 0 && su <= u);
    }
    offsets[u + 1] = run;
  }
  if (tid < a.S && P.slot_u[tid] >= 0) {
    const int u = P.slot_u[tid];
    int before = 0, pos = 0;
    for (int s = 0; s < a.S; ++s) {
      const int su = P.slot_u[s];
      before += (su >= 0 && su < u);
      pos += (s < tid && su == u);
    }
    slots[before + pos] = tid;
  }
}

// Router only (gi_moe_route_topk_softmax): one wave per token.
__global__ __launch_bounds__(256) void route_kernel(Args a, int32_t* out_idx, void* out_w,
                                                    int w_dtype) {
  __shared__ int r_idx[4][64];
  __shared__ float r_w[4][64];
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x >> 6;
  const int t = blockIdx.x * 4 + wave;
  if (t >= a.M) return;
  route_token_any(a, t, lane, r_idx[wave], r_w[wave]);
  if (lane < a.top_k) {
    const int s = t * a.top_k + lane;
    out_idx[s] = r_idx[wave][lane];
    const float p = r_w[wave][lane];
    if (w_dtype == GI_DTYPE_BF16) ((uint16_t*)out_w)[s] = f32_to_bf16(p);
    else if (w_dtype == GI_DTYPE_FP16) ((_Float16*)out_w)[s] = (_Float16)p;
    else ((float*)out_w)[s] = p;
  }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
constexpr size_t kAlign = 256;
inline size_t round_up(size_t v, size_t a = kAlign) { return (v + a - 1) / a * a; }

// status word | decode-kernel state (epochs, exchange buffers; fixed offset,
// kept between calls) | barrier counters | partial slabs
struct WsLayout {
  size_t status, state, ctr, part, total;
};

// Intermediate columns per task.  32 columns (512-thread workgroups) beat 16
// for a single token as well: half the partial slabs, half the per-task
// prologue, and 176 tasks at U=8 still cover most of the chip.
constexpr int kTaskCols = 32;
int tiles_per_expert(int I, int cg) { return (I + cg - 1) / cg; }

WsLayout ws_layout(int S, int H, int I, int cg) {
  WsLayout L;
  L.status = 0;
  L.state = kAlign;
  L.ctr = L.state + round_up(moe_decode_state_bytes());
  L.part = L.ctr + round_up((size_t)kCtrSlots * kCtrStride * sizeof(int));
  L.total = round_up(L.part + (size_t)S * tiles_per_expert(I, cg) * H * sizeof(float));
  return L;
}

// Start of the prefill buffers: past the status word, the decode state and
// the barrier counters (the partial slabs are scratch of one launch).
size_t prefill_base(int H, int I) { return ws_layout(1, H, I, kTaskCols).part; }

struct OccEntry {
  int device;
  const void* fn;
  size_t dyn;
  int blocks;
};
std::mutex g_occ_mu;
OccEntry g_occ[64];
int g_occ_n = 0;

int blocks_per_cu(const void* fn, int threads, size_t dyn, int* out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  {
    std::lock_guard<std::mutex> lk(g_occ_mu);
    for (int i = 0; i < g_occ_n; ++i)
      if (g_occ[i].device == dev && g_occ[i].fn == fn && g_occ[i].dyn == dyn) {
        *out = g_occ[i].blocks;
        return GI_OK;
      }
  }
  int b = 0;
  e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&b, fn, threads, dyn);
  if (e != hipSuccess) return hip_fail(e, "hipOccupancyMaxActiveBlocksPerMultiprocessor");
  std::lock_guard<std::mutex> lk(g_occ_mu);
  if (g_occ_n < 64) g_occ[g_occ_n++] = OccEntry{dev, fn, dyn, b};
  *out = b;
  return GI_OK;
}

// Persistent grid: every workgroup resident (the grid barrier needs it), no
// more workgroups than tasks; the reduction's output quads per pass.
int launch_grid(const void* fn, int T, Args& k, int umax, int* grid_out) {
  int bpc = 0;
  int st = blocks_per_cu(fn, T, 0, &bpc);
  if (st != GI_OK) return st;
  if (bpc < 1) return fail(GI_ERR_UNSUPPORTED, "fused MoE kernel does not fit on a CU");
  const long long tasks = (long long)(umax > 0 ? umax : 1) * k.Tg;
  const long long resident = (long long)bpc * device_cu_count();
  const int grid = (int)(tasks < resident ? tasks : resident);
  const int total_quads = k.M * (k.H / 4);
  const int per = (total_quads + grid - 1) / grid;
  int qpw = 1;
  while (qpw < per && qpw < T) qpw <<= 1;
  k.qpw = qpw;
  *grid_out = grid;
  return GI_OK;
}

template <int KBW, int DGW>
int launch_mfma_variant(Args k, int umax, hipStream_t stream) {
  const void* fn = (const void*)fused_moe_mfma_kernel<KBW, DGW>;
  int grid = 0;
  const int st = launch_grid(fn, kMfmaThreads, k, umax, &grid);
  if (st != GI_OK) return st;
  hipLaunchKernelGGL((fused_moe_mfma_kernel<KBW, DGW>), dim3(grid), dim3(kMfmaThreads), 0, stream, k);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return hip_fail(e, "fused MoE launch");
  return GI_OK;
}

int launch_mfma_shape(const Args& k, int umax, hipStream_t stream) {
  // (32-k blocks per wave, 64-column down groups per wave) by hidden size
  if (k.H <= 512) return launch_mfma_variant<2, 1>(k, umax, stream);
  if (k.H <= 2816) return launch_mfma_variant<11, 6>(k, umax, stream);
  return launch_mfma_variant<16, 8>(k, umax, stream);
}

template <int CG, int NT, int JGM, int CPR>
int launch_variant(Args k, int umax, hipStream_t stream) {
  constexpr int T = 16 * CG;
  const void* fn = (const void*)fused_moe_kernel<CG, NT, JGM, CPR>;
  int bpc = 0;
  int st = blocks_per_cu(fn, T, 0, &bpc);
  if (st != GI_OK) return st;
  if (bpc < 1) return fail(GI_ERR_UNSUPPORTED, "fused MoE kernel does not fit on a CU");
  const long long tasks = (long long)(umax > 0 ? umax : 1) * k.Tg;
  const long long resident = (long long)bpc * device_cu_count();
  const int grid = (int)(tasks < resident ? tasks : resident);
  // reduction split: output quads per workgroup pass (power of two <= T)
  const int total_quads = k.M * (k.H / 4);
  const int per = (total_quads + grid - 1) / grid;
  int qpw = 1;
  while (qpw < per && qpw < T) qpw <<= 1;
  k.qpw = qpw;
  hipLaunchKernelGGL((fused_moe_kernel<CG, NT, JGM, CPR>), dim3(grid), dim3(T), 0,
                     stream, k);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return hip_fail(e, "fused MoE launch");
  return GI_OK;
}

template <int CG, int NT>
int launch_shape(const Args& k, int umax, hipStream_t stream) {
  // (row steps of 32 packed rows, 1 KB chunks per down row) by hidden size
  if (k.H <= 512) return launch_variant<CG, NT, 2, 4>(k, umax, stream);
  if (k.H <= 2816) return launch_variant<CG, NT, 11, 11>(k, umax, stream);
  return launch_variant<CG, NT, 16, 16>(k, umax, stream);
}

int check_moe_shapes(const MoeHostArgs& a) {
  if (a.M < 0 || a.H <= 0 || a.I <= 0 || a.E <= 0 || a.top_k <= 0)
    return fail(GI_ERR_INVALID_ARG, "fused MoE: M must be >= 0 and H, I, E, top_k positive");
  if (a.H % 8 || a.I % 8)
    return fail(GI_ERR_INVALID_ARG, "fused MoE: H and I must be multiples of 8 (8 codes per int32)");
  if (a.gs <= 0 || a.gs % 8)
    return fail(GI_ERR_INVALID_ARG, "fused MoE: group_size must be a positive multiple of 8");
  if (a.E > kMaxExperts) return fail(GI_ERR_UNSUPPORTED, "fused MoE: at most 1024 experts");
  if (a.top_k > kMaxSlots) return fail(GI_ERR_UNSUPPORTED, "fused MoE: top_k must be <= 256");
  if (a.Ggu <= 0 || a.Gd <= 0)
    return fail(GI_ERR_INVALID_ARG, "fused MoE: scale tensors need at least one group");
  if (a.H > 4096) return fail(GI_ERR_UNSUPPORTED, "fused MoE: H <= 4096 is supported");
  // partial slabs are addressed with 32-bit byte offsets
  if ((long long)kMaxSlots * tiles_per_expert(a.I, kTaskCols) * a.H * 4 >= (1LL << 31))
    return fail(GI_ERR_UNSUPPORTED, "fused MoE: 256 * ceil(I/32) * H * 4 must stay below 2^31 bytes");
  if (a.logits && a.top_k > 64)
    return fail(GI_ERR_UNSUPPORTED, "fused MoE: in-kernel routing supports top_k <= 64");
  if (!a.x || !a.gu_packed || !a.gu_scales || !a.d_packed || !a.d_scales || !a.out)
    return fail(GI_ERR_INVALID_ARG, "fused MoE: null tensor pointer");
  if (!a.logits && (!a.idx || !a.w))
    return fail(GI_ERR_INVALID_ARG, "fused MoE: null expert_indices / expert_weights");
  if ((((uintptr_t)a.x) | ((uintptr_t)a.gu_packed) | ((uintptr_t)a.d_packed)) % 16)
    return fail(GI_ERR_INVALID_ARG, "fused MoE: x and packed weights must be 16-byte aligned");
  if ((((uintptr_t)a.gu_scales) | ((uintptr_t)a.d_scales) | ((uintptr_t)a.out)) % 8)
    return fail(GI_ERR_INVALID_ARG, "fused MoE: scales and out must be 8-byte aligned");
  return GI_OK;
}

}  // namespace

int check_moe_args(const MoeHostArgs& h) { return check_moe_shapes(h); }

size_t moe_decode_scratch_offset() { return ws_layout(1, 8, 8, kTaskCols).state; }

int moe_rows_per_launch(int top_k) { return top_k > 0 ? kMaxSlots / top_k : 0; }

size_t moe_workspace_bytes(int rows, int top_k, int H, int I, int E) {
  (void)E;
  const int per = moe_rows_per_launch(top_k);
  int r = rows < per ? rows : per;
  if (r < 1) r = 1;
  // the largest tile count any launch of this call may use; many rows may
  // take the grouped-GEMM prefill path instead
  const WsLayout L = ws_layout(r * top_k, H, I, kTaskCols);
  if (rows < kPrefillMinRows) return L.total;
  // the prefill buffers follow the status word, the decode state and the
  // barrier counters, which later calls on the same workspace still need
  const size_t pf = prefill_base(H, I) + moe_prefill_workspace_bytes(rows, top_k, H, I, E);
  return pf > L.total ? pf : L.total;
}

// The same workspace serves every activation dtype: fp16 / fp32 calls keep
// their activations after the decode state and the barrier counters.
size_t moe_workspace_bytes_any(int rows, int top_k, int H, int I, int E) {
  const size_t b = moe_workspace_bytes(rows, top_k, H, I, E);
  const size_t g = prefill_base(H, I) + moe_generic_workspace_bytes(rows, top_k, H, I);
  return g > b ? g : b;
}

int launch_fused_moe(const MoeHostArgs& h) {
  int st = check_moe_shapes(h);
  if (st != GI_OK) return st;
  if (h.M == 0) return GI_OK;
  // Matrix-core path when every scale group is whole 32-k blocks and there is
  // more than one token (one packed word then serves every token of the
  // expert): launches of up to 8 rows, their activations resident in LDS.
  // A single token, or other group sizes, take the VALU path.
  const bool mfma = h.gs % 32 == 0 && h.M > 1;
  const int rows_vl = moe_rows_per_launch(h.top_k);
  const int rows_per = mfma ? (rows_vl < kResidentTokens ? rows_vl : kResidentTokens) : rows_vl;
  if (!h.workspace || h.workspace_bytes < moe_workspace_bytes_any(h.M, h.top_k, h.H, h.I, h.E))
    return fail(GI_ERR_WORKSPACE,
                "fused MoE: workspace missing or smaller than gi_fused_moe_workspace_bytes()");
  if (((uintptr_t)h.workspace) % kAlign)
    return fail(GI_ERR_WORKSPACE, "fused MoE: workspace must be 256-byte aligned");
  if (h.x_dtype == GI_DTYPE_FP16) {
    // one fp16 token: the one-token kernel's fp16 variant (split bf16
    // operands); more rows: the 8-row kernel's fp16 variant (fp16 products on
    // q - 8 operands), one launch per 8 rows (~30 us each at the Gemma shapes,
    // against ~120 us for the VALU kernels' launch of 64 slots)
    const int per = moe_rows_per_launch(h.top_k);
    const WsLayout L = ws_layout((h.M < per ? h.M : per) * h.top_k, h.H, h.I, kTaskCols);
    char* ws0 = (char*)h.workspace;
    if (h.M == 1 && moe_decode1_supported(h)) return launch_moe_decode1(h, ws0 + L.state, (int*)(ws0 + L.status));
    if (moe_decode_supported(h)) return launch_moe_decode(h, ws0 + L.state, (int*)(ws0 + L.status));
  }
  if (h.x_dtype != GI_DTYPE_BF16) {
    const size_t base = prefill_base(h.H, h.I);
    return launch_moe_generic(h, h.x_dtype, (char*)h.workspace + base, h.workspace_bytes - base);
  }
  if (moe_prefill_supported(h)) {
    const size_t base = prefill_base(h.H, h.I);
    const WsLayout L = ws_layout(1, h.H, h.I, kTaskCols);
    return launch_moe_prefill(h, (char*)h.workspace + base, h.workspace_bytes - base,
                              (int*)((char*)h.workspace + L.ctr) + 4 * kCtrStride);
  }
  if (moe_decode1_supported(h) || moe_decode_supported(h)) {
    // the same layout as the size query (gi_fused_moe_workspace_bytes)
    const int per = moe_rows_per_launch(h.top_k);
    const WsLayout L = ws_layout((h.M < per ? h.M : per) * h.top_k, h.H, h.I, kTaskCols);
    char* ws0 = (char*)h.workspace;
    if (h.M == 1 && moe_decode1_supported(h)) return launch_moe_decode1(h, ws0 + L.state, (int*)(ws0 + L.status));
    return launch_moe_decode(h, ws0 + L.state, (int*)(ws0 + L.status));
  }

  char* ws = (char*)h.workspace;
  Args k{};
  k.gu_packed = h.gu_packed;
  k.gu_scales = (const uint16_t*)h.gu_scales;
  k.d_packed = h.d_packed;
  k.d_scales = (const uint16_t*)h.d_scales;
  k.logits = h.logits;
  k.logits_dtype = h.logits_dtype;
  k.expert_scale = h.expert_scale;
  k.out_idx = h.out_idx;
  k.out_w = (uint16_t*)h.out_w;
  k.idx_is64 = h.idx_is64;
  k.w_dtype = h.w_dtype;
  k.H = h.H;
  k.I = h.I;
  k.E = h.E;
  k.top_k = h.top_k;
  k.gs = h.gs;
  k.Ggu = h.Ggu;
  k.Gd = h.Gd;
  k.overwrite = h.overwrite;
  k.spin_limit = h.spin_limit > 0 ? h.spin_limit : kDefaultSpin;
  k.host_flag = device_error_flag(true, h.stream);

  const size_t idx_es = h.idx_is64 ? 8 : 4;
  const size_t w_es = h.w_dtype == GI_DTYPE_FP32 ? 4 : 2;
  for (int r0 = 0; r0 < h.M; r0 += rows_per) {
    const int rows = (h.M - r0) < rows_per ? (h.M - r0) : rows_per;
    const int cg = kTaskCols;
    const WsLayout L = ws_layout(rows * h.top_k, h.H, h.I, cg);
    k.status = (int*)(ws + L.status);
    k.ctr = (int*)(ws + L.ctr);
    k.part = (float*)(ws + L.part);
    k.part_bytes = (uint32_t)(L.total - L.part);
    k.M = rows;
    k.S = rows * h.top_k;
    k.Tg = tiles_per_expert(h.I, cg);
    k.x = (const uint16_t*)h.x + (size_t)r0 * h.H;
    k.out = (uint16_t*)h.out + (size_t)r0 * h.H;
    k.idx = h.idx ? (const char*)h.idx + (size_t)r0 * h.top_k * idx_es : nullptr;
    k.w = h.w ? (const char*)h.w + (size_t)r0 * h.top_k * w_es : nullptr;
    if (h.logits) k.logits = (const char*)h.logits + (size_t)r0 * h.E * (h.logits_dtype == GI_DTYPE_FP32 ? 4 : 2);
    k.out_idx = h.out_idx ? h.out_idx + (size_t)r0 * h.top_k : nullptr;
    k.out_w = h.out_w ? (uint16_t*)h.out_w + (size_t)r0 * h.top_k : nullptr;
    const int umax = k.S < h.E ? k.S : h.E;
    if (mfma) st = launch_mfma_shape(k, umax, h.stream);
    else st = rows == 1 ? launch_shape<kTaskCols, 1>(k, umax, h.stream) : launch_shape<kTaskCols, 2>(k, umax, h.stream);
    if (st != GI_OK) return st;
  }
  return GI_OK;
}

int launch_moe_align(const void* idx, int is64, int M, int top_k, int E, int32_t* uniq,
                     int32_t* nuniq, int32_t* s2u, int32_t* offsets, int32_t* slots,
                     hipStream_t stream) {
  if (M <= 0 || top_k <= 0 || E <= 0)
    return fail(GI_ERR_INVALID_ARG, "moe_align: M, top_k, E must be positive");
  if ((long long)M * top_k > kMaxSlots) return fail(GI_ERR_UNSUPPORTED, "moe_align: M*top_k must be <= 256");
  if (E > kMaxExperts) return fail(GI_ERR_UNSUPPORTED, "moe_align: at most 1024 experts");
  if (!idx || !uniq || !nuniq || !s2u || !offsets || !slots)
    return fail(GI_ERR_INVALID_ARG, "moe_align: null pointer");
  Args k{};
  k.idx = idx;
  k.idx_is64 = is64;
  k.M = M;
  k.top_k = top_k;
  k.E = E;
  k.S = M * top_k;
  hipLaunchKernelGGL(moe_align_kernel, dim3(1), dim3(256), 0, stream, k, uniq, nuniq, s2u, offsets,
                     slots);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return hip_fail(e, "moe_align launch");
  return GI_OK;
}

int launch_route(const void* logits, int logits_dtype, const float* expert_scale, int M, int E,
                 int top_k, int32_t* out_idx, void* out_w, int w_dtype, hipStream_t stream) {
  if (M < 0 || E <= 0 || top_k <= 0) return fail(GI_ERR_INVALID_ARG, "route: bad M, E or top_k");
  if (E > kMaxExperts) return fail(GI_ERR_UNSUPPORTED, "route: at most 1024 experts");
  if (top_k > E || top_k > 64) return fail(GI_ERR_UNSUPPORTED, "route: top_k must be <= min(E, 64)");
  if (logits_dtype != GI_DTYPE_BF16 && logits_dtype != GI_DTYPE_FP32)
    return fail(GI_ERR_UNSUPPORTED, "route: logits must be bf16 or fp32");
  if (w_dtype != GI_DTYPE_BF16 && w_dtype != GI_DTYPE_FP16 && w_dtype != GI_DTYPE_FP32)
    return fail(GI_ERR_UNSUPPORTED, "route: weights must be bf16, fp16 or fp32");
  if (!logits || !out_idx || !out_w) return fail(GI_ERR_INVALID_ARG, "route: null pointer");
  if (M == 0) return GI_OK;
  Args k{};
  k.logits = logits;
  k.logits_dtype = logits_dtype;
  k.expert_scale = expert_scale;
  k.M = M;
  k.E = E;
  k.top_k = top_k;
  hipLaunchKernelGGL(route_kernel, dim3((M + 3) / 4), dim3(256), 0, stream, k, out_idx, out_w,
                     w_dtype);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return hip_fail(e, "route launch");
  return GI_OK;
}

int read_workspace_status(void* workspace, int32_t* host_status, hipStream_t stream) {
  if (!workspace || !host_status) return fail(GI_ERR_INVALID_ARG, "workspace_status: null pointer");
  hipError_t e = hipMemcpyAsync(host_status, workspace, sizeof(int32_t), hipMemcpyDeviceToHost, stream);
  if (e != hipSuccess) return hip_fail(e, "workspace_status copy");
  e = hipStreamSynchronize(stream);
  if (e != hipSuccess) return hip_fail(e, "workspace_status sync");
  e = hipMemsetAsync(workspace, 0, sizeof(int32_t), stream);
  if (e != hipSuccess) return hip_fail(e, "workspace_status clear");
  e = hipStreamSynchronize(stream);
  if (e != hipSuccess) return hip_fail(e, "workspace_status sync");
  return GI_OK;
}

}  // namespace gi
