// Token-Union W4A16 fused MoE for small token counts (decode M=1, verify M<=8,
// and any launch of up to 256 slots), on gfx950.
//
// Reference behaviour restated (paths relative to the GemmaInfer repo):
//   routing        gemmainfer/models/gemma.py:77-80
//   dedup          csrc/marlin.cu:285-335 (gate_up) / :453-505 (down)
//   gate_up + GELU csrc/marlin.cu:337-426
//   down + combine csrc/marlin.cu:507-586
//
// One launch does the whole layer.  Every workgroup first recomputes the
// routing (layer mode) and the Token-Union alignment in LDS -- both are tiny
// and recomputing them is cheaper than a dependent launch or an extra
// inter-workgroup hop.  The grid is persistent (no larger than what the GPU
// keeps resident) and walks a task list ordered
//
//   [gate_up(u, c) for u < U, c < Tg] ++ [down(u, d) for u < U, d < Td]
//
//   gate_up(u, c): 16 gate + 16 up columns of unique expert u over the full
//     hidden dimension, for every token routed to u; gelu_tanh(gate)*up is
//     rounded to bf16 (as the reference stores it) into act[slot, :].  Then
//     one release-increment of gu_ctr[u].
//   down(u, d): 64 output columns of expert u over the full intermediate
//     dimension.  Its packed weights and scales are loaded into registers
//     BEFORE it waits for gu_ctr[u] == Tg, so the wait overlaps the HBM
//     stream.  It writes w[slot]*y into the fp32 buffer ypart[slot, cols] and
//     increments col_ctr[d]; the U-th arrival (last arriver) adds, for every
//     token, its slots' partials in slot order to out -- a fixed-order fp32
//     combine with one bf16 rounding, no float atomics.
//
// Deadlock freedom: gate_up tasks never wait and precede every down task in
// each workgroup's task sequence; all workgroups are resident, so the
// lowest-numbered unfinished task can always make progress.  Waits are still
// bounded (spin_limit) and report GI_DEVICE_SPIN_TIMEOUT instead of hanging.
// Counters are reset by their last user, so the workspace is left zeroed.

#include <limits.h>

#include <mutex>

#include "../../include/gemmainfer_amd.h"
#include "gi_common.h"
#include "gi_internal.h"

namespace gi {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;
constexpr int kMaxSlots = 256;
constexpr int kMaxExperts = 1024;
constexpr int kGuCols = 16;            // pair columns per gate_up task
constexpr int kGuRowsPerStep = 64;     // packed rows per step: 4 waves x 16 lane rows
constexpr int kDnCols = 64;            // output columns per down task
constexpr int kDnRowsPerStep = 16;     // packed rows per step: 4 waves x 4 lane rows
constexpr int kDefaultSpin = 1 << 22;

struct MoeArgs {
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
  uint16_t* act;    // [S, I] bf16
  float* ypart;     // [S, H] fp32
  int* gu_ctr;      // [min(S, E)]
  int* col_ctr;     // [Td]
  int* status;      // [1]
  int idx_is64, w_dtype, logits_dtype;
  int M, H, I, E, top_k, gs, Ggu, Gd;
  int Tg, Td, S, stage_stride;
  int overwrite;
  int spin_limit;
};

// ---------------------------------------------------------------------------
// Shared state of the prologue (routing + alignment), static LDS.
// ---------------------------------------------------------------------------
struct Prologue {
  int first_slot[kMaxExperts];
  int slot_u[kMaxSlots];      // unique index of each slot, -1 if skipped
  int slot_e[kMaxSlots];      // expert id of each slot, -1 if skipped
  float slot_w[kMaxSlots];    // routing weight of each slot (bf16-rounded)
  int rank_of_slot[kMaxSlots];
  int uexp[kMaxSlots];        // expert of each unique index
  int list[kMaxSlots];        // slots of the current task's expert, ascending
  int route_idx[kWaves][64];
  float route_w[kWaves][64];
  int wave_cnt[kWaves];
  int n_unique;
  int n_list;
  int flag;
};

__device__ __forceinline__ uint32_t orderable_key(float f) {
  uint32_t u = __float_as_uint(f);
  if (f != f) return 0xffffffffu;  // NaN ranks above every number
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float key_value(uint32_t k) {
  if (k == 0xffffffffu) return __uint_as_float(0x7fc00000u);
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

// Top-k + softmax of one token's logits by one wave (gemma.py:77-80).  Lane l
// holds experts l, l+64, ...; each of top_k rounds takes the wave maximum of
// (value, -index) and retires it.  Lane r < top_k receives the r-th expert
// and its softmax weight times expert_scale (fp32).  Every real value has a
// non-zero orderable key, so key 0 marks a retired entry.
__device__ __forceinline__ void route_one_token(const void* logits, int dt, const float* es,
                                                int E, int top_k, int t, int lane,
                                                int* idx_out, float* w_out) {
  constexpr int kPerLane = kMaxExperts / kWave;
  uint32_t keys[kPerLane];
  const size_t base = (size_t)t * E;
#pragma unroll
  for (int v = 0; v < kPerLane; ++v) {
    const int e = lane + v * kWave;
    uint32_t k = 0;
    if (e < E) {
      const float f = dt == GI_DTYPE_BF16 ? bf16_to_f32(((const uint16_t*)logits)[base + e])
                                          : ((const float*)logits)[base + e];
      k = orderable_key(f);
    }
    keys[v] = k;
  }
  int my_idx = 0;
  float my_val = 0.f;
  for (int r = 0; r < top_k; ++r) {
    unsigned long long best = 0ull;
#pragma unroll
    for (int v = 0; v < kPerLane; ++v) {
      const int e = lane + v * kWave;
      const unsigned long long kk =
          ((unsigned long long)keys[v] << 32) | (unsigned long long)(0xffffffffu - (uint32_t)e);
      if (keys[v] != 0u && kk > best) best = kk;
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
      const unsigned long long o = __shfl_xor(best, off, kWave);
      best = o > best ? o : best;
    }
    const int win = (int)(0xffffffffu - (uint32_t)(best & 0xffffffffull));
    if ((win & (kWave - 1)) == lane) {
#pragma unroll
      for (int v = 0; v < kPerLane; ++v)
        if (v == (win >> 6)) keys[v] = 0u;
    }
    if (lane == r) {
      my_idx = win;
      my_val = key_value((uint32_t)(best >> 32));
    }
  }
  const float vmax = __shfl(my_val, 0, kWave);
  const float ex = lane < top_k ? expf(my_val - vmax) : 0.f;
  float sum = ex;
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) sum += __shfl_xor(sum, off, kWave);
  if (lane < top_k) {
    float p = ex / sum;
    if (es) p *= es[my_idx];
    idx_out[lane] = my_idx;
    w_out[lane] = p;
  }
}

// Routing (layer mode) or id/weight load, then the Token-Union alignment:
// first-occurrence rank of every distinct valid id in slot order
// (marlin.cu:298-319) and each slot's unique index.  All threads.
__device__ void prologue(const MoeArgs& a, Prologue& P) {
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid >> 6;
  const int S = a.S;
  if (a.logits) {
    for (int t = wave; t < a.M; t += kWaves) {
      route_one_token(a.logits, a.logits_dtype, a.expert_scale, a.E, a.top_k, t, lane,
                      P.route_idx[wave], P.route_w[wave]);
      if (lane < a.top_k) {
        const int s = t * a.top_k + lane;
        const int e = P.route_idx[wave][lane];
        const float wr = round_to_bf16(P.route_w[wave][lane]);
        P.slot_e[s] = e;
        P.slot_w[s] = wr;
        if (blockIdx.x == 0) {
          if (a.out_idx) a.out_idx[s] = e;
          if (a.out_w) a.out_w[s] = f32_to_bf16(wr);
        }
      }
    }
  } else if (tid < S) {
    const int e = load_expert_id(a.idx, a.idx_is64, tid);
    P.slot_e[tid] = (e >= 0 && e < a.E) ? e : -1;
    P.slot_w[tid] = a.w ? load_weight_as_bf16(a.w, a.w_dtype, tid) : 0.f;
  }
  for (int i = tid; i < a.E; i += kThreads) P.first_slot[i] = INT_MAX;
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
  for (int w = 0; w < kWaves; ++w) {
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
__device__ void gather_list(const MoeArgs& a, Prologue& P, int u) {
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid >> 6;
  const bool mine = tid < a.S && P.slot_u[tid] == u;
  const unsigned long long bal = __ballot(mine);
  const int below = __popcll(bal & ((1ull << lane) - 1ull));
  __syncthreads();  // earlier readers of list / wave_cnt are done
  if (lane == 0) P.wave_cnt[wave] = __popcll(bal);
  __syncthreads();
  int base = 0, total = 0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    const int c = P.wave_cnt[w];
    base += (w < wave) ? c : 0;
    total += c;
  }
  if (mine) P.list[base + below] = tid;
  if (tid == 0) P.n_list = total;
  __syncthreads();
}

// Stage packed rows [0, nrows) of chunk entries n < nch into LDS as
// pair-permuted bf16 plus the -136*sum bias.  Entry n reads source row
// P.list[c0 + n] / div of `src` (row length ld elements).
__device__ __forceinline__ void stage_rows(const uint16_t* __restrict__ src, int ld,
                                           const Prologue& P, int c0, int div, int nch,
                                           int nrows, int stride, uint4* xs, float* xb) {
  for (int i = threadIdx.x; i < nch * nrows; i += kThreads) {
    const int n = i / nrows, r = i - n * nrows;
    const int row = P.list[c0 + n] / div;
    const uint4 d = *(const uint4*)(src + (size_t)row * ld + 8 * r);
    xs[n * stride + r] = pair_permute(d);
    xb[n * stride + r] = neg_bias_136(d);
  }
}

// ---------------------------------------------------------------------------
// gate_up task
// ---------------------------------------------------------------------------
template <int NT, int JM>
__device__ void gate_up_task(const MoeArgs& a, Prologue& P, int u, int c, uint4* xs, float* xb,
                             float* red) {
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid >> 6;
  const int rsub = lane >> 2, colq = lane & 3;
  const int Kp = a.H >> 3, twoI = 2 * a.I, rpg = a.gs >> 3, ss = a.stage_stride;
  const int e = P.uexp[u];
  const int col = c * kGuCols + colq * 4;
  const bool col_ok = col < a.I;
  const int32_t* wp = a.gu_packed + (size_t)e * Kp * twoI;
  const uint16_t* sp = a.gu_scales + (size_t)e * a.Ggu * twoI;

  // Prefetch every packed word and scale this lane needs (12 x 16 B at H=2816).
  uint4 wg[JM], wu[JM];
  uint2 sg[JM], su[JM];
  bool ok[JM];
#pragma unroll
  for (int j = 0; j < JM; ++j) {
    const int r = j * kGuRowsPerStep + wave * 16 + rsub;
    const int g = r / rpg;
    ok[j] = col_ok && r < Kp && g < a.Ggu;
    if (ok[j]) {
      const int32_t* rowp = wp + (size_t)r * twoI + col;
      wg[j] = load_nt_u4(rowp);
      wu[j] = load_nt_u4(rowp + a.I);
      const uint16_t* srow = sp + (size_t)g * twoI + col;
      sg[j] = *(const uint2*)srow;
      su[j] = *(const uint2*)(srow + a.I);
    }
  }
  gather_list(a, P, u);
  const int nmatch = P.n_list;
  for (int c0 = 0; c0 < nmatch; c0 += NT) {
    const int nch = min(NT, nmatch - c0);
    stage_rows(a.x, a.H, P, c0, a.top_k, nch, Kp, ss, xs, xb);
    __syncthreads();
    float ag[4][NT], au[4][NT];
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int n = 0; n < NT; ++n) ag[q][n] = au[q][n] = 0.f;
#pragma unroll
    for (int j = 0; j < JM; ++j) {
      if (!ok[j]) continue;
      const int r = j * kGuRowsPerStep + wave * 16 + rsub;
      const float s_g[4] = {bf16lo(sg[j].x), bf16hi(sg[j].x), bf16lo(sg[j].y), bf16hi(sg[j].y)};
      const float s_u[4] = {bf16lo(su[j].x), bf16hi(su[j].x), bf16lo(su[j].y), bf16hi(su[j].y)};
      const uint32_t gw[4] = {wg[j].x, wg[j].y, wg[j].z, wg[j].w};
      const uint32_t uw[4] = {wu[j].x, wu[j].y, wu[j].z, wu[j].w};
#pragma unroll
      for (int n = 0; n < NT; ++n) {
        if (n < nch) {
          const uint4 xp = xs[n * ss + r];
          const float b = xb[n * ss + r];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            ag[q][n] += s_g[q] * dot8_q4(gw[q], xp, b);
            au[q][n] += s_u[q] * dot8_q4(uw[q], xp, b);
          }
        }
      }
    }
    // Reduce over the 16 lane rows of each wave (lane bits 2..5), then waves.
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int n = 0; n < NT; ++n) {
        ag[q][n] = reduce_across_groups<4>(ag[q][n]);
        au[q][n] = reduce_across_groups<4>(au[q][n]);
      }
    // red layout: [wave][n][gate|up][kGuCols]
    if (rsub == 0) {
#pragma unroll
      for (int n = 0; n < NT; ++n)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          red[((wave * NT + n) * 2 + 0) * kGuCols + colq * 4 + q] = ag[q][n];
          red[((wave * NT + n) * 2 + 1) * kGuCols + colq * 4 + q] = au[q][n];
        }
    }
    __syncthreads();
    if (tid < nch * kGuCols) {
      const int n = tid / kGuCols, i = tid - n * kGuCols;
      const int ci = c * kGuCols + i;
      if (ci < a.I) {
        float g = 0.f, up = 0.f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
          g += red[((w * NT + n) * 2 + 0) * kGuCols + i];
          up += red[((w * NT + n) * 2 + 1) * kGuCols + i];
        }
        const int slot = P.list[c0 + n];
        a.act[(size_t)slot * a.I + ci] = f32_to_bf16(gelu_tanh(g) * up);
      }
    }
    __syncthreads();
  }
  if (tid == 0) {
    // Normally a gate_up increment is never the last of the Tg + Td; it can be
    // only after a down task gave up waiting, and then it resets the counter.
    const int old = atomic_add_release(&a.gu_ctr[u], 1);
    if (old == a.Tg + a.Td - 1) store_relaxed(&a.gu_ctr[u], 0);
  }
}

// ---------------------------------------------------------------------------
// down task (+ last-arriver combine)
// ---------------------------------------------------------------------------
template <int NT, int JM>
__device__ void down_task(const MoeArgs& a, Prologue& P, int u, int d, uint4* xs, float* xb,
                          float* red) {
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid >> 6;
  const int rsub = lane >> 4, colq = lane & 15;
  const int Ip = a.I >> 3, rpg = a.gs >> 3, ss = a.stage_stride;
  const int e = P.uexp[u];
  const int col = d * kDnCols + colq * 4;
  const bool col_ok = col < a.H;
  const int32_t* wp = a.d_packed + (size_t)e * Ip * a.H;
  const uint16_t* sp = a.d_scales + (size_t)e * a.Gd * a.H;

  uint4 wd[JM];
  uint2 sd[JM];
  bool ok[JM];
#pragma unroll
  for (int j = 0; j < JM; ++j) {
    const int r = j * kDnRowsPerStep + wave * 4 + rsub;
    const int g = r / rpg;
    ok[j] = col_ok && r < Ip && g < a.Gd;
    if (ok[j]) {
      wd[j] = load_nt_u4(wp + (size_t)r * a.H + col);
      sd[j] = *(const uint2*)(sp + (size_t)g * a.H + col);
    }
  }
  gather_list(a, P, u);

  // Wait until every gate_up task of expert u has published its activations.
  if (tid == 0) {
    int spins = 0, bad = 0;
    while (load_acquire(&a.gu_ctr[u]) < a.Tg) {
      if (++spins >= a.spin_limit || load_relaxed(a.status) != 0) {
        bad = 1;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
    if (bad) atomicOr(a.status, GI_DEVICE_SPIN_TIMEOUT);
  }
  __syncthreads();

  const int nmatch = P.n_list;
  for (int c0 = 0; c0 < nmatch; c0 += NT) {
    const int nch = min(NT, nmatch - c0);
    stage_rows(a.act, a.I, P, c0, 1, nch, Ip, ss, xs, xb);
    __syncthreads();
    float acc[4][NT];
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int n = 0; n < NT; ++n) acc[q][n] = 0.f;
#pragma unroll
    for (int j = 0; j < JM; ++j) {
      if (!ok[j]) continue;
      const int r = j * kDnRowsPerStep + wave * 4 + rsub;
      const float s_d[4] = {bf16lo(sd[j].x), bf16hi(sd[j].x), bf16lo(sd[j].y), bf16hi(sd[j].y)};
      const uint32_t dw[4] = {wd[j].x, wd[j].y, wd[j].z, wd[j].w};
#pragma unroll
      for (int n = 0; n < NT; ++n) {
        if (n < nch) {
          const uint4 xp = xs[n * ss + r];
          const float b = xb[n * ss + r];
#pragma unroll
          for (int q = 0; q < 4; ++q) acc[q][n] += s_d[q] * dot8_q4(dw[q], xp, b);
        }
      }
    }
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int n = 0; n < NT; ++n) acc[q][n] = reduce_across_groups<16>(acc[q][n]);
    if (rsub == 0) {
#pragma unroll
      for (int n = 0; n < NT; ++n)
#pragma unroll
        for (int q = 0; q < 4; ++q) red[(wave * NT + n) * kDnCols + colq * 4 + q] = acc[q][n];
    }
    __syncthreads();
    for (int i = tid; i < nch * kDnCols; i += kThreads) {
      const int n = i / kDnCols, cc = i - n * kDnCols;
      const int hc = d * kDnCols + cc;
      if (hc < a.H) {
        float y = 0.f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) y += red[(w * NT + n) * kDnCols + cc];
        const int slot = P.list[c0 + n];
        a.ypart[(size_t)slot * a.H + hc] = y * P.slot_w[slot];
      }
    }
    __syncthreads();
  }

  if (tid == 0) {
    // Every down task of u has passed its wait once the counter reaches Tg+Td.
    const int old = atomicAdd(&a.gu_ctr[u], 1);
    if (old == a.Tg + a.Td - 1) store_relaxed(&a.gu_ctr[u], 0);
    const int arrived = atomic_add_acq_rel(&a.col_ctr[d], 1);
    P.flag = arrived == P.n_unique - 1;
  }
  __syncthreads();
  if (P.flag) {
    // Last arriver for column tile d: fixed-order combine into out.
    for (int i = tid; i < a.M * kDnCols; i += kThreads) {
      const int t = i / kDnCols, cc = i - t * kDnCols;
      const int hc = d * kDnCols + cc;
      if (hc < a.H) {
        uint16_t* o = a.out + (size_t)t * a.H + hc;
        float acc = a.overwrite ? 0.f : bf16_to_f32(*o);
        for (int k = 0; k < a.top_k; ++k) {
          const int s = t * a.top_k + k;
          if (P.slot_u[s] >= 0) acc += a.ypart[(size_t)s * a.H + hc];
        }
        *o = f32_to_bf16(acc);
      }
    }
    if (tid == 0) store_relaxed(&a.col_ctr[d], 0);
  }
}

template <int NT, int JM>
__global__ __launch_bounds__(kThreads) void fused_moe_kernel(MoeArgs a) {
  __shared__ Prologue P;
  __shared__ float red[kWaves * NT * 64];
  extern __shared__ uint4 dyn[];
  uint4* xs = dyn;
  float* xb = (float*)(dyn + NT * a.stage_stride);
  prologue(a, P);
  const int U = P.n_unique;
  const int n_gu = U * a.Tg;
  const int n_all = n_gu + U * a.Td;
  for (int t = blockIdx.x; t < n_all; t += gridDim.x) {
    if (t < n_gu) {
      gate_up_task<NT, JM>(a, P, t / a.Tg, t % a.Tg, xs, xb, red);
    } else {
      const int td = t - n_gu;
      down_task<NT, JM>(a, P, td / a.Td, td % a.Td, xs, xb, red);
    }
  }
}

// Export of the alignment (gi_moe_align): one workgroup.
__global__ __launch_bounds__(kThreads) void moe_align_kernel(MoeArgs a, int32_t* uniq,
                                                              int32_t* nuniq, int32_t* s2u,
                                                              int32_t* offsets, int32_t* slots) {
  __shared__ Prologue P;
  prologue(a, P);
  const int tid = threadIdx.x;
  const int U = P.n_unique;
  if (tid < U) uniq[tid] = P.uexp[tid];
  if (tid == 0) *nuniq = U;
  if (tid < a.S) s2u[tid] = P.slot_u[tid];
  if (tid == 0) {
    int run = 0;
    offsets[0] = 0;
    for (int u = 0; u < U; ++u) {
      int cnt = 0;
      for (int s = 0; s < a.S; ++s) cnt += P.slot_u[s] == u;
      run += cnt;
      offsets[u + 1] = run;
    }
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
__global__ __launch_bounds__(kThreads) void route_kernel(const void* logits, int dt,
                                                         const float* es, int M, int E,
                                                         int top_k, int32_t* out_idx,
                                                         void* out_w, int w_dtype) {
  __shared__ int r_idx[kWaves][64];
  __shared__ float r_w[kWaves][64];
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x >> 6;
  const int t = blockIdx.x * kWaves + wave;
  if (t >= M) return;
  route_one_token(logits, dt, es, E, top_k, t, lane, r_idx[wave], r_w[wave]);
  if (lane < top_k) {
    const int s = t * top_k + lane;
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
namespace {

constexpr size_t kAlign = 256;
inline size_t round_up(size_t v) { return (v + kAlign - 1) / kAlign * kAlign; }

struct WsLayout {
  size_t status, gu_ctr, col_ctr, act, ypart, total;
};

WsLayout ws_layout(int S, int H, int I, int E) {
  WsLayout L;
  const int umax = S < E ? S : E;
  const int td = (H + kDnCols - 1) / kDnCols;
  L.status = 0;
  L.gu_ctr = round_up(L.status + sizeof(int));
  L.col_ctr = round_up(L.gu_ctr + (size_t)umax * sizeof(int));
  L.act = round_up(L.col_ctr + (size_t)td * sizeof(int));
  L.ypart = round_up(L.act + (size_t)S * I * sizeof(uint16_t));
  L.total = round_up(L.ypart + (size_t)S * H * sizeof(float));
  return L;
}

// Blocks per CU of one kernel instantiation at a given dynamic LDS size,
// cached per (device, instantiation, LDS bytes).
struct OccEntry {
  int device;
  const void* fn;
  size_t dyn;
  int blocks;
};
std::mutex g_occ_mu;
OccEntry g_occ[64];
int g_occ_n = 0;

int blocks_per_cu(const void* fn, size_t dyn, int* out) {
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
  e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&b, fn, kThreads, dyn);
  if (e != hipSuccess) return hip_fail(e, "hipOccupancyMaxActiveBlocksPerMultiprocessor");
  std::lock_guard<std::mutex> lk(g_occ_mu);
  if (g_occ_n < 64) g_occ[g_occ_n++] = OccEntry{dev, fn, dyn, b};
  *out = b;
  return GI_OK;
}

template <int NT, int JM>
int launch_variant(const MoeArgs& k, int umax, hipStream_t stream) {
  const size_t dyn = (size_t)NT * k.stage_stride * (sizeof(uint4) + sizeof(float));
  const void* fn = (const void*)fused_moe_kernel<NT, JM>;
  int bpc = 0;
  int st = blocks_per_cu(fn, dyn, &bpc);
  if (st != GI_OK) return st;
  if (bpc < 1) return fail(GI_ERR_UNSUPPORTED, "fused MoE kernel does not fit on a CU");
  const long long tasks = (long long)umax * (k.Tg + k.Td);
  const long long resident = (long long)bpc * device_cu_count();
  const int grid = (int)(tasks < resident ? tasks : resident);
  if (grid <= 0) return GI_OK;
  hipLaunchKernelGGL((fused_moe_kernel<NT, JM>), dim3(grid), dim3(kThreads), dyn, stream, k);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return hip_fail(e, "fused MoE launch");
  return GI_OK;
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
  if ((a.H >> 3) > kGuRowsPerStep * 8 || (a.I >> 3) > kDnRowsPerStep * 8)
    return fail(GI_ERR_UNSUPPORTED, "fused MoE: H <= 4096 and I <= 1024 are supported");
  if (a.logits && a.top_k > 64)
    return fail(GI_ERR_UNSUPPORTED, "fused MoE: in-kernel routing supports top_k <= 64");
  if (!a.x || !a.gu_packed || !a.gu_scales || !a.d_packed || !a.d_scales || !a.out)
    return fail(GI_ERR_INVALID_ARG, "fused MoE: null tensor pointer");
  if (!a.logits && (!a.idx || !a.w))
    return fail(GI_ERR_INVALID_ARG, "fused MoE: null expert_indices / expert_weights");
  if ((((uintptr_t)a.x) | ((uintptr_t)a.gu_packed) | ((uintptr_t)a.d_packed)) % 16)
    return fail(GI_ERR_INVALID_ARG, "fused MoE: x and packed weights must be 16-byte aligned");
  if ((((uintptr_t)a.gu_scales) | ((uintptr_t)a.d_scales)) % 8)
    return fail(GI_ERR_INVALID_ARG, "fused MoE: scales must be 8-byte aligned");
  return GI_OK;
}

}  // namespace

int moe_rows_per_launch(int top_k) { return top_k > 0 ? kMaxSlots / top_k : 0; }

size_t moe_workspace_bytes(int rows, int top_k, int H, int I, int E) {
  const int per = moe_rows_per_launch(top_k);
  int r = rows < per ? rows : per;
  if (r < 1) r = 1;
  return ws_layout(r * top_k, H, I, E).total;
}

int launch_fused_moe(const MoeHostArgs& h) {
  int st = check_moe_shapes(h);
  if (st != GI_OK) return st;
  if (h.M == 0) return GI_OK;
  const int rows_per = moe_rows_per_launch(h.top_k);
  if (h.logits && h.M > rows_per)
    return fail(GI_ERR_UNSUPPORTED, "fused MoE layer: M*top_k must be <= 256");
  const int rows0 = h.M < rows_per ? h.M : rows_per;
  const WsLayout L = ws_layout(rows0 * h.top_k, h.H, h.I, h.E);
  if (!h.workspace || h.workspace_bytes < L.total)
    return fail(GI_ERR_WORKSPACE,
                "fused MoE: workspace missing or smaller than gi_fused_moe_workspace_bytes()");
  if (((uintptr_t)h.workspace) % kAlign)
    return fail(GI_ERR_WORKSPACE, "fused MoE: workspace must be 256-byte aligned");

  char* ws = (char*)h.workspace;
  MoeArgs k{};
  k.gu_packed = h.gu_packed;
  k.gu_scales = (const uint16_t*)h.gu_scales;
  k.d_packed = h.d_packed;
  k.d_scales = (const uint16_t*)h.d_scales;
  k.logits = h.logits;
  k.logits_dtype = h.logits_dtype;
  k.expert_scale = h.expert_scale;
  k.out_idx = h.out_idx;
  k.out_w = (uint16_t*)h.out_w;
  k.status = (int*)(ws + L.status);
  k.gu_ctr = (int*)(ws + L.gu_ctr);
  k.col_ctr = (int*)(ws + L.col_ctr);
  k.act = (uint16_t*)(ws + L.act);
  k.ypart = (float*)(ws + L.ypart);
  k.idx_is64 = h.idx_is64;
  k.w_dtype = h.w_dtype;
  k.H = h.H;
  k.I = h.I;
  k.E = h.E;
  k.top_k = h.top_k;
  k.gs = h.gs;
  k.Ggu = h.Ggu;
  k.Gd = h.Gd;
  k.Tg = (h.I + kGuCols - 1) / kGuCols;
  k.Td = (h.H + kDnCols - 1) / kDnCols;
  k.overwrite = h.overwrite;
  k.spin_limit = h.spin_limit > 0 ? h.spin_limit : kDefaultSpin;
  const int Kp = h.H >> 3, Ip = h.I >> 3;
  k.stage_stride = Kp > Ip ? Kp : Ip;
  const int jg = (Kp + kGuRowsPerStep - 1) / kGuRowsPerStep;
  const int jd = (Ip + kDnRowsPerStep - 1) / kDnRowsPerStep;
  const int jneed = jg > jd ? jg : jd;

  const size_t idx_es = h.idx_is64 ? 8 : 4;
  const size_t w_es = h.w_dtype == GI_DTYPE_FP32 ? 4 : 2;
  for (int r0 = 0; r0 < h.M; r0 += rows_per) {
    const int rows = (h.M - r0) < rows_per ? (h.M - r0) : rows_per;
    k.M = rows;
    k.S = rows * h.top_k;
    k.x = (const uint16_t*)h.x + (size_t)r0 * h.H;
    k.out = (uint16_t*)h.out + (size_t)r0 * h.H;
    k.idx = h.idx ? (const char*)h.idx + (size_t)r0 * h.top_k * idx_es : nullptr;
    k.w = h.w ? (const char*)h.w + (size_t)r0 * h.top_k * w_es : nullptr;
    const int umax = k.S < h.E ? k.S : h.E;
    // Tokens per pass over the prefetched weights: 1 for single-token decode.
    const bool single = rows == 1;
    if (jneed <= 2) {
      st = single ? launch_variant<1, 2>(k, umax, h.stream) : launch_variant<4, 2>(k, umax, h.stream);
    } else if (jneed <= 6) {
      st = single ? launch_variant<1, 6>(k, umax, h.stream) : launch_variant<4, 6>(k, umax, h.stream);
    } else {
      st = single ? launch_variant<1, 8>(k, umax, h.stream) : launch_variant<4, 8>(k, umax, h.stream);
    }
    if (st != GI_OK) return st;
  }
  return GI_OK;
}

int launch_moe_align(const void* idx, int is64, int M, int top_k, int E, int32_t* uniq,
                     int32_t* nuniq, int32_t* s2u, int32_t* offsets, int32_t* slots,
                     hipStream_t stream) {
  if (M <= 0 || top_k <= 0 || E <= 0) return fail(GI_ERR_INVALID_ARG, "moe_align: M, top_k, E must be positive");
  if ((long long)M * top_k > kMaxSlots) return fail(GI_ERR_UNSUPPORTED, "moe_align: M*top_k must be <= 256");
  if (E > kMaxExperts) return fail(GI_ERR_UNSUPPORTED, "moe_align: at most 1024 experts");
  if (!idx || !uniq || !nuniq || !s2u || !offsets || !slots)
    return fail(GI_ERR_INVALID_ARG, "moe_align: null pointer");
  MoeArgs k{};
  k.idx = idx;
  k.idx_is64 = is64;
  k.w = nullptr;
  k.w_dtype = GI_DTYPE_FP32;
  k.M = M;
  k.top_k = top_k;
  k.E = E;
  k.S = M * top_k;
  hipLaunchKernelGGL(moe_align_kernel, dim3(1), dim3(kThreads), 0, stream, k, uniq, nuniq, s2u,
                     offsets, slots);
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
  const int blocks = (M + kWaves - 1) / kWaves;
  hipLaunchKernelGGL(route_kernel, dim3(blocks), dim3(kThreads), 0, stream, logits, logits_dtype,
                     expert_scale, M, E, top_k, out_idx, out_w, w_dtype);
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
