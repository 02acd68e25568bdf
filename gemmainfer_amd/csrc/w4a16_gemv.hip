// W4A16 linear C[M, N] = A[M, K] @ dequant(B) on gfx950, with an optional
// fused final-logit softcap epilogue (lm_head).
//
// Reference behaviour restated (paths relative to the GemmaInfer repo):
//   csrc/marlin.cu:704-856 launch_marlin_w4a16 (split-K / tiled / coalesced
//   kernels at :13-260), csrc/pybind.cpp:46-85 (CPU semantics),
//   gemmainfer/models/gemma.py:351-357 + csrc/softcapping.cu:7-19 (epilogue).
//
// One kernel for every shape: a workgroup owns 64 output columns and one
// K-slice of the packed rows.  Lane (rsub = lane>>4, colq = lane&15) loads
// 16-byte words of 4 adjacent columns, four packed rows per wave per load, so
// one wave instruction reads 4 rows x 256 contiguous bytes.  Weights stream
// through registers in batches of 8 row-steps with the next batch's loads in
// flight while the current one is reduced.  When the grid would be too small
// to fill 256 CUs (narrow N), K is split; the slices write fp32 partials and
// the last slice to arrive for a column tile sums them in slice order (a
// deterministic reduction -- the reference zeroes C and adds bf16 atomics,
// marlin.cu:201,777).  Token rows are processed NT at a time over the same
// weight stream.

#include <mutex>

#include "../../include/gemmainfer_amd.h"
#include "gi_common.h"
#include "gi_internal.h"
#include "moe_shared.h"

namespace gi {

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;
constexpr int kCols = 64;           // output columns per workgroup
constexpr int kRowsPerStep = 16;    // packed rows per step (4 waves x 4 lane rows)
constexpr int kBatch = 8;           // steps per register batch
constexpr int kTargetWgs = 1024;    // split K until the grid reaches this many workgroups

struct GemvArgs {
  const uint16_t* A;     // [M, K] bf16
  const int32_t* B;      // [K/8, N]
  const uint16_t* S;     // [G, N] bf16
  uint16_t* C;           // [M, N] bf16
  float* part;           // [ks, M, N] fp32 (ks > 1)
  int* ctr;              // [n_tiles] (ks > 1)
  int M, K, N, gs, G;
  int ks, rows_per_split, stage_stride;
  float cap;             // > 0: C = cap * tanh(y / cap)
};

__device__ __forceinline__ float epilogue(float y, float cap) {
  return cap > 0.f ? cap * tanhf(y / cap) : y;
}

template <int NT>
__global__ __launch_bounds__(kThreads) void w4a16_kernel(GemvArgs a) {
  extern __shared__ uint4 dyn[];
  __shared__ float red[kWaves * NT * kCols];
  __shared__ int last;
  uint4* xs = dyn;
  float* xb = (float*)(dyn + NT * a.stage_stride);

  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid >> 6;
  const int rsub = lane >> 4, colq = lane & 15;
  const int tile = blockIdx.x, split = blockIdx.y;
  const int Kp = a.K >> 3, rpg = a.gs >> 3;
  const int r_begin = split * a.rows_per_split;
  const int r_end = min(Kp, r_begin + a.rows_per_split);
  const int nrows = max(0, r_end - r_begin);
  const int col = tile * kCols + colq * 4;
  const bool col_ok = col < a.N;
  const int steps = (nrows + kRowsPerStep - 1) / kRowsPerStep;
  const uint32_t mq = q4_magic();
  const int nbatch = (steps + kBatch - 1) / kBatch;

  for (int t0 = 0; t0 < a.M; t0 += NT) {
    const int nch = min(NT, a.M - t0);
    __syncthreads();  // previous chunk's LDS readers are done
    for (int i = tid; i < nch * nrows; i += kThreads) {
      const int n = i / nrows, r = i - n * nrows;
      const uint4 d = *(const uint4*)(a.A + (size_t)(t0 + n) * a.K + 8 * (r_begin + r));
      xs[n * a.stage_stride + r] = pair_permute(d);
      xb[n * a.stage_stride + r] = q4_bias(d);
    }
    __syncthreads();

    float acc[4][NT];
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int n = 0; n < NT; ++n) acc[q][n] = 0.f;

    uint4 wcur[kBatch];
    uint2 scur[kBatch];
    auto load_batch = [&](int b, uint4* w, uint2* s) {
#pragma unroll
      for (int j = 0; j < kBatch; ++j) {
        const int rl = (b * kBatch + j) * kRowsPerStep + wave * 4 + rsub;  // local row
        const int r = r_begin + rl;
        const int g = r / rpg;
        if (col_ok && rl < nrows && g < a.G) {
          w[j] = load_nt_u4(a.B + (size_t)r * a.N + col);
          s[j] = *(const uint2*)(a.S + (size_t)g * a.N + col);
        } else {
          w[j] = make_uint4(0x88888888u, 0x88888888u, 0x88888888u, 0x88888888u);
          s[j] = make_uint2(0u, 0u);
        }
      }
    };
    if (nbatch > 0) load_batch(0, wcur, scur);
    for (int b = 0; b < nbatch; ++b) {
      uint4 wnxt[kBatch];
      uint2 snxt[kBatch];
      if (b + 1 < nbatch) load_batch(b + 1, wnxt, snxt);
#pragma unroll
      for (int j = 0; j < kBatch; ++j) {
        const int rl = (b * kBatch + j) * kRowsPerStep + wave * 4 + rsub;
        if (rl < nrows) {
          const float sv[4] = {bf16lo(scur[j].x), bf16hi(scur[j].x), bf16lo(scur[j].y),
                               bf16hi(scur[j].y)};
          const uint32_t wv[4] = {wcur[j].x, wcur[j].y, wcur[j].z, wcur[j].w};
#pragma unroll
          for (int n = 0; n < NT; ++n) {
            if (n < nch) {
              const uint4 xp = xs[n * a.stage_stride + rl];
              const float bias = xb[n * a.stage_stride + rl];
#pragma unroll
              for (int q = 0; q < 4; ++q) acc[q][n] += sv[q] * dot8_q4(wv[q], xp, bias, mq);
            }
          }
        }
      }
      if (b + 1 < nbatch) {
#pragma unroll
        for (int j = 0; j < kBatch; ++j) {
          wcur[j] = wnxt[j];
          scur[j] = snxt[j];
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
        for (int q = 0; q < 4; ++q) red[(wave * NT + n) * kCols + colq * 4 + q] = acc[q][n];
    }
    __syncthreads();
    for (int i = tid; i < nch * kCols; i += kThreads) {
      const int n = i / kCols, cc = i - n * kCols;
      const int oc = tile * kCols + cc;
      if (oc < a.N) {
        float y = 0.f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) y += red[(w * NT + n) * kCols + cc];
        const size_t o = (size_t)(t0 + n) * a.N + oc;
        if (a.ks == 1) a.C[o] = f32_to_bf16(epilogue(y, a.cap));
        else st_coherent_f32(a.part + (size_t)split * a.M * a.N + o, y);
      }
    }
  }
  if (a.ks == 1) return;

  // Last K-slice to arrive for this column tile reduces the partials in order
  // (partials travel through sc1 stores/loads, see gi_common.h).
  wait_vmem();
  __syncthreads();
  if (tid == 0) last = atomic_add_relaxed(&a.ctr[tile], 1) == a.ks - 1;
  __syncthreads();
  if (!last) return;
  for (int i = tid; i < a.M * kCols; i += kThreads) {
    const int t = i / kCols, cc = i - t * kCols;
    const int oc = tile * kCols + cc;
    if (oc < a.N) {
      const size_t o = (size_t)t * a.N + oc;
      float y = 0.f;
      for (int s = 0; s < a.ks; ++s) y += ld_coherent_f32(a.part + (size_t)s * a.M * a.N + o);
      a.C[o] = f32_to_bf16(epilogue(y, a.cap));
    }
  }
  if (tid == 0) store_relaxed(&a.ctr[tile], 0);
}

// ---------------------------------------------------------------------------
// Decode-shape path (M <= 8): the same tiling (64 columns x one K slice per
// workgroup, 4 packed rows x 256 B per wave instruction) with every global
// load of the workgroup issued before any is used -- the slice's token rows
// (staged as soon as they land), then S steps of weight words and their
// scales, which the products take as they land -- so a launch is one memory
// round trip, the products and the split-K reduction.  Masked loads (rows
// past the slice or past the last scale group, columns past N, tokens past
// M) read zeros through the buffer range check; a zero scale then zeroes the
// word's contribution, so no lane branches.  The plan picks S so that the
// grid is about 256 workgroups: all of the matrix is requested at once.
constexpr int kGemvTargetWgs = 320;
constexpr int kGemvNt = 2;  // cache policy: non-temporal (weights are read once)

template <int NT, int S>
__global__ __launch_bounds__(kThreads) void w4a16_gemv_kernel(GemvArgs a) {
  constexpr int kRows = S * kRowsPerStep;  // packed rows per slice
  __shared__ uint4 xs[NT][kRows];
  __shared__ float xb[NT][kRows];
  __shared__ float red[kWaves * NT * kCols];
  __shared__ int last;
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid >> 6;
  const int rsub = lane >> 4, colq = lane & 15;
  const int tile = blockIdx.x, split = blockIdx.y;
  const int Kp = a.K >> 3, rpg = a.gs >> 3;
  const int r_begin = split * kRows;
  const int nrows = min(kRows, Kp - r_begin);
  const int col = tile * kCols + colq * 4;
  const bool col_ok = col < a.N;

  const __amdgpu_buffer_rsrc_t rb = buffer_rsrc(a.B, (uint32_t)((size_t)Kp * a.N * 4));
  const __amdgpu_buffer_rsrc_t rs = buffer_rsrc(a.S, (uint32_t)((size_t)a.G * a.N * 2));
  const __amdgpu_buffer_rsrc_t ra = buffer_rsrc(a.A, (uint32_t)((size_t)a.M * a.K * 2));
  constexpr uint32_t kOob = 0xFFFFFFF0u;
  constexpr int kXPer = (NT * kRows + kThreads - 1) / kThreads;  // 16-byte x vectors per thread
  uint4 xv[kXPer];
#pragma unroll
  for (int i = 0; i < kXPer; ++i) {
    const int idx = tid + kThreads * i;
    const int n = idx / kRows, rr = idx - n * kRows;
    const bool ok = n < NT && n < a.M && rr < nrows;
    const u32x4_t d = __builtin_amdgcn_raw_buffer_load_b128(
        ra, ok ? (uint32_t)(((size_t)n * a.K + 8 * (r_begin + rr)) * 2) : kOob, 0, 0);
    xv[i] = make_uint4(d.x, d.y, d.z, d.w);
  }
  __builtin_amdgcn_sched_barrier(0);
  uint4 w[S];
  uint2 sc[S];
#pragma unroll
  for (int j = 0; j < S; ++j) {
    const int rl = j * kRowsPerStep + wave * 4 + rsub;
    const int r = r_begin + rl;
    const bool ok = col_ok && rl < nrows;
    const u32x4_t d = __builtin_amdgcn_raw_buffer_load_b128(rb, ok ? (uint32_t)(((size_t)r * a.N + col) * 4) : kOob,
                                                            0, kGemvNt);
    w[j] = make_uint4(d.x, d.y, d.z, d.w);
    const int g = r / rpg;
    const u32x2_t e = __builtin_amdgcn_raw_buffer_load_b64(rs, (ok && g < a.G) ? (uint32_t)((g * a.N + col) * 2) : kOob,
                                                           0, 0);
    sc[j] = make_uint2(e.x, e.y);
  }
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int i = 0; i < kXPer; ++i) {
    const int idx = tid + kThreads * i;
    const int n = idx / kRows, rr = idx - n * kRows;
    if (n < NT) {
      xs[n][rr] = pair_permute(xv[i]);
      xb[n][rr] = q4_bias(xv[i]);
    }
  }
  __syncthreads();

  const uint32_t mq = q4_magic();
  float acc[4][NT];
#pragma unroll
  for (int q = 0; q < 4; ++q)
#pragma unroll
    for (int n = 0; n < NT; ++n) acc[q][n] = 0.f;
#pragma unroll
  for (int j = 0; j < S; ++j) {
    const int rl = j * kRowsPerStep + wave * 4 + rsub;
    const float sv[4] = {bf16lo(sc[j].x), bf16hi(sc[j].x), bf16lo(sc[j].y), bf16hi(sc[j].y)};
    const Q4Pairs u[4] = {unpack_q4(w[j].x, mq), unpack_q4(w[j].y, mq), unpack_q4(w[j].z, mq),
                          unpack_q4(w[j].w, mq)};
#pragma unroll
    for (int n = 0; n < NT; ++n) {
      const uint4 xp = xs[n][rl];
      const float bias = xb[n][rl];
#pragma unroll
      for (int q = 0; q < 4; ++q) acc[q][n] = fmaf(sv[q], dot_unpacked(u[q], xp, bias), acc[q][n]);
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
      for (int q = 0; q < 4; ++q) red[(wave * NT + n) * kCols + colq * 4 + q] = acc[q][n];
  }
  __syncthreads();
  const int mt = min(NT, a.M);
  for (int i = tid; i < mt * kCols; i += kThreads) {
    const int n = i / kCols, cc = i - n * kCols;
    const int oc = tile * kCols + cc;
    if (oc < a.N) {
      const float y = (red[(0 * NT + n) * kCols + cc] + red[(1 * NT + n) * kCols + cc]) +
                      (red[(2 * NT + n) * kCols + cc] + red[(3 * NT + n) * kCols + cc]);
      const size_t o = (size_t)n * a.N + oc;
      if (a.ks == 1) a.C[o] = f32_to_bf16(epilogue(y, a.cap));
      else st_coherent_f32(a.part + (size_t)split * a.M * a.N + o, y);
    }
  }
  if (a.ks == 1) return;

  // Last K slice to arrive for this column tile sums the partials in slice order.
  wait_vmem();
  __syncthreads();
  if (tid == 0) last = atomic_add_relaxed(&a.ctr[tile], 1) == a.ks - 1;
  __syncthreads();
  if (!last) return;
  for (int i = tid; i < mt * kCols; i += kThreads) {
    const int t = i / kCols, cc = i - t * kCols;
    const int oc = tile * kCols + cc;
    if (oc < a.N) {
      const size_t o = (size_t)t * a.N + oc;
      float y = 0.f;
      for (int s2 = 0; s2 < a.ks; ++s2) y += ld_coherent_f32(a.part + (size_t)s2 * a.M * a.N + o);
      a.C[o] = f32_to_bf16(epilogue(y, a.cap));
    }
  }
  if (tid == 0) store_relaxed(&a.ctr[tile], 0);
}

// ---------------------------------------------------------------------------
// One or two token rows and K <= 8192: NC (8 or 16) columns per workgroup
// over ALL of K, so N / NC workgroups fill the chip without a K split and a
// launch has no inter-workgroup exchange at all.  A lane loads the 16 bytes
// of 4 columns: LPR = NC / 4 lanes cover a packed row, a wave instruction
// reads RW = 64 / LPR rows x 4NC bytes (NC 16: 16 rows x 64 B; NC 8: 32 rows
// x 32 B), a step of the 4 waves 4RW rows.  Every load goes out first: the
// token rows (staged into LDS as soon as they land: the waits count in issue
// order, so rows issued after the weights would wait for every weight word),
// then the scales, then the weights, whose steps the products take as they
// land; rows past K read zeros through the buffer range check.  The sums over
// the lanes of a column group: DPP rotations inside each row of 16 lanes, permlane swaps
// across the four rows, then the 4 wave partials of a column in LDS, added in
// a fixed order.
// Workgroup b runs on XCD b % 8: with a grid of whole rounds of 8 the tiles
// are handed out so that each XCD holds a contiguous run of them, and tiles
// that share a 128-byte line of the words meet in one L2.
constexpr int kNarrowColsMax = 16;
constexpr int kMaxSegs = 4;
constexpr int kNarrowColsM1 = 16;  // tile width of the one- and two-row calls
constexpr bool kNarrowXcdOrder = true;

// Several projections of the same token rows in one launch: segment s owns
// column tiles [tile0, tile0 + ceil(N / NC)).  GATED: segments 0 and 1 are
// the gate and up projections of a gated MLP with the same N; every
// workgroup computes both for its NC columns and writes
// bf16(bf16(gelu_tanh(bf16(gate))) * bf16(up)) to segment 0's output.
struct NarrowSeg {
  const int32_t* B;  // [K/8, N]
  const uint16_t* S; // [G, N]
  uint16_t* C;       // [M, N]
  int N, G, tile0;
};
struct NarrowArgs {
  const uint16_t* A;  // [M, K]
  int M, K, gs, nseg;
  uint32_t gmul;      // ceil(2^20 / (gs / 8)): scale group of a packed row by a multiply
  float cap;
  NarrowSeg seg[kMaxSegs];
};

// The segment that owns column tile b.  Every segment's fields are loaded in
// one batch and selected: a branch per segment would wait for each argument
// load in turn before the kernel's first vector load.
template <bool SINGLE>
__device__ __forceinline__ NarrowSeg select_seg(const NarrowSeg (&seg)[kMaxSegs], int b) {
  int si = 0;
  if constexpr (!SINGLE) {
#pragma unroll
    for (int i = 1; i < kMaxSegs; ++i) si += b >= seg[i].tile0 ? 1 : 0;
  }
  NarrowSeg sg = seg[0];
#pragma unroll
  for (int i = 1; i < kMaxSegs; ++i) {
    const bool t = si >= i;
    sg.B = t ? seg[i].B : sg.B;
    sg.S = t ? seg[i].S : sg.S;
    sg.C = t ? seg[i].C : sg.C;
    sg.N = t ? seg[i].N : sg.N;
    sg.G = t ? seg[i].G : sg.G;
    sg.tile0 = t ? seg[i].tile0 : sg.tile0;
  }
  return sg;
}

template <int S>
struct NarrowW {
  uint4 w[S];
  uint2 sc[S];
};

template <int NC>
struct NarrowShape {
  static constexpr int LPR = NC / 4;      // lanes per packed row
  static constexpr int RW = kWave / LPR;  // rows per wave instruction
  static constexpr int RS = kWaves * RW;  // rows per step
};

// The loads of one projection's S steps.  Rows past K read zeros through the
// buffer's range check (their x rows are zero too); a column past N (the last
// tile of an N that is not a multiple of NC) reads other columns' words and
// scales, into sums that are never stored.  The word offsets advance by a
// constant per step; the scale group of packed row r is (r * gmul) >> 20 with
// gmul = ceil(2^20 / rpg), which equals r / rpg for every r and rpg below 1024
// (the error r * (gmul * rpg - 2^20) stays below 2^20).
template <int NC, int S>
__device__ __forceinline__ void narrow_issue(const NarrowSeg& sg, int Kp, uint32_t gmul, int col, int wave, int rrow,
                                             NarrowW<S>& o) {
  using Sh = NarrowShape<NC>;
  const __amdgpu_buffer_rsrc_t rb = buffer_rsrc(sg.B, (uint32_t)((size_t)Kp * sg.N * 4));
  const __amdgpu_buffer_rsrc_t rs = buffer_rsrc(sg.S, (uint32_t)((size_t)sg.G * sg.N * 2));
  const uint32_t n = (uint32_t)sg.N, r0 = (uint32_t)(Sh::RW * wave + rrow);
  const uint32_t wo = (r0 * n + (uint32_t)col) * 4u;
  // the scales first: the waits count in issue order, and step j's products
  // need its scales, not the later steps' words
#pragma unroll
  for (int j = 0; j < S; ++j) {
    const uint32_t g = ((r0 + (uint32_t)(Sh::RS * j)) * gmul) >> 20;
    const u32x2_t e = __builtin_amdgcn_raw_buffer_load_b64(rs, (g * n + (uint32_t)col) * 2u, 0, 0);
    o.sc[j] = make_uint2(e.x, e.y);
  }
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int j = 0; j < S; ++j) {
    const u32x4_t d = __builtin_amdgcn_raw_buffer_load_b128(rb, wo + (uint32_t)j * (Sh::RS * 4u) * n, 0, kGemvNt);
    o.w[j] = make_uint4(d.x, d.y, d.z, d.w);
  }
}

template <int NC, int NT, int S, int kRows>
__device__ __forceinline__ void narrow_products(const NarrowW<S>& in, const uint4 (&xs)[NT][kRows],
                                                const float (&xb)[NT][kRows], int wave, int rrow, uint32_t mq,
                                                float (&acc)[4][NT]) {
  using Sh = NarrowShape<NC>;
#pragma unroll
  for (int q = 0; q < 4; ++q)
#pragma unroll
    for (int n = 0; n < NT; ++n) acc[q][n] = 0.f;
#pragma unroll
  for (int j = 0; j < S; ++j) {
    const int r = Sh::RS * j + Sh::RW * wave + rrow;
    const float sv[4] = {bf16lo(in.sc[j].x), bf16hi(in.sc[j].x), bf16lo(in.sc[j].y), bf16hi(in.sc[j].y)};
    const Q4Pairs u[4] = {unpack_q4(in.w[j].x, mq), unpack_q4(in.w[j].y, mq), unpack_q4(in.w[j].z, mq),
                          unpack_q4(in.w[j].w, mq)};
#pragma unroll
    for (int n = 0; n < NT; ++n) {
      const uint4 xp = xs[n][r];
      const float bias = xb[n][r];
#pragma unroll
      for (int q = 0; q < 4; ++q) acc[q][n] = fmaf(sv[q], dot_unpacked(u[q], xp, bias), acc[q][n]);
    }
  }
  // lanes c, c + LPR, c + 2LPR, ... of each 16-lane row share a column group
#pragma unroll
  for (int q = 0; q < 4; ++q)
#pragma unroll
    for (int n = 0; n < NT; ++n) {
      float v = acc[q][n];
      if constexpr (NC == 8) v += dpp_f32<0x122>(v);  // row_ror:2
      v += dpp_f32<0x124>(v);                         // row_ror:4
      v += dpp_f32<0x128>(v);                         // row_ror:8
      // then the four 16-lane rows: (r0 + r2) + (r1 + r3), in every lane
      const auto h = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
      const float x = __uint_as_float(h[0]) + __uint_as_float(h[1]);
      const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
      acc[q][n] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
}

template <int NC, int NT, int S, bool GATED>
__global__ __launch_bounds__(kThreads) void w4a16_narrow_kernel(NarrowArgs a) {
  using Sh = NarrowShape<NC>;
  constexpr int kRows = S * Sh::RS;  // packed rows covered (>= K / 8)
  constexpr int kOut = GATED ? 2 : 1;
  __shared__ uint4 xs[NT][kRows];
  __shared__ float xb[NT][kRows];
  __shared__ float red[kOut][kWaves][NT][NC];
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid >> 6;
  const int rrow = lane / Sh::LPR, colq = lane % Sh::LPR;
  const int Kp = a.K >> 3;
  const int nb = (int)gridDim.x, b0 = (int)blockIdx.x;
  // XCD-aware order for grids of whole rounds of 8 (arithmetic, not a branch:
  // the argument loads below then go out in one batch)
  const int xo = (kNarrowXcdOrder && (nb & 7) == 0) ? 1 : 0;
  const int b = b0 + xo * ((b0 & 7) * (nb >> 3) + (b0 >> 3) - b0);
  const NarrowSeg sg = select_seg<GATED>(a.seg, b);
  const int c0 = (b - sg.tile0) * NC;
  const int col = c0 + colq * 4;

  const __amdgpu_buffer_rsrc_t ra = buffer_rsrc(a.A, (uint32_t)((size_t)a.M * a.K * 2));
  constexpr uint32_t kOob = 0xFFFFFFF0u;
  constexpr int kXPer = (NT * kRows + kThreads - 1) / kThreads;
  uint4 xv[kXPer];
#pragma unroll
  for (int i = 0; i < kXPer; ++i) {
    const int idx = tid + kThreads * i;
    const int n = idx / kRows, rr = idx - n * kRows;
    const bool ok = n < NT && n < a.M && rr < Kp;
    const u32x4_t d = __builtin_amdgcn_raw_buffer_load_b128(ra, ok ? (uint32_t)(((size_t)n * a.K + 8 * rr) * 2) : kOob,
                                                            0, 0);
    xv[i] = make_uint4(d.x, d.y, d.z, d.w);
  }
  __builtin_amdgcn_sched_barrier(0);
  NarrowW<S> w0;
  narrow_issue<NC, S>(sg, Kp, a.gmul, col, wave, rrow, w0);
  NarrowW<S> w1;
  if constexpr (GATED) narrow_issue<NC, S>(a.seg[1], Kp, a.gmul, col, wave, rrow, w1);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int i = 0; i < kXPer; ++i) {
    const int idx = tid + kThreads * i;
    const int n = idx / kRows, rr = idx - n * kRows;
    if (n < NT) {
      xs[n][rr] = pair_permute(xv[i]);
      xb[n][rr] = q4_bias(xv[i]);
    }
  }
  __syncthreads();

  const uint32_t mq = q4_magic();
  const int slot = wave;  // one partial per wave and column
  {
    float acc[4][NT];
    narrow_products<NC, NT, S, kRows>(w0, xs, xb, wave, rrow, mq, acc);
    if (lane < Sh::LPR) {
#pragma unroll
      for (int n = 0; n < NT; ++n)
#pragma unroll
        for (int q = 0; q < 4; ++q) red[0][slot][n][colq * 4 + q] = acc[q][n];
    }
  }
  if constexpr (GATED) {
    float acc[4][NT];
    narrow_products<NC, NT, S, kRows>(w1, xs, xb, wave, rrow, mq, acc);
    if (lane < Sh::LPR) {
#pragma unroll
      for (int n = 0; n < NT; ++n)
#pragma unroll
        for (int q = 0; q < 4; ++q) red[kOut - 1][slot][n][colq * 4 + q] = acc[q][n];
    }
  }
  __syncthreads();
  if (tid < NT * NC) {
    const int n = tid / NC, cc = tid - n * NC;
    const int oc = c0 + cc;
    if (n < a.M && oc < sg.N) {
      float y = 0.f;
#pragma unroll
      for (int i = 0; i < kWaves; ++i) y += red[0][i][n][cc];
      if constexpr (GATED) {
        float u = 0.f;
#pragma unroll
        for (int i = 0; i < kWaves; ++i) u += red[kOut - 1][i][n][cc];
        // activations.py:26-28 on bf16 tensors: each linear's output, the
        // gelu and the product are rounded to bf16
        const float g = round_to_bf16(gelu_tanh(round_to_bf16(y)));
        sg.C[(size_t)n * sg.N + oc] = f32_to_bf16(g * round_to_bf16(u));
      } else {
        sg.C[(size_t)n * sg.N + oc] = f32_to_bf16(epilogue(y, a.cap));
      }
    }
  }
}

constexpr int kNarrowSteps[] = {2, 3, 4, 6, 8, 12, 16};

// Packed rows a narrow launch addresses (whole steps of 64 or 128 rows, rows
// past K included): every word offset stays below 2^32 when this many rows of
// N columns do.
size_t narrow_rows(int Kp) {
  size_t rows = 0;
  for (int rs : {64, 128})
    for (int st : kNarrowSteps)
      if (st * rs >= Kp) {
        rows = std::max(rows, (size_t)st * rs);
        break;
      }
  return rows;
}

bool narrow_path(int M, int K, int N) {
  const int Kp = K / 8;
  return M <= 2 && Kp <= 64 * 16 && N >= 1024 && narrow_rows(Kp) * N * 4 < (1ull << 32);
}

template <int NC, int NT, bool G>
int launch_narrow_t(const NarrowArgs& k, int tiles, int steps, hipStream_t stream) {
  const dim3 grid((unsigned)tiles);
  switch (steps) {
#define GI_NARROW_CASE(S)                                                                         \
  case S:                                                                                         \
    hipLaunchKernelGGL((w4a16_narrow_kernel<NC, NT, S, G>), grid, dim3(kThreads), 0, stream, k); \
    break;
    GI_NARROW_CASE(2) GI_NARROW_CASE(3) GI_NARROW_CASE(4) GI_NARROW_CASE(6) GI_NARROW_CASE(8)
    GI_NARROW_CASE(12) GI_NARROW_CASE(16)
#undef GI_NARROW_CASE
    default:
      return fail(GI_ERR_UNSUPPORTED, "w4a16: no narrow-tile variant for this shape");
  }
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? GI_OK : hip_fail(e, "w4a16 narrow launch");
}

int launch_narrow(const void* A, int M, int K, int gs, float cap, const NarrowSeg* segs, int nseg, bool gated,
                  hipStream_t stream) {
  // one plain projection uses the M=1 tile width; several projections and the
  // gated form keep 16 columns (their grids are already large)
  const int nc = (!gated && nseg == 1) ? kNarrowColsM1 : kNarrowColsMax;
  NarrowArgs k{};
  k.A = (const uint16_t*)A;
  k.M = M;
  k.K = K;
  k.gs = gs;
  k.gmul = (uint32_t)(((1u << 20) + (uint32_t)(gs / 8) - 1) / (uint32_t)(gs / 8));
  k.cap = cap;
  k.nseg = nseg;
  int tiles = 0;
  for (int i = 0; i < nseg; ++i) {
    k.seg[i] = segs[i];
    k.seg[i].tile0 = gated ? 0 : tiles;
    if (!gated) tiles += (segs[i].N + nc - 1) / nc;
  }
  if (gated) tiles = (segs[0].N + nc - 1) / nc;
  for (int i = nseg; i < kMaxSegs; ++i) k.seg[i].tile0 = 0x7fffffff;
  const int rows_per_step = kWaves * (kWave / (nc / 4));
  const int need = (K / 8 + rows_per_step - 1) / rows_per_step;
  int steps = 0;
  for (int st : kNarrowSteps)
    if (st >= need) {
      steps = st;
      break;
    }
  if (steps == 0) return fail(GI_ERR_UNSUPPORTED, "w4a16: no narrow-tile variant for this shape");
  if (nc == 8) {
    if (M <= 1) return launch_narrow_t<8, 1, false>(k, tiles, steps, stream);
    return launch_narrow_t<8, 2, false>(k, tiles, steps, stream);
  }
  if (gated) {
    if (M <= 1) return launch_narrow_t<16, 1, true>(k, tiles, steps, stream);
    return launch_narrow_t<16, 2, true>(k, tiles, steps, stream);
  }
  if (M <= 1) return launch_narrow_t<16, 1, false>(k, tiles, steps, stream);
  return launch_narrow_t<16, 2, false>(k, tiles, steps, stream);
}

// ---------------------------------------------------------------------------
// Matrix-core path for up to 16 token rows and a wide N (lm_head): the
// products run on v_mfma_f32_16x16x32_bf16 (with 3..16 rows the VALU dot
// products would cost more than the weight stream; with one or two rows this
// kernel's long register ring still streams a 380 MB lm_head faster than
// 16384 narrow workgroups do) with A = the token
// rows (zero rows past M) and B = the unpacked int4 words (16 + q), plus one
// product with a constant -24 operand per k block for the offset.  A
// workgroup owns 256 columns over all of K (wave w: 64 of them; lane
// (lq, lr) loads the 16 bytes of columns 4lr..4lr+3 at packed row 4kb + lq,
// i.e. the B operands of four 16-column products).  The weights stream
// through a ring of kMfRing register slots (the load for k block kb + ring
// goes out as kb is consumed).  The k blocks of a pass are straight-line
// code (kMfPass of them, the tail past K reads zeros from the buffer
// resource), so that every wait has an exact count: a ring carried around a
// loop is drained at the loop header.  x and the scales of the workgroup's
// columns sit in LDS.  Groups end every KPG = gs/32 k blocks:
// y += scale * (D + Db); groups at or past G (a floor-size scales tensor)
// are dropped like the reference's kernels (marlin.cu:128).
// ---------------------------------------------------------------------------
using moe::f32x4_t;
constexpr int kMfThreads = 256;  // the 4-wave form (the 8-wave form: twice both)
constexpr int kMfCols = 256;     // output columns per workgroup (64 per wave)
constexpr int kMfRing = 8;       // k blocks in flight per wave
constexpr int kMfPass = 96;   // k blocks per straight-line pass (K <= 3072 in one pass)
constexpr int kMfMaxM = 16;
constexpr int kMfXChunks = 4096;  // staged x chunks per workgroup at most (the 64 KB LDS bound)
constexpr int kMfSB = 8;   // scale entries per thread loaded in the first batch
constexpr uint32_t kMfOob = 0xFFFFFFF0u;

struct MfArgs {
  const uint16_t* A;  // [M, K] bf16
  const int32_t* B;   // [K/8, N]
  const uint16_t* S;  // [G, N] bf16
  uint16_t* C;        // [M, N] bf16
  int M, K, N, G;
  uint32_t b_bytes;
  float cap;
  float* part;  // [ks, M, N] fp32 (matrix-core narrow path, ks > 1)
  int* ctr;     // [N / 64] arrival counters (ks > 1)
  int ks;       // K slices over gridDim.y
};

// NW waves per workgroup (4 or 8): 64 NW columns.  With 8 waves a 512-column
// workgroup stages x once for twice the columns and the lm_head grid (512
// workgroups, two per CU) is one round; with 4 waves (256 columns) its 1024
// workgroups, three per CU by LDS, ran a third-full second round.
template <int KPG, int NW>
__global__ __launch_bounds__(NW * kWave, 2) void w4a16_mfma_kernel(MfArgs a) {
  constexpr int T = NW * kWave, kCols = 64 * NW, kQuads = 16 * NW;
  constexpr int kXB = kMfXChunks / T;  // staged x chunks per thread
  constexpr int kQsh = NW == 8 ? 7 : 6;
  static_assert(kQuads == 1 << kQsh, "quads per group are a power of two");
  extern __shared__ uint4 mf_lds[];
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid >> 6;
  const int lq = lane >> 4, lr = lane & 15;
  const int Kp = a.K >> 3, KB = a.K >> 5;
  const int col0 = blockIdx.x * kCols;
  uint4* xs = mf_lds;                                     // [M + 1][Kp], row M zero
  uint2* ss = (uint2*)(mf_lds + (size_t)(a.M + 1) * Kp);  // [G][kQuads]: scales of column quad c
  const __amdgpu_buffer_rsrc_t rb = buffer_rsrc(a.B, a.b_bytes);
  const uint32_t rstep = (uint32_t)a.N * 16u;  // 4 packed rows
  const uint32_t voff = (uint32_t)lq * (uint32_t)a.N * 4u + (uint32_t)(col0 + wave * 64 + 4 * lr) * 4u;
  // Every start-up load goes out before any use: the x rows (one batch: the
  // LDS bound of this path keeps them within kXB chunks per thread), the
  // first kMfSB scale entries per thread and, for a one-pass K, the weight
  // ring.  The staged values are written to LDS as they land, and the
  // barrier waits for LDS only, so the ring stays in flight (staged one
  // round trip at a time, the x rows and scales held every workgroup ~16
  // memory round trips before its first weight load).  Offsets past the
  // tensors read zeros (row M, the zero operand row, included).
  const int nxs = (a.M + 1) * Kp, nss = a.G * kQuads;
  const __amdgpu_buffer_rsrc_t rx = buffer_rsrc(a.A, (uint32_t)a.M * (uint32_t)a.K * 2u);
  const __amdgpu_buffer_rsrc_t rs =
      buffer_rsrc(a.S + col0, (uint32_t)(((size_t)(a.G - 1) * a.N + kCols) * 2));
  u32x4_t xv[kXB];
  {
    // chunk i = j * T + tid is chunk r of row n (i = n * Kp + r)
    const int dn = T / Kp, dr = T - dn * Kp;
    int n = tid / Kp, r = tid - n * Kp;
#pragma unroll
    for (int j = 0; j < kXB; ++j) {
      const bool in = j * T + tid < nxs && n < a.M;
      xv[j] = __builtin_amdgcn_raw_buffer_load_b128(rx, in ? (uint32_t)(n * a.K + 8 * r) * 2u : kMfOob, 0, 0);
      n += dn;
      r += dr;
      const bool wrap = r >= Kp;
      r -= wrap ? Kp : 0;
      n += wrap ? 1 : 0;
    }
  }
  u32x2_t sv[kMfSB];
#pragma unroll
  for (int j = 0; j < kMfSB; ++j) {
    const int i = j * T + tid;
    const uint32_t off =
        i < nss ? ((uint32_t)(i >> kQsh) * (uint32_t)a.N + 4u * (uint32_t)(i & (kQuads - 1))) * 2u : kMfOob;
    sv[j] = __builtin_amdgcn_raw_buffer_load_b64(rs, off, 0, 0);
  }
  uint4 w[kMfRing];
  const bool one_pass = KB <= kMfPass;
  if (one_pass) {
#pragma unroll
    for (int s = 0; s < kMfRing; ++s) {
      const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(rb, voff + (uint32_t)s * rstep, 0, 2);
      w[s] = make_uint4(v.x, v.y, v.z, v.w);
    }
  }
  // x rows in the matrix-core k order, and this workgroup's scales
#pragma unroll
  for (int j = 0; j < kXB; ++j) {
    const int i = j * T + tid;
    if (i < nxs) xs[i] = moe::mfma_k_order(make_uint4(xv[j].x, xv[j].y, xv[j].z, xv[j].w));
  }
#pragma unroll
  for (int j = 0; j < kMfSB; ++j) {
    const int i = j * T + tid;
    if (i < nss) ss[i] = make_uint2(sv[j].x, sv[j].y);
  }
  for (int i = kMfSB * T + tid; i < nss; i += T) {
    const int g = i >> kQsh, c = i & (kQuads - 1);
    ss[i] = *(const uint2*)(a.S + (size_t)g * a.N + col0 + 4 * c);
  }
  lds_barrier();

  const uint32_t mq = q4_magic();
  const f32x4_t zf = {0.f, 0.f, 0.f, 0.f};
  const uint4 bc = make_uint4(moe::kQ4BiasPair, moe::kQ4BiasPair, moe::kQ4BiasPair, moe::kQ4BiasPair);
  const uint4* xrow = xs + (size_t)(lr < a.M ? lr : a.M) * Kp + lq;
  const uint2* srow = ss + wave * 16 + lr;
  f32x4_t y[4] = {zf, zf, zf, zf};
  for (int kp = 0; kp < KB; kp += kMfPass) {
    if (!one_pass) {
#pragma unroll
      for (int s = 0; s < kMfRing; ++s) {
        const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(rb, voff + (uint32_t)(kp + s) * rstep, 0, 2);
        w[s] = make_uint4(v.x, v.y, v.z, v.w);
      }
    }
    f32x4_t D[4] = {zf, zf, zf, zf};
    f32x4_t Db = zf;
#pragma unroll
    for (int j = 0; j < kMfPass; ++j) {
      const int kb = kp + j;
      if (kb < KB) {
        const uint4 A = xrow[4 * kb];
        const uint4 wv = w[j % kMfRing];
        D[0] = moe::mfma_bf16(A, moe::q4_operand(wv.x, mq), D[0]);
        D[1] = moe::mfma_bf16(A, moe::q4_operand(wv.y, mq), D[1]);
        D[2] = moe::mfma_bf16(A, moe::q4_operand(wv.z, mq), D[2]);
        D[3] = moe::mfma_bf16(A, moe::q4_operand(wv.w, mq), D[3]);
        Db = moe::mfma_bf16(A, bc, Db);
        // a group ends after k block kb (kMfPass is a multiple of KPG, so
        // groups never straddle passes), or K ends
        if ((j + 1) % KPG == 0 || kb == KB - 1) {
          const int g = kb / KPG;
          if (g < a.G) {
            const uint2 sv = srow[g * kQuads];
            const float sc[4] = {bf16lo(sv.x), bf16hi(sv.x), bf16lo(sv.y), bf16hi(sv.y)};
#pragma unroll
            for (int q = 0; q < 4; ++q)
#pragma unroll
              for (int jj = 0; jj < 4; ++jj) y[q][jj] += sc[q] * (D[q][jj] + Db[jj]);
          }
#pragma unroll
          for (int q = 0; q < 4; ++q) D[q] = zf;
          Db = zf;
        }
      }
      if (j + kMfRing < kMfPass) {
        const u32x4_t v =
            __builtin_amdgcn_raw_buffer_load_b128(rb, voff + (uint32_t)(kb + kMfRing) * rstep, 0, 2);
        w[j % kMfRing] = make_uint4(v.x, v.y, v.z, v.w);
      }
    }
  }
  // token rows 4lq + jj, columns col0 + 64 wave + 4 lr + q
#pragma unroll
  for (int jj = 0; jj < 4; ++jj) {
    const int t = 4 * lq + jj;
    if (t < a.M) {
      uint32_t o[2];
#pragma unroll
      for (int h = 0; h < 2; ++h)
        o[h] = (uint32_t)f32_to_bf16(epilogue(y[2 * h][jj], a.cap)) |
               ((uint32_t)f32_to_bf16(epilogue(y[2 * h + 1][jj], a.cap)) << 16);
      *(uint2*)(a.C + (size_t)t * a.N + col0 + wave * 64 + 4 * lr) = make_uint2(o[0], o[1]);
    }
  }
}

// ---------------------------------------------------------------------------
// Matrix-core path for 3..16 rows and the narrower N of the dense projections:
// a workgroup of 8 waves owns 64 columns over all of K, the waves splitting K
// into 8 ranges of KBW k blocks (KBW a multiple of the group's k blocks, so
// no group straddles two waves).  Lane (lq, lr) loads the 16 bytes of columns
// 4lr..4lr+3 at packed row 4kb + lq: the B operands of four 16-column
// products, as on the lm_head path.  Every weight and scale load of a wave
// goes out first (k blocks past K and columns past N read zeros), then the
// token rows are staged into LDS in the matrix-core k order; the partial
// sums of the 8 waves are added in LDS in a fixed order.  No K split across
// workgroups, so a launch has no inter-workgroup exchange.
constexpr size_t kAlign = 256;
inline size_t round_up(size_t v) { return (v + kAlign - 1) / kAlign * kAlign; }
// Split-K workspace: arrival counters at the front, partials from a fixed
// offset.  Calls of different shapes share one workspace, so the counter
// region must never be reused for partials (a counter left non-zero by
// another call's partials breaks the last-arriver test): it is sized for
// N <= 64 * 16384.
constexpr size_t kCtrBytes = 16384 * sizeof(int);
constexpr int kMnWaves = 8;
constexpr int kMnThreads = kMnWaves * kWave;
constexpr int kMnCols = 64;

// Segments as on the VALU narrow path: several projections of the same rows
// in one grid (segment s owns 64-column tiles [tile0, tile0 + ceil(N/64))),
// or GATED: the gate and up projections of a gated MLP, both computed by
// every workgroup for its 64 columns, written as
// bf16(bf16(gelu_tanh(bf16(gate))) * bf16(up)).  With a K split the fp32
// partials are indexed by the grid's global column (tile * 64 + c).
struct MnArgs {
  const uint16_t* A;  // [M, K]
  int M, K, ks, ntot;  // ntot = tiles * 64
  float cap;
  float* part;  // [ks][GATED ? 2 : 1][M][ntot] (ks > 1)
  int* ctr;     // [tiles] (ks > 1)
  NarrowSeg seg[kMaxSegs];
};

template <int KBW, int KPG>
__device__ __forceinline__ void mn_issue(const NarrowSeg& sg, int Kp, int KB, int col, int kb0, int lq,
                                         uint4 (&w)[KBW], uint2 (&sc)[KBW / KPG]) {
  constexpr uint32_t kOob = 0xFFFFFFF0u;
  const bool col_ok = col < sg.N;
  const __amdgpu_buffer_rsrc_t rb = buffer_rsrc(sg.B, (uint32_t)((size_t)Kp * sg.N * 4));
  const __amdgpu_buffer_rsrc_t rs = buffer_rsrc(sg.S, (uint32_t)((size_t)sg.G * sg.N * 2));
#pragma unroll
  for (int s = 0; s < KBW; ++s) {
    const int kb = kb0 + s;
    const bool ok = col_ok && kb < KB;
    const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(
        rb, ok ? (uint32_t)(((size_t)(4 * kb + lq) * sg.N + col) * 4) : kOob, 0, kGemvNt);
    w[s] = make_uint4(v.x, v.y, v.z, v.w);
  }
#pragma unroll
  for (int t = 0; t < KBW / KPG; ++t) {
    const int g = kb0 / KPG + t;
    const u32x2_t v = __builtin_amdgcn_raw_buffer_load_b64(
        rs, (col_ok && g < sg.G) ? (uint32_t)((g * sg.N + col) * 2) : kOob, 0, 0);
    sc[t] = make_uint2(v.x, v.y);
  }
}

template <int KBW, int KPG>
__device__ __forceinline__ void mn_products(const uint4 (&w)[KBW], const uint2 (&sc)[KBW / KPG], const uint4* xrow,
                                            int kb0, int KB, uint32_t mq, f32x4_t (&y)[4]) {
  const f32x4_t zf = {0.f, 0.f, 0.f, 0.f};
  const uint4 bc = make_uint4(moe::kQ4BiasPair, moe::kQ4BiasPair, moe::kQ4BiasPair, moe::kQ4BiasPair);
  const uint4 z4 = make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
  for (int q = 0; q < 4; ++q) y[q] = zf;
#pragma unroll
  for (int t = 0; t < KBW / KPG; ++t) {
    f32x4_t D[4] = {zf, zf, zf, zf};
    f32x4_t Db = zf;
#pragma unroll
    for (int s = 0; s < KPG; ++s) {
      const int j = t * KPG + s;
      const int kb = kb0 + j;
      const uint4 A = kb < KB ? xrow[4 * kb] : z4;
      D[0] = moe::mfma_bf16(A, moe::q4_operand(w[j].x, mq), D[0]);
      D[1] = moe::mfma_bf16(A, moe::q4_operand(w[j].y, mq), D[1]);
      D[2] = moe::mfma_bf16(A, moe::q4_operand(w[j].z, mq), D[2]);
      D[3] = moe::mfma_bf16(A, moe::q4_operand(w[j].w, mq), D[3]);
      Db = moe::mfma_bf16(A, bc, Db);
    }
    const float scv[4] = {bf16lo(sc[t].x), bf16hi(sc[t].x), bf16lo(sc[t].y), bf16hi(sc[t].y)};
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) y[q][jj] += scv[q] * (D[q][jj] + Db[jj]);
  }
}

__device__ __forceinline__ float mn_out(float y, float u, float cap, bool gated) {
  // activations.py:26-28 on bf16 tensors for the gated form
  return gated ? round_to_bf16(gelu_tanh(round_to_bf16(y))) * round_to_bf16(u) : epilogue(y, cap);
}

template <int KBW, int KPG, bool GATED>
__global__ __launch_bounds__(kMnThreads) void w4a16_mfma_narrow_kernel(MnArgs a) {
  extern __shared__ uint4 mf_lds[];
  constexpr int kOut = GATED ? 2 : 1;
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid >> 6;
  const int lq = lane >> 4, lr = lane & 15;
  const int Kp = a.K >> 3, KB = a.K >> 5;
  const NarrowSeg sg = select_seg<GATED>(a.seg, (int)blockIdx.x);
  const int c0 = ((int)blockIdx.x - sg.tile0) * kMnCols;
  const int col = c0 + 4 * lr;
  const int slice = blockIdx.y;
  const int kb0 = (slice * kMnWaves + wave) * KBW;
  // this K slice of the token rows (row M, rows past it and packed rows past
  // K read as zero), loaded first and staged in the matrix-core k order as
  // soon as they land: the waits count in issue order, so rows issued after
  // the weights would wait for every weight word
  constexpr uint32_t kOob = 0xFFFFFFF0u;
  constexpr int kSp = kMnWaves * KBW * 4;  // packed rows of a slice
  constexpr int kXn = ((kMfMaxM + 1) * kSp + kMnThreads - 1) / kMnThreads;  // M <= 16 rows
  // the long slices (large K) keep the rows' loads behind the weights: their
  // registers would not fit beside the weight words
  constexpr bool kXFirst = kXn <= 8;
  const int r0 = slice * kSp;
  uint4* xs = mf_lds;  // [M + 1][kSp]
  const __amdgpu_buffer_rsrc_t ra = buffer_rsrc(a.A, (uint32_t)((size_t)a.M * a.K * 2));
  auto x_load = [&](int i) {
    const int n = i / kSp, r = r0 + (i - n * kSp);
    const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(
        ra, (n < a.M && r < Kp) ? (uint32_t)(((size_t)n * a.K + 8 * r) * 2) : kOob, 0, 0);
    return make_uint4(v.x, v.y, v.z, v.w);
  };
  uint4 xv[kXFirst ? kXn : 1];
  if constexpr (kXFirst) {
#pragma unroll
    for (int j = 0; j < kXn; ++j) xv[j] = x_load(tid + j * kMnThreads);
    __builtin_amdgcn_sched_barrier(0);
  }
  uint4 w0[KBW];
  uint2 s0[KBW / KPG];
  mn_issue<KBW, KPG>(sg, Kp, KB, col, kb0, lq, w0, s0);
  uint4 w1[GATED ? KBW : 1];
  uint2 s1[GATED ? KBW / KPG : 1];
  if constexpr (GATED) mn_issue<KBW, KPG>(a.seg[1], Kp, KB, col, kb0, lq, w1, s1);
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (kXFirst) {
#pragma unroll
    for (int j = 0; j < kXn; ++j) {
      const int i = tid + j * kMnThreads;
      if (i < (a.M + 1) * kSp) xs[i] = moe::mfma_k_order(xv[j]);
    }
  } else {
    for (int i = tid; i < (a.M + 1) * kSp; i += kMnThreads) xs[i] = moe::mfma_k_order(x_load(i));
  }
  __syncthreads();

  const uint32_t mq = q4_magic();
  // k block kb of this wave sits at packed row 4 (kb - slice * 8 KBW) + lq of the slice
  const uint4* xrow = xs + (size_t)(lr < a.M ? lr : a.M) * kSp + lq - 4 * (slice * kMnWaves * KBW);
  f32x4_t y0[4], y1[4];
  mn_products<KBW, KPG>(w0, s0, xrow, kb0, KB, mq, y0);
  if constexpr (GATED) mn_products<KBW, KPG>(w1, s1, xrow, kb0, KB, mq, y1);
  // y[q][jj]: token row 4lq + jj, column 4lr + q of the tile
  __syncthreads();  // every wave is done with xs
  float* red = (float*)mf_lds;  // [kOut][8 waves][16 rows][64 columns]
#pragma unroll
  for (int jj = 0; jj < 4; ++jj) {
    *(float4*)(red + ((size_t)wave * 16 + 4 * lq + jj) * kMnCols + 4 * lr) =
        make_float4(y0[0][jj], y0[1][jj], y0[2][jj], y0[3][jj]);
    if constexpr (GATED)
      *(float4*)(red + ((size_t)(kMnWaves + wave) * 16 + 4 * lq + jj) * kMnCols + 4 * lr) =
          make_float4(y1[0][jj], y1[1][jj], y1[2][jj], y1[3][jj]);
  }
  __syncthreads();
  const int gcol0 = (int)blockIdx.x * kMnCols;
  for (int i = tid; i < a.M * kMnCols; i += kMnThreads) {
    const int t = i / kMnCols, c = i - t * kMnCols;
    const int oc = c0 + c;
    if (oc < sg.N) {
      float v[kOut];
#pragma unroll
      for (int o = 0; o < kOut; ++o) {
        v[o] = 0.f;
#pragma unroll
        for (int ww = 0; ww < kMnWaves; ++ww) v[o] += red[((size_t)(o * kMnWaves + ww) * 16 + t) * kMnCols + c];
      }
      if (a.ks == 1)
        sg.C[(size_t)t * sg.N + oc] = f32_to_bf16(mn_out(v[0], v[kOut - 1], a.cap, GATED));
      else
#pragma unroll
        for (int o = 0; o < kOut; ++o)
          st_coherent_f32(a.part + (((size_t)slice * kOut + o) * a.M + t) * a.ntot + gcol0 + c, v[o]);
    }
  }
  if (a.ks == 1) return;
  // the last K slice to arrive for this column tile sums the partials in slice order
  __shared__ int last;
  wait_vmem();
  __syncthreads();
  if (tid == 0) last = atomic_add_relaxed(&a.ctr[blockIdx.x], 1) == a.ks - 1;
  __syncthreads();
  if (!last) return;
  for (int i = tid; i < a.M * kMnCols; i += kMnThreads) {
    const int t = i / kMnCols, c = i - t * kMnCols;
    const int oc = c0 + c;
    if (oc < sg.N) {
      float v[kOut];
#pragma unroll
      for (int o = 0; o < kOut; ++o) {
        v[o] = 0.f;
        for (int s2 = 0; s2 < a.ks; ++s2)
          v[o] += ld_coherent_f32(a.part + (((size_t)s2 * kOut + o) * a.M + t) * a.ntot + gcol0 + c);
      }
      sg.C[(size_t)t * sg.N + oc] = f32_to_bf16(mn_out(v[0], v[kOut - 1], a.cap, GATED));
    }
  }
  if (tid == 0) store_relaxed(&a.ctr[blockIdx.x], 0);
}

constexpr size_t kMnMaxLds = 150 * 1024;
constexpr int kMnKbw[] = {2, 4, 8, 12, 16, 24, 32};

// LDS of a launch: the slice's token rows, then (reused) the waves' sums
size_t mfma_narrow_lds(int M, int kbw, bool gated) {
  const size_t xs = (size_t)(M + 1) * kMnWaves * kbw * 4 * 16;
  const size_t red = (size_t)(gated ? 2 : 1) * kMnWaves * 16 * kMnCols * 4;
  return xs > red ? xs : red;
}

// k blocks per wave at most: twice the weights (gated) or twice the scales
// (group size 64) per wave would otherwise spill, and the slice's token rows
// must fit the LDS
int mn_max_kbw(int gs, bool gated, int M) {
  const int cap = gated ? 8 : (gs == 64 ? 16 : 32);
  int best = 0;
  for (int v : kMnKbw)
    if (v <= cap && mfma_narrow_lds(M, v, gated) <= kMnMaxLds) best = v;
  return best;
}

bool mfma_narrow_ok(int M, int K, int gs, bool gated) {
  return M >= 3 && M <= kMfMaxM && K % 32 == 0 && (gs == 64 || gs == 128) &&
         mn_max_kbw(gs, gated, M) >= gs / 32;
}

bool mfma_narrow_path(int M, int K, int N, int gs) {
  return mfma_narrow_ok(M, K, gs, false) && (size_t)(K / 8) * N * 4 < (1ull << 32);
}

template <int KBW, int KPG, bool G>
int launch_mfma_narrow_variant(const MnArgs& k, int tiles, size_t lds, hipStream_t stream) {
  static bool attr_set[64];
  int dev = 0;
  hipError_t e0 = hipGetDevice(&dev);
  if (e0 != hipSuccess) return hip_fail(e0, "hipGetDevice");
  if (dev >= 0 && dev < 64 && !attr_set[dev]) {
    e0 = hipFuncSetAttribute((const void*)w4a16_mfma_narrow_kernel<KBW, KPG, G>,
                             hipFuncAttributeMaxDynamicSharedMemorySize, (int)kMnMaxLds);
    if (e0 != hipSuccess) return hip_fail(e0, "hipFuncSetAttribute(max dynamic LDS)");
    attr_set[dev] = true;
  }
  hipLaunchKernelGGL((w4a16_mfma_narrow_kernel<KBW, KPG, G>), dim3((unsigned)tiles, (unsigned)k.ks),
                     dim3(kMnThreads), lds, stream, k);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? GI_OK : hip_fail(e, "w4a16 matrix-core narrow launch");
}

// K split of the matrix-core narrow path: enough slices that the grid has
// about kMnTargetWgs workgroups, each wave at least one scale group of k blocks.
constexpr int kMnTargetWgs = 256;
struct MnPlan {
  int kbw, ks;
};
MnPlan mn_plan(int M, int K, int tiles, int gs, bool gated) {
  const int KB = K / 32, kpg = gs / 32;
  const int ks_want = (kMnTargetWgs + tiles - 1) / tiles;
  const int per_slice = (KB + ks_want - 1) / ks_want;
  const int need = (per_slice + kMnWaves - 1) / kMnWaves;  // k blocks per wave
  const int vmax = mn_max_kbw(gs, gated, M);
  MnPlan p{vmax, 1};
  for (int v : kMnKbw)
    if (v >= need && v >= kpg && v <= vmax) {
      p.kbw = v;
      break;
    }
  p.ks = (KB + kMnWaves * p.kbw - 1) / (kMnWaves * p.kbw);
  return p;
}
int mn_tiles(const int* N, int n) {
  int t = 0;
  for (int i = 0; i < n; ++i) t += (N[i] + kMnCols - 1) / kMnCols;
  return t;
}
size_t mn_workspace_bytes(int M, int K, int tiles, int gs, bool gated) {
  const MnPlan p = mn_plan(M, K, tiles, gs, gated);
  return p.ks > 1 ? round_up(kCtrBytes + (size_t)p.ks * (gated ? 2 : 1) * M * tiles * kMnCols * sizeof(float)) : 0;
}

// segs: the projections (for gated: gate then up, same N); caller checked
// mfma_narrow_ok and the 32-bit offsets of every segment.
int launch_mfma_narrow(const void* A, int M, int K, int gs, float cap, const NarrowSeg* segs, int nseg, bool gated,
                       void* workspace, size_t workspace_bytes, hipStream_t stream) {
  MnArgs k{};
  k.A = (const uint16_t*)A;
  k.M = M;
  k.K = K;
  k.cap = cap;
  int tiles = 0;
  for (int i = 0; i < nseg; ++i) {
    k.seg[i] = segs[i];
    k.seg[i].tile0 = gated ? 0 : tiles;
    if (!gated) tiles += (segs[i].N + kMnCols - 1) / kMnCols;
  }
  if (gated) tiles = (segs[0].N + kMnCols - 1) / kMnCols;
  for (int i = nseg; i < kMaxSegs; ++i) k.seg[i].tile0 = 0x7fffffff;
  k.ntot = tiles * kMnCols;
  const MnPlan p = mn_plan(M, K, tiles, gs, gated);
  k.ks = p.ks;
  if (p.ks > 1) {
    if ((size_t)tiles * sizeof(int) > kCtrBytes)
      return fail(GI_ERR_UNSUPPORTED, "w4a16: N too large for the split matrix-core path");
    if (!workspace || workspace_bytes < mn_workspace_bytes(M, K, tiles, gs, gated) ||
        ((uintptr_t)workspace) % kAlign)
      return fail(GI_ERR_WORKSPACE, "w4a16: workspace missing, misaligned or smaller than the workspace query");
    k.ctr = (int*)workspace;
    k.part = (float*)((char*)workspace + kCtrBytes);
  }
  const size_t lds = mfma_narrow_lds(M, p.kbw, gated);
  const int kpg = gs / 32;
  switch ((gated ? 10000 : 0) + p.kbw * 10 + kpg) {
#define GI_MN_CASE(G, KBW, KPG)                      \
  case (G ? 10000 : 0) + KBW * 10 + KPG:            \
    return launch_mfma_narrow_variant<KBW, KPG, G>(k, tiles, lds, stream);
    GI_MN_CASE(false, 2, 2) GI_MN_CASE(false, 4, 2) GI_MN_CASE(false, 8, 2) GI_MN_CASE(false, 12, 2)
    GI_MN_CASE(false, 16, 2) GI_MN_CASE(false, 4, 4) GI_MN_CASE(false, 8, 4) GI_MN_CASE(false, 12, 4)
    GI_MN_CASE(false, 16, 4) GI_MN_CASE(false, 24, 4) GI_MN_CASE(false, 32, 4)
    GI_MN_CASE(true, 2, 2) GI_MN_CASE(true, 4, 2) GI_MN_CASE(true, 8, 2) GI_MN_CASE(true, 4, 4)
    GI_MN_CASE(true, 8, 4)
#undef GI_MN_CASE
    default:
      return fail(GI_ERR_UNSUPPORTED, "w4a16: no matrix-core narrow variant for this shape");
  }
}

bool mfma_path(int M, int K, int N, int gs, int G) {
  // wide N (lm_head): the matrix cores stream best from one row up (rows past
  // M are zero operand rows)
  if (M < 1 || M > kMfMaxM || K % 32 || (gs != 64 && gs != 128) || N % kMfCols || N / kMfCols < 256) return false;
  // 32-bit buffer offsets, including reads past the last row of a pass
  const long long kb_pad = (long long)(K / 32 + kMfPass - 1) / kMfPass * kMfPass;
  if (kb_pad * 4 * N * 4 >= (1LL << 32)) return false;
  // 32-bit offsets into the scales (one workgroup's columns over all groups)
  if ((long long)G * N * 2 >= (1LL << 32)) return false;
  const size_t lds = (size_t)(M + 1) * (K / 8) * 16 + (size_t)G * (kMfCols / 4) * 8;
  static_assert((size_t)kMfXChunks * 16 >= 64 * 1024, "the x rows fit one staging batch");
  return lds <= 64 * 1024;
}


struct Plan {
  int ks, rows_per_split, tiles, nt;
  size_t ctr_off, part_off, total;
};

constexpr int kGemvSteps[] = {1, 2, 3, 4, 6, 8, 12};

Plan make_plan(int M, int K, int N) {
  Plan p;
  const int Kp = K >> 3;
  p.tiles = (N + kCols - 1) / kCols;
  if (M <= 8) {  // decode-shape path: S steps of 16 packed rows per K slice
    p.nt = M <= 1 ? 1 : M <= 2 ? 2 : M <= 4 ? 4 : 8;
    int steps = kGemvSteps[6];
    for (int st : kGemvSteps) {
      const int ks = (Kp + st * kRowsPerStep - 1) / (st * kRowsPerStep);
      if ((long)p.tiles * ks <= kGemvTargetWgs) {
        steps = st;
        break;
      }
    }
    p.rows_per_split = steps * kRowsPerStep;
    p.ks = (Kp + p.rows_per_split - 1) / p.rows_per_split;
    p.ctr_off = 0;
    p.part_off = kCtrBytes;
    p.total = p.ks > 1 ? round_up(p.part_off + (size_t)p.ks * M * N * sizeof(float)) : 0;
    return p;
  }
  p.nt = M <= 1 ? 1 : (M <= 4 ? 4 : 8);
  int ks = (kTargetWgs + p.tiles - 1) / p.tiles;
  const int max_ks = (Kp + kRowsPerStep - 1) / kRowsPerStep;
  if (ks > max_ks) ks = max_ks;
  if (ks < 1) ks = 1;
  // rows per split: a whole number of 16-row steps
  int rps = (Kp + ks - 1) / ks;
  rps = (rps + kRowsPerStep - 1) / kRowsPerStep * kRowsPerStep;
  ks = (Kp + rps - 1) / rps;
  // x staging must fit in 64 KB of LDS
  while ((size_t)p.nt * rps * (sizeof(uint4) + sizeof(float)) > 56 * 1024 && rps > kRowsPerStep) {
    ks *= 2;
    rps = (Kp + ks - 1) / ks;
    rps = (rps + kRowsPerStep - 1) / kRowsPerStep * kRowsPerStep;
    ks = (Kp + rps - 1) / rps;
  }
  p.ks = ks;
  p.rows_per_split = rps;
  p.ctr_off = 0;
  p.part_off = kCtrBytes;
  p.total = ks > 1 ? round_up(p.part_off + (size_t)ks * M * N * sizeof(float)) : 0;
  return p;
}

}  // namespace

size_t w4a16_workspace_bytes(int M, int K, int N, int gs) {
  if (M <= 0 || K <= 0 || N <= 0) return 0;
  if (narrow_path(M, K, N)) return 0;
  if (gs > 0 && mfma_narrow_path(M, K, N, gs))
    return mn_workspace_bytes(M, K, (N + kMnCols - 1) / kMnCols, gs, false);
  // the matrix-core path needs none (scales with the full ceil(K / gs) groups)
  if (gs > 0 && mfma_path(M, K, N, gs, (K + gs - 1) / gs)) return 0;
  return make_plan(M, K, N).total;
}

int launch_w4a16(const void* A, const int32_t* B, const void* scales, int n_groups, void* C,
                 int M, int K, int N, int gs, float softcap, void* workspace,
                 size_t workspace_bytes, hipStream_t stream) {
  if (M < 0 || K <= 0 || N <= 0) return fail(GI_ERR_INVALID_ARG, "w4a16: K and N must be positive, M >= 0");
  if (K % 8) return fail(GI_ERR_INVALID_ARG, "w4a16: K must be a multiple of 8 (8 codes per int32)");
  if (N % 4) return fail(GI_ERR_UNSUPPORTED, "w4a16: N must be a multiple of 4");
  if (gs <= 0 || gs % 8) return fail(GI_ERR_INVALID_ARG, "w4a16: group_size must be a positive multiple of 8");
  if (n_groups <= 0) return fail(GI_ERR_INVALID_ARG, "w4a16: scales need at least one group");
  if (!A || !B || !scales || !C) return fail(GI_ERR_INVALID_ARG, "w4a16: null tensor pointer");
  if ((((uintptr_t)A) | ((uintptr_t)B)) % 16)
    return fail(GI_ERR_INVALID_ARG, "w4a16: A and B_packed must be 16-byte aligned");
  if (((uintptr_t)scales) % 8) return fail(GI_ERR_INVALID_ARG, "w4a16: scales must be 8-byte aligned");
  if (M == 0) return GI_OK;
  if (mfma_path(M, K, N, gs, n_groups)) {
    MfArgs k{};
    k.A = (const uint16_t*)A;
    k.B = B;
    k.S = (const uint16_t*)scales;
    k.C = (uint16_t*)C;
    k.M = M;
    k.K = K;
    k.N = N;
    k.G = n_groups;
    k.b_bytes = (uint32_t)((size_t)(K / 8) * N * 4);
    k.cap = softcap;
    // 8 waves (512 columns) where N and LDS allow, else 4 (256 columns)
    const size_t xl = (size_t)(M + 1) * (K / 8) * 16;
    const size_t lds8 = xl + (size_t)n_groups * (2 * kMfCols / 4) * 8;
    const bool w8 = N % (2 * kMfCols) == 0 && lds8 <= 64 * 1024;
    const size_t lds = w8 ? lds8 : xl + (size_t)n_groups * (kMfCols / 4) * 8;
    const dim3 grid(N / (w8 ? 2 * kMfCols : kMfCols)), block(w8 ? 2 * kMfThreads : kMfThreads);
    if (gs == 64) {
      if (w8) hipLaunchKernelGGL((w4a16_mfma_kernel<2, 8>), grid, block, lds, stream, k);
      else hipLaunchKernelGGL((w4a16_mfma_kernel<2, 4>), grid, block, lds, stream, k);
    } else {
      if (w8) hipLaunchKernelGGL((w4a16_mfma_kernel<4, 8>), grid, block, lds, stream, k);
      else hipLaunchKernelGGL((w4a16_mfma_kernel<4, 4>), grid, block, lds, stream, k);
    }
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_fail(e, "w4a16 matrix-core launch");
    return GI_OK;
  }
  if (mfma_narrow_path(M, K, N, gs)) {
    const NarrowSeg sg{B, (const uint16_t*)scales, (uint16_t*)C, N, n_groups, 0};
    return launch_mfma_narrow(A, M, K, gs, softcap, &sg, 1, false, workspace, workspace_bytes, stream);
  }
  if (narrow_path(M, K, N)) {
    NarrowSeg sg{B, (const uint16_t*)scales, (uint16_t*)C, N, n_groups, 0};
    return launch_narrow(A, M, K, gs, softcap, &sg, 1, false, stream);
  }
  const Plan p = make_plan(M, K, N);
  if (p.ks > 1 && (size_t)p.tiles * sizeof(int) > kCtrBytes)
    return fail(GI_ERR_UNSUPPORTED, "w4a16: N too large for the split-K path (N <= 1048576)");
  if (p.ks > 1) {
    if (!workspace || workspace_bytes < p.total)
      return fail(GI_ERR_WORKSPACE, "w4a16: workspace missing or smaller than gi_w4a16_workspace_bytes()");
    if (((uintptr_t)workspace) % kAlign)
      return fail(GI_ERR_WORKSPACE, "w4a16: workspace must be 256-byte aligned");
  }
  GemvArgs k{};
  k.A = (const uint16_t*)A;
  k.B = B;
  k.S = (const uint16_t*)scales;
  k.C = (uint16_t*)C;
  k.ctr = p.ks > 1 ? (int*)((char*)workspace + p.ctr_off) : nullptr;
  k.part = p.ks > 1 ? (float*)((char*)workspace + p.part_off) : nullptr;
  k.M = M;
  k.K = K;
  k.N = N;
  k.gs = gs;
  k.G = n_groups;
  k.ks = p.ks;
  k.rows_per_split = p.rows_per_split;
  k.stage_stride = p.rows_per_split;
  k.cap = softcap;
  const dim3 grid(p.tiles, p.ks);
  if (M <= 8) {
    const int steps = p.rows_per_split / kRowsPerStep;
    switch (p.nt * 100 + steps) {
#define GI_GEMV_CASE(NT, S)                                                                    \
  case NT * 100 + S:                                                                           \
    hipLaunchKernelGGL((w4a16_gemv_kernel<NT, S>), grid, dim3(kThreads), 0, stream, k); \
    break;
#define GI_GEMV_NT(NT) GI_GEMV_CASE(NT, 1) GI_GEMV_CASE(NT, 2) GI_GEMV_CASE(NT, 3) GI_GEMV_CASE(NT, 4) \
  GI_GEMV_CASE(NT, 6) GI_GEMV_CASE(NT, 8) GI_GEMV_CASE(NT, 12)
      GI_GEMV_NT(1)
      GI_GEMV_NT(2)
      GI_GEMV_NT(4)
      GI_GEMV_NT(8)
#undef GI_GEMV_NT
#undef GI_GEMV_CASE
      default:
        return fail(GI_ERR_UNSUPPORTED, "w4a16: no decode-shape variant for this plan");
    }
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_fail(e, "w4a16 launch");
    return GI_OK;
  }
  const size_t dyn = (size_t)p.nt * p.rows_per_split * (sizeof(uint4) + sizeof(float));
  if (p.nt == 1) hipLaunchKernelGGL(w4a16_kernel<1>, grid, dim3(kThreads), dyn, stream, k);
  else if (p.nt == 4) hipLaunchKernelGGL(w4a16_kernel<4>, grid, dim3(kThreads), dyn, stream, k);
  else hipLaunchKernelGGL(w4a16_kernel<8>, grid, dim3(kThreads), dyn, stream, k);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return hip_fail(e, "w4a16 launch");
  return GI_OK;
}

// ---- several projections of one input, and the gated MLP --------------------
namespace {

int check_linear(const void* A, const int32_t* B, const void* scales, int n_groups, const void* C, int M, int K,
                 int N, int gs, const char* who) {
  if (M < 0 || K <= 0 || N <= 0) return fail(GI_ERR_INVALID_ARG, std::string(who) + ": K, N > 0 and M >= 0 required");
  if (K % 8 || N % 4) return fail(GI_ERR_INVALID_ARG, std::string(who) + ": K % 8 == 0 and N % 4 == 0 required");
  if (gs <= 0 || gs % 8 || n_groups <= 0)
    return fail(GI_ERR_INVALID_ARG, std::string(who) + ": bad group size or group count");
  if (!A || !B || !scales || !C) return fail(GI_ERR_INVALID_ARG, std::string(who) + ": null tensor pointer");
  if ((((uintptr_t)A) | ((uintptr_t)B)) % 16 || ((uintptr_t)scales) % 8)
    return fail(GI_ERR_INVALID_ARG, std::string(who) + ": A/B_packed 16-byte and scales 8-byte alignment required");
  return GI_OK;
}

bool narrow_multi(int M, int K, const int* N, int n) {
  if (M > 2 || K / 8 > 64 * 16) return false;
  long total = 0;
  for (int i = 0; i < n; ++i) {
    if (narrow_rows(K / 8) * N[i] * 4 >= (1ull << 32)) return false;
    total += N[i];
  }
  return total >= 1024;
}

__global__ __launch_bounds__(256) void gelu_mul_kernel(const uint16_t* g, const uint16_t* u, uint16_t* out, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    const float gl = round_to_bf16(gelu_tanh(bf16_to_f32(g[i])));
    out[i] = f32_to_bf16(gl * bf16_to_f32(u[i]));
  }
}

size_t gated_tmp_off(int M, int K, int N) { return round_up(make_plan(M, K, N).total); }

bool mfma_multi(int M, int K, const int* N, int n, int gs) {
  if (!mfma_narrow_ok(M, K, gs, false)) return false;
  for (int i = 0; i < n; ++i)
    if ((size_t)(K / 8) * N[i] * 4 >= (1ull << 32)) return false;
  return true;
}

bool gated_narrow(int M, int K, int N) {
  return M <= 2 && K / 8 <= 64 * 16 && narrow_rows(K / 8) * N * 4 < (1ull << 32);
}
bool gated_mfma(int M, int K, int N, int gs) {
  return mfma_narrow_ok(M, K, gs, true) && (size_t)(K / 8) * N * 4 < (1ull << 32);
}

}  // namespace

int launch_w4a16_multi(const void* A, int n, const int32_t* const* B, const void* const* scales, const int* n_groups,
                       void* const* C, const int* N, int M, int K, int gs, void* workspace, size_t workspace_bytes,
                       hipStream_t stream) {
  if (n <= 0 || n > kMaxSegs) return fail(GI_ERR_INVALID_ARG, "w4a16_multi: 1 to 4 projections");
  if (!B || !scales || !n_groups || !C || !N) return fail(GI_ERR_INVALID_ARG, "w4a16_multi: null array");
  for (int i = 0; i < n; ++i) {
    const int st = check_linear(A, B[i], scales[i], n_groups[i], C[i], M, K, N[i], gs, "w4a16_multi");
    if (st != GI_OK) return st;
  }
  if (M == 0) return GI_OK;
  NarrowSeg sg[kMaxSegs];
  for (int i = 0; i < n; ++i) sg[i] = NarrowSeg{B[i], (const uint16_t*)scales[i], (uint16_t*)C[i], N[i], n_groups[i], 0};
  if (narrow_multi(M, K, N, n)) return launch_narrow(A, M, K, gs, 0.f, sg, n, false, stream);
  if (mfma_multi(M, K, N, n, gs))
    return launch_mfma_narrow(A, M, K, gs, 0.f, sg, n, false, workspace, workspace_bytes, stream);
  for (int i = 0; i < n; ++i) {
    const int st = launch_w4a16(A, B[i], scales[i], n_groups[i], C[i], M, K, N[i], gs, 0.f, workspace,
                                workspace_bytes, stream);
    if (st != GI_OK) return st;
  }
  return GI_OK;
}

size_t w4a16_multi_workspace_bytes(int n, const int* N, int M, int K, int gs) {
  if (n <= 0 || n > kMaxSegs || !N || M <= 0 || K <= 0) return 0;
  if (narrow_multi(M, K, N, n)) return 0;
  if (gs > 0 && mfma_multi(M, K, N, n, gs)) return mn_workspace_bytes(M, K, mn_tiles(N, n), gs, false);
  size_t b = 0;
  for (int i = 0; i < n; ++i) {
    const size_t x = w4a16_workspace_bytes(M, K, N[i], gs);
    if (x > b) b = x;
  }
  return b;
}

size_t w4a16_gated_workspace_bytes(int M, int K, int N, int gs) {
  if (M <= 0 || K <= 0 || N <= 0) return 0;
  if (gated_narrow(M, K, N)) return 0;
  if (gs > 0 && gated_mfma(M, K, N, gs)) return mn_workspace_bytes(M, K, (N + kMnCols - 1) / kMnCols, gs, true);
  return gated_tmp_off(M, K, N) + 2 * round_up((size_t)M * N * 2);
}

int launch_w4a16_gated(const void* A, const int32_t* gB, const void* gS, int gG, const int32_t* uB, const void* uS,
                       int uG, void* out, int M, int K, int N, int gs, void* workspace, size_t workspace_bytes,
                       hipStream_t stream) {
  int st = check_linear(A, gB, gS, gG, out, M, K, N, gs, "w4a16_gated_mlp");
  if (st != GI_OK) return st;
  st = check_linear(A, uB, uS, uG, out, M, K, N, gs, "w4a16_gated_mlp");
  if (st != GI_OK) return st;
  if (M == 0) return GI_OK;
  const NarrowSeg sg[2] = {NarrowSeg{gB, (const uint16_t*)gS, (uint16_t*)out, N, gG, 0},
                           NarrowSeg{uB, (const uint16_t*)uS, nullptr, N, uG, 0}};
  if (gated_narrow(M, K, N)) return launch_narrow(A, M, K, gs, 0.f, sg, 2, true, stream);
  if (gated_mfma(M, K, N, gs))
    return launch_mfma_narrow(A, M, K, gs, 0.f, sg, 2, true, workspace, workspace_bytes, stream);
  const size_t need = w4a16_gated_workspace_bytes(M, K, N, gs);
  if (!workspace || workspace_bytes < need || ((uintptr_t)workspace) % kAlign)
    return fail(GI_ERR_WORKSPACE, "w4a16_gated_mlp: workspace missing, misaligned or smaller than "
                                  "gi_w4a16_gated_mlp_workspace_bytes()");
  uint16_t* tg = (uint16_t*)((char*)workspace + gated_tmp_off(M, K, N));
  uint16_t* tu = (uint16_t*)((char*)tg + round_up((size_t)M * N * 2));
  st = launch_w4a16(A, gB, gS, gG, tg, M, K, N, gs, 0.f, workspace, workspace_bytes, stream);
  if (st != GI_OK) return st;
  st = launch_w4a16(A, uB, uS, uG, tu, M, K, N, gs, 0.f, workspace, workspace_bytes, stream);
  if (st != GI_OK) return st;
  const int64_t n = (int64_t)M * N;
  const int blocks = (int)((n + 255) / 256 < 4096 ? (n + 255) / 256 : 4096);
  hipLaunchKernelGGL(gelu_mul_kernel, dim3(blocks), dim3(256), 0, stream, tg, tu, (uint16_t*)out, n);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? GI_OK : hip_fail(e, "w4a16_gated_mlp launch");
}

}  // namespace gi
