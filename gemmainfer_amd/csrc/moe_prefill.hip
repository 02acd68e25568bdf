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
//   front    one launch: routing (layer mode, 16 tokens per workgroup); the
//            align in the last routing workgroup to finish (per-expert
//            counts, offsets, the pairs of each expert (pos -> pair) and the
//            inverse map (pair -> pos)); beside them the reorder of x into the
//            matrix-core k order
//   gate/up  grid (I/128 column tiles, E): 16-token row tiles of the expert's
//            pairs (A = gathered x rows) times the unpacked int4 words (B),
//            v_mfma_f32_16x16x32_bf16, 48 pairs per pass; act =
//            bf16(gelu_tanh(gate) * up) (marlin.cu:414-423)
//   down     grid (H/256 column units, E): the same over the act rows, fp32
//            results per pair
//   combine  one workgroup per token: out[t] (+)= sum over its slots in slot
//            order of w * y, the weights rounded to bf16 (marlin.cu:631-636),
//            one bf16 rounding of the sum (the reference adds bf16 atomics,
//            marlin.cu:583; the order here is fixed)
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
constexpr int kPThreads = 256;  // 4 waves x 64 columns
constexpr int kPRT = 3;         // 16-token row tiles per pass
constexpr int kAlignThreads = 1024;
constexpr uint32_t kOob = 0xFFFFFFF0u;

struct PfArgs {
  const uint16_t* x;
  uint16_t* xk;        // [M][H] x with each 8-value chunk in the matrix-core k order
  const int32_t* gu;
  const uint16_t* gus;
  const int32_t* dn;
  const uint16_t* dns;
  const int* offsets;  // [E + 1] first position of each expert
  const int* order;    // [P] pair at each position
  uint16_t* act;       // [P][I] bf16, positions in expert order, chunks in k order
  float* y;            // [P][H] fp32, row = pair index
  int M, H, I, E, top_k, Ggu, Gd, gsh;  // group size = 32 << gsh
  uint32_t x_bytes, gu_bytes, gu_total, dn_bytes, dn_total, act_bytes;
};

// Router inputs of the front launch (the fields the shared routing reads).
struct PfRoute {
  const void* logits;
  int logits_dtype;
  const float* expert_scale;
  int M, E, top_k;
};

// ---------------------------------------------------------------------------
// align (one workgroup of kAlignThreads)
// ---------------------------------------------------------------------------
constexpr int kAlignPer = 8;  // pairs per thread kept in registers

// Per-expert offsets [E + 1] and the pairs of each expert (order: pos ->
// pair; ids outside [0, E) are skipped as at marlin.cu:288-289); load_id(p)
// reads pair p's id.
struct AlignLds {
  int cnt[1024];
  int fill[1024];
  int wsum[kAlignThreads / kWave];
};
template <class LoadId>
__device__ __forceinline__ void align_block(LoadId load_id, int P, int E, int* offsets, int* order, AlignLds& s) {
  const int tid = threadIdx.x;
  for (int e = tid; e < E; e += kAlignThreads) {
    s.cnt[e] = 0;
    s.fill[e] = 0;
  }
  __syncthreads();
  // Up to kAlignPer pairs per thread: every id is loaded once, up front
  // (indices clamped to the last pair, so no load sits under a per-lane
  // condition), and both passes below reuse the registers.
  const bool cached = P > 0 && P <= kAlignThreads * kAlignPer;
  int ev[kAlignPer];
  if (cached) {
#pragma unroll
    for (int i = 0; i < kAlignPer; ++i) {
      const int p = tid + kAlignThreads * i;
      ev[i] = load_id(p < P ? p : P - 1);
      if (p >= P) ev[i] = -1;
    }
#pragma unroll
    for (int i = 0; i < kAlignPer; ++i)
      if (ev[i] >= 0 && ev[i] < E) atomicAdd(&s.cnt[ev[i]], 1);
  } else {
    for (int p = tid; p < P; p += kAlignThreads) {
      const int e = load_id(p);
      if (e >= 0 && e < E) atomicAdd(&s.cnt[e], 1);
    }
  }
  __syncthreads();
  // exclusive scan of the counts (E <= 1024: one expert per thread)
  const int lane = tid & (kWave - 1), wave = tid >> 6;
  const int c = tid < E ? s.cnt[tid] : 0;
  int incl = c;
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const int v = __shfl_up(incl, off, kWave);
    if (lane >= off) incl += v;
  }
  if (lane == kWave - 1) s.wsum[wave] = incl;
  __syncthreads();
  int base = 0;
  for (int w2 = 0; w2 < wave; ++w2) base += s.wsum[w2];
  const int excl = base + incl - c;
  if (tid < E) {
    offsets[tid] = excl;
    s.cnt[tid] = excl;
  }
  if (tid == E - 1) offsets[E] = excl + c;
  __syncthreads();
  if (cached) {
#pragma unroll
    for (int i = 0; i < kAlignPer; ++i) {
      const int p = tid + kAlignThreads * i;
      if (p < P) {
        const int e = ev[i];
        if (e >= 0 && e < E) order[s.cnt[e] + atomicAdd(&s.fill[e], 1)] = p;
      }
    }
    return;
  }
  for (int p = tid; p < P; p += kAlignThreads) {
    const int e = load_id(p);
    if (e >= 0 && e < E) order[s.cnt[e] + atomicAdd(&s.fill[e], 1)] = p;
  }
}

// ---------------------------------------------------------------------------
// front launch: routing, align and the x reorder in one launch
// ---------------------------------------------------------------------------
struct PfFront {
  PfRoute r;
  int nroute;            // routing workgroups (0: the caller gave the ids)
  int32_t* out_idx;      // routed ids (int32)
  uint16_t* out_w;       // routed weights (bf16, marlin.cu:631-636)
  const void* idx;       // the ids the align reads (the routed ones, or the caller's)
  int idx_is64, P;
  int* offsets;          // [E + 1]
  int* order;            // [P]
  int* arrive;           // arrivals of the routing workgroups (zero between launches)
  const uint4* x;
  uint4* xk;             // x with each 8-value chunk in the matrix-core k order
  int nx;                // 16-byte chunks of x
};

// Workgroups [0, nroute) route 16 tokens each (one wave per token) and the
// last of them to finish runs the align over every routed id; with the ids
// from the caller, workgroup 0 runs the align.  The other workgroups reorder
// x (one pass instead of a reorder per product operand), one 16-byte chunk
// per thread, beside them.  The routed ids are handed to the aligning
// workgroup through the device coherence point: agent-scope stores, each
// wave's stores complete before the workgroup barrier and the arrival, and
// agent-scope loads after it.
__global__ __launch_bounds__(kAlignThreads) void prefill_front_kernel(PfFront f) {
  __shared__ AlignLds als;
  __shared__ int r_idx[kAlignThreads / kWave][64];
  __shared__ float r_w[kAlignThreads / kWave][64];
  __shared__ int last;
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid >> 6;
  const int nlead = f.nroute > 0 ? f.nroute : 1;
  if ((int)blockIdx.x >= nlead) {
    const int i = (blockIdx.x - nlead) * kAlignThreads + tid;
    if (i < f.nx) f.xk[i] = moe::mfma_k_order(f.x[i]);
    return;
  }
  const int E = f.r.E;
  if (f.nroute == 0) {
    align_block([&](int p) { return load_expert_id(f.idx, f.idx_is64, p); }, f.P, E, f.offsets, f.order, als);
    return;
  }
  const int t = blockIdx.x * (kAlignThreads / kWave) + wave;
  if (t < f.r.M) {
    moe::route_token_any(f.r, t, lane, r_idx[wave], r_w[wave]);
    if (lane < f.r.top_k) {
      const int s = t * f.r.top_k + lane;
      __hip_atomic_store(f.out_idx + s, r_idx[wave][lane], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      f.out_w[s] = f32_to_bf16(r_w[wave][lane]);
    }
  }
  wait_vmem();
  __syncthreads();
  if (tid == 0) last = atomic_add_relaxed(f.arrive, 1) == f.nroute - 1;
  __syncthreads();
  if (!last) return;
  if (tid == 0) store_relaxed(f.arrive, 0);  // every routing workgroup has arrived: zero for the next launch
  const int32_t* ids = f.out_idx;
  align_block([&](int p) { return __hip_atomic_load(ids + p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }, f.P, E,
              f.offsets, f.order, als);
}

// ---------------------------------------------------------------------------
// grouped products (gate/up and down share the structure)
// ---------------------------------------------------------------------------
// A workgroup of 4 waves owns 256 output columns of one expert over all of K;
// wave w owns 64 of them: lane (lq, lr) loads the 16 bytes of columns
// 4lr..4lr+3 at packed row 4kb + lq, the B operands of four 16-column
// products.  Each 16-token row tile of the expert's pairs is one A operand
// (16 bytes of the lane's token row at k 32kb + 8lq .. +7; the rows are
// stored in the operand's k order).  Every wave needs the same A operands, so
// wave rt (< kPRT) loads row tile rt and stages it through LDS, kPChunk k
// blocks at a time (one barrier per chunk), instead of each wave loading all
// of them.  Words stream through a register ring kPChunk k blocks ahead (loads
// past K read an offset past the resource: zeros, no memory access).  No
// cross-wave reduction: every wave covers all of K.
constexpr int kPRingGu = 8;  // weight k blocks in flight per wave, gate/up (bounded by registers)
constexpr int kPRingDn = 8;  // the same, down
constexpr int kPChunk = 8;   // k blocks of A tiles staged in LDS per barrier (two chunk buffers)

// 16 bytes of a lane's row at k block kb (zeros past the expert's pairs or
// past K: offset past the resource).
__device__ __forceinline__ uint4 row_operand(__amdgpu_buffer_rsrc_t r, uint32_t row_off, int kb, int lq) {
  const uint32_t off = row_off == kOob ? kOob : row_off + (uint32_t)(32 * kb + 8 * lq) * 2u;
  const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
  return make_uint4(v.x, v.y, v.z, v.w);
}

// The products of one wave over k blocks [0, KB): y[rt][q] (rows 4lq + jj of
// row tile rt, column 4lr + q of the wave's 64) = sum over groups of
// scale * (D + Db).  Weights: rw/wbase (+ kb * wstep), activations: ra with
// this wave's own row tile offset (waves < kPRT), scales:
// sc_lds[g * 64 + 16 w + lr] (4 bf16; groups past G scale by zero), aring:
// two chunk buffers [2][kPChunk][kPRT][64] uint4.  The group size (32 <<
// GSH) is a compile-time value, so every group end inside a chunk is known to
// the compiler (a chunk holds whole groups); a last partial group is finished
// at K.  The first RT row tiles are multiplied (rows past the expert's pairs
// are zeros): RT is a compile-time value, so the loop has no branch on the
// tile count (a branch inside it split the scheduling region: slower).
template <int kPRing, int GSH, int RT>
__device__ __forceinline__ void grouped_products(__amdgpu_buffer_rsrc_t rw, uint32_t wbase, uint32_t wstep,
                                                 uint32_t wsoff, __amdgpu_buffer_rsrc_t ra, uint32_t roff_own,
                                                 int KB, int G, const uint2* sc_lds, uint4* aring,
                                                 f32x4_t (&y)[kPRT][4]) {
  constexpr int kKbpg = 1 << GSH;
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x >> 6;
  const int lq = lane >> 4, lr = lane & 15;
  const bool loader = wave < RT;
  const uint32_t mq = q4_magic();
  const f32x4_t zf = {0.f, 0.f, 0.f, 0.f};
  const uint4 bc = make_uint4(moe::kQ4BiasPair, moe::kQ4BiasPair, moe::kQ4BiasPair, moe::kQ4BiasPair);
  auto own = [&](int kb) { return kb < KB ? roff_own : kOob; };
  // the expert's offset joins the per-lane offset (no scalar offset beside
  // an out-of-range one, which could wrap into range); wbase == kOob marks a
  // wave with no columns
  const bool wlive = wbase != kOob;
  const uint32_t wb = wbase + wsoff;
  auto wload = [&](int kb) {
    const u32x4_t v =
        __builtin_amdgcn_raw_buffer_load_b128(rw, (wlive && kb < KB) ? wb + (uint32_t)kb * wstep : kOob, 0, 2);
    return make_uint4(v.x, v.y, v.z, v.w);
  };
  f32x4_t D[kPRT][4], Db[kPRT];
  auto epilogue = [&](int g) {
    const uint2 sv = g < G ? sc_lds[g * 64 + 16 * wave + lr] : make_uint2(0u, 0u);
    const float sc[4] = {bf16lo(sv.x), bf16hi(sv.x), bf16lo(sv.y), bf16hi(sv.y)};
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) y[rt][q][jj] += sc[q] * (D[rt][q][jj] + Db[rt][jj]);
  };
#pragma unroll
  for (int rt = 0; rt < kPRT; ++rt)
#pragma unroll
    for (int q = 0; q < 4; ++q) y[rt][q] = zf;
  static_assert(kPChunk % kKbpg == 0 && kPRing == kPChunk, "chunks hold whole groups; one ring slot per k block");
  auto abuf = [&](int c, int j, int rt) -> uint4& { return aring[(((c & 1) * kPChunk + j) * kPRT + rt) * 64 + lane]; };
  // A tiles stream through LDS a chunk of kPChunk k blocks at a time (one
  // barrier per chunk): loader wave rt keeps the next chunk of its row tile
  // in registers and writes it into the free chunk buffer.  The chunk loop is
  // a real loop (its body fits the instruction cache); inside it every ring
  // and buffer index is a compile-time value.
  uint4 wr[kPRing], ar[kPChunk];
  const int nch = (KB + kPChunk - 1) / kPChunk;
  __syncthreads();  // the previous call's readers of the chunk buffers are done
  // issue order: the first chunk's A tiles, the weight ring, the next chunk's
  // A tiles; the first chunk is written to LDS as soon as it lands (the
  // weight ring is not waited for there: its latency overlaps the A tiles')
  uint4 a0[kPChunk];
  if (loader) {
#pragma unroll
    for (int j = 0; j < kPChunk; ++j) a0[j] = row_operand(ra, own(j), j, lq);
  }
#pragma unroll
  for (int s = 0; s < kPRing; ++s) wr[s] = wload(s);
  if (loader) {
#pragma unroll
    for (int j = 0; j < kPChunk; ++j) ar[j] = row_operand(ra, own(kPChunk + j), kPChunk + j, lq);
#pragma unroll
    for (int j = 0; j < kPChunk; ++j) abuf(0, j, wave) = a0[j];
  }
  if (!wlive) {
    // a wave with no columns (the last column tile when I is not a multiple
    // of 128): its share of the A staging and the barriers, no products
    // (the issue slots go to the other waves of its SIMD); y stays zero
#pragma unroll 1
    for (int c = 0; c < nch; ++c) {
      lds_barrier();
      if (loader) {
        const int kn = (c + 2) * kPChunk;
#pragma unroll
        for (int j = 0; j < kPChunk; ++j) {
          abuf(c + 1, j, wave) = ar[j];
          ar[j] = row_operand(ra, own(kn + j), kn + j, lq);
        }
      }
    }
    return;
  }
#pragma unroll 1
  for (int c = 0; c < nch; ++c) {
    lds_barrier();  // chunk c is in its buffer; every reader of chunk c - 1 is done
    if (loader) {
      const int kn = (c + 2) * kPChunk;
#pragma unroll
      for (int j = 0; j < kPChunk; ++j) {
        abuf(c + 1, j, wave) = ar[j];
        ar[j] = row_operand(ra, own(kn + j), kn + j, lq);
      }
    }
#pragma unroll
    for (int j = 0; j < kPChunk; ++j) {
      const int kb = c * kPChunk + j;
      const uint4 w = wr[j];
      const uint4 q0 = moe::q4_operand(w.x, mq), q1 = moe::q4_operand(w.y, mq);
      const uint4 q2 = moe::q4_operand(w.z, mq), q3 = moe::q4_operand(w.w, mq);
      const bool gstart = j % kKbpg == 0;  // compile-time: a group's first product starts from zero
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        const uint4 A = abuf(c, j, rt);
        D[rt][0] = moe::mfma_bf16(A, q0, gstart ? zf : D[rt][0]);
        D[rt][1] = moe::mfma_bf16(A, q1, gstart ? zf : D[rt][1]);
        D[rt][2] = moe::mfma_bf16(A, q2, gstart ? zf : D[rt][2]);
        D[rt][3] = moe::mfma_bf16(A, q3, gstart ? zf : D[rt][3]);
        Db[rt] = moe::mfma_bf16(A, bc, gstart ? zf : Db[rt]);
      }
      // issue order: the A reads, then each product followed by three VALU
      // operations (the next word's unpack), so that one wave's unpack runs
      // under its own products (left to itself the compiler puts the whole
      // unpack first: gate/up 111-113 -> 108 us at M=512)
      __builtin_amdgcn_sched_group_barrier(0x100, 3, 0);  // LDS reads
#pragma unroll
      for (int p = 0; p < 5 * RT; ++p) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one matrix-core product
        __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);  // three VALU
      }
      // a group ends at its last k block or at K (a group that K ends inside
      // is finished there: the next group start, past K, resets D); k blocks
      // past K multiply zeros (their loads read nothing) and add nothing
      if (kb < KB && (j % kKbpg == kKbpg - 1 || kb == KB - 1)) epilogue(kb >> GSH);
      wr[j] = wload(kb + kPRing);
    }
  }
}

// A workgroup's scale table in LDS: entry i (group i >> 6, column quad
// i & 63, whose first column is col_of(quad)) holds the quad's 4 scales of
// the group, from one expert's [G][N] table.  Loads go out kScB per thread
// before any LDS write (one memory round trip per 2048 entries instead of one
// per 256); quads past N read zeros without a memory access.  The first batch
// is issued on its own (issue(0), before the workgroup's other start-up
// loads); store() writes it and stages the rest, if any.
constexpr int kScB = 8;
template <class ColOf>
struct ScaleStage {
  __amdgpu_buffer_rsrc_t r;
  int n, N;
  ColOf col_of;
  u32x2_t v[kScB];
  __device__ __forceinline__ ScaleStage(const uint16_t* sc_e, int G, int N_, ColOf c)
      : r(buffer_rsrc(sc_e, (uint32_t)G * (uint32_t)N_ * 2u)), n(G * 64), N(N_), col_of(c) {}
  __device__ __forceinline__ void issue(int b) {
#pragma unroll
    for (int j = 0; j < kScB; ++j) {
      const int i = b + j * kPThreads + (int)threadIdx.x;
      const int col = col_of(i & 63);
      const uint32_t off = i < n && col + 4 <= N ? ((uint32_t)(i >> 6) * (uint32_t)N + (uint32_t)col) * 2u : kOob;
      v[j] = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0);
    }
  }
  __device__ __forceinline__ void write(int b, uint2* lds) const {
#pragma unroll
    for (int j = 0; j < kScB; ++j) {
      const int i = b + j * kPThreads + (int)threadIdx.x;
      if (i < n) lds[i] = make_uint2(v[j].x, v[j].y);
    }
  }
  __device__ __forceinline__ void store(uint2* lds) {
    write(0, lds);
    for (int b = kPThreads * kScB; b < n; b += kPThreads * kScB) {
      issue(b);
      write(b, lds);
    }
  }
};
template <class ColOf>
__device__ __forceinline__ ScaleStage<ColOf> scale_stage(const uint16_t* sc_e, int G, int N, ColOf c) {
  return ScaleStage<ColOf>(sc_e, G, N, c);
}


// gate/up: workgroup (tile t, expert e) owns gate columns [128t, 128t+128)
// (waves 0, 1) and the same up columns (waves 2, 3); act = bf16(gelu(g)*u).
template <int GSH>
__global__ __launch_bounds__(kPThreads, 2) void prefill_gu_kernel(PfArgs a) {
  __shared__ float yb[16][256];   // one row tile's gate | up sums
  __shared__ uint4 aring[2 * kPChunk * kPRT * 64];
  extern __shared__ uint2 gsc[];  // [Ggu][64]: 4 scales of each column quad
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid >> 6;
  const int lq = lane >> 4, lr = lane & 15;
  const int tile = blockIdx.x, e = blockIdx.y;
  const int twoI = 2 * a.I;
  // column of quad c (0..63) of this workgroup: waves 0-1 gate, 2-3 up
  auto quad_col = [&](int c) { return (c < 32 ? 0 : a.I) + 128 * tile + 4 * (c & 31); };
  const int off_e = a.offsets[e], n_e = a.offsets[e + 1] - off_e;
  if (n_e <= 0) return;
  auto scales = scale_stage(a.gus + (size_t)e * a.Ggu * twoI, a.Ggu, twoI, quad_col);
  scales.issue(0);
  scales.store(gsc);
  __syncthreads();
  const __amdgpu_buffer_rsrc_t rw = buffer_rsrc(a.gu, a.gu_total);
  const __amdgpu_buffer_rsrc_t rx = buffer_rsrc(a.xk, a.x_bytes);
  const int col = quad_col(16 * wave + lr);
  const uint32_t wbase = ((uint32_t)lq * twoI + col) * 4u;
  const uint32_t wstep = (uint32_t)twoI * 16u;  // 4 packed rows
  // a wave whose 64 gate (or up) columns all lie past I (the last tile when
  // I is not a multiple of 128) has no products to run
  const bool glive = 128 * tile + 64 * (wave & 1) < a.I;
  for (int base = 0; base < n_e; base += 16 * kPRT) {
    // this wave's row tile (waves < kPRT load the A operands for all)
    const int jo = base + 16 * wave + lr;
    const uint32_t roff = wave < kPRT && jo < n_e ? (uint32_t)(a.order[off_e + jo] / a.top_k) * (uint32_t)a.H * 2u
                                                 : kOob;
    f32x4_t y[kPRT][4];
    // (all three row tiles: a second instantiation for passes of at most 32
    // pairs, as in down, made this kernel spill and measured slower)
    grouped_products<kPRingGu, GSH, kPRT>(rw, glive ? wbase : kOob, wstep, e * a.gu_bytes, rx, roff, a.H >> 5,
                                          a.Ggu, gsc, aring, y);
#pragma unroll
    for (int rt = 0; rt < kPRT; ++rt) {
      __syncthreads();
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) yb[4 * lq + jj][64 * wave + 4 * lr + q] = y[rt][q][jj];
      __syncthreads();
      for (int i = tid; i < 16 * 128; i += kPThreads) {
        const int t = i >> 7, c = i & 127;
        const int j = base + 16 * rt + t;
        const int ic = 128 * tile + c;
        if (j < n_e && ic < a.I)
          a.act[(size_t)(off_e + j) * a.I + (ic & ~7) + moe::mfma_k_pos(ic & 7)] =
              f32_to_bf16(gelu_tanh(yb[t][c]) * yb[t][128 + c]);
      }
    }
  }
}

// down: workgroup (unit d, expert e) owns output columns [256d, 256d+256);
// y fp32 rows of the expert's pairs, at each pair's index.
template <int GSH>
__global__ __launch_bounds__(kPThreads, 2) void prefill_down_kernel(PfArgs a) {
  __shared__ uint4 aring[2 * kPChunk * kPRT * 64];
  // the pair of each row of a pass, in the chunk buffers once the products
  // are done (no LDS beyond theirs: the 160 KB limit check counts them only)
  int* prow = reinterpret_cast<int*>(aring);
  extern __shared__ uint2 dsc[];  // [Gd][64]: 4 scales of each column quad
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid >> 6;
  const int lq = lane >> 4, lr = lane & 15;
  const int unit = blockIdx.x, e = blockIdx.y;
  const int off_e = a.offsets[e], n_e = a.offsets[e + 1] - off_e;
  if (n_e <= 0) return;
  auto scales = scale_stage(a.dns + (size_t)e * a.Gd * a.H, a.Gd, a.H, [unit](int c) { return 256 * unit + 4 * c; });
  scales.issue(0);
  scales.store(dsc);
  __syncthreads();
  const int col = 256 * unit + 64 * wave + 4 * lr;
  const bool live = 256 * unit + 64 * wave < a.H;  // a partial last unit: the wave still joins the barriers
  const __amdgpu_buffer_rsrc_t rw = buffer_rsrc(a.dn, a.dn_total);
  const __amdgpu_buffer_rsrc_t ra = buffer_rsrc(a.act, a.act_bytes);
  const uint32_t wbase = ((uint32_t)lq * a.H + col) * 4u;
  const uint32_t wstep = (uint32_t)a.H * 16u;
  for (int base = 0; base < n_e; base += 16 * kPRT) {
    // each row's pair index (its result row): loaded here, written to LDS
    // after the products (the load must not hold the products' first loads)
    const int pr = tid < 16 * kPRT && base + tid < n_e ? a.order[off_e + base + tid] : 0;
    const int jo = base + 16 * wave + lr;
    const uint32_t roff = wave < kPRT && jo < n_e ? (uint32_t)(off_e + jo) * (uint32_t)a.I * 2u : kOob;
    f32x4_t y[kPRT][4];
    // two row tiles when the pass has at most 32 pairs (half the experts at
    // M = 512): a third fewer products and epilogue operations
    if (n_e - base <= 32)
      grouped_products<kPRingDn, GSH, 2>(rw, live ? wbase : kOob, wstep, e * a.dn_bytes, ra, roff, a.I >> 5,
                                         a.Gd, dsc, aring, y);
    else
      grouped_products<kPRingDn, GSH, kPRT>(rw, live ? wbase : kOob, wstep, e * a.dn_bytes, ra, roff, a.I >> 5,
                                            a.Gd, dsc, aring, y);
    lds_barrier();  // every wave's last reads of the chunk buffers are done
    if (tid < 16 * kPRT) prow[tid] = pr;
    lds_barrier();  // (the next pass's products start with a barrier before they write the buffers)
#pragma unroll
    for (int rt = 0; rt < kPRT; ++rt)
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const int j = base + 16 * rt + 4 * lq + jj;
        if (live && j < n_e)
          *(float4*)(a.y + (size_t)prow[16 * rt + 4 * lq + jj] * a.H + col) =
              make_float4(y[rt][0][jj], y[rt][1][jj], y[rt][2][jj], y[rt][3][jj]);
      }
  }
}

// ---------------------------------------------------------------------------
// combine: out[t] (+)= sum over slots, in slot order, of w * y[pair]
// ---------------------------------------------------------------------------
// A pair's routing as the combine reads it: whether its id is in [0, E)
// (other ids are skipped, marlin.cu:288-289) and its weight rounded to bf16
// (marlin.cu:631-636), from the caller's (or the routed) ids and weights.
// Its result row is the pair index itself.
struct PfSlots {
  const void* idx;
  const void* w;
  int idx_is64, w_dtype, E;
};
__device__ __forceinline__ void slot_of(const PfSlots& s, int p, int& ok, float& wv) {
  const int id = load_expert_id(s.idx, s.idx_is64, p);
  wv = load_weight_as_bf16(s.w, s.w_dtype, p);
  ok = id >= 0 && id < s.E;
}

__global__ __launch_bounds__(256) void prefill_combine_kernel(const float* y, PfSlots sl, uint16_t* out, int H,
                                                              int top_k, int overwrite) {
  const int t = blockIdx.x;
  for (int c = threadIdx.x * 4; c < H; c += 256 * 4) {
    float4 s = overwrite ? make_float4(0.f, 0.f, 0.f, 0.f)
                         : make_float4(bf16_to_f32(out[(size_t)t * H + c]), bf16_to_f32(out[(size_t)t * H + c + 1]),
                                       bf16_to_f32(out[(size_t)t * H + c + 2]), bf16_to_f32(out[(size_t)t * H + c + 3]));
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int k = 0; k < top_k; ++k) {
      int ok;
      float wv;
      slot_of(sl, t * top_k + k, ok, wv);
      const float4 v = *(const float4*)(y + (size_t)(t * top_k + k) * H + c);
      if (!ok) continue;
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

// The same for top_k <= 8 with every load of the workgroup issued before any
// use: a slot's result row is its pair index, so the three column chunks of
// each thread (H <= 3072 per pass) over all slots and the previous output go
// out together with the slots' ids and weights (one memory round trip).  A
// skipped slot's row is read and not used.  Same arithmetic and order as
// prefill_combine_kernel.
constexpr int kCombineSlots = 8;
constexpr int kCombineChunks = 3;
__global__ __launch_bounds__(256) void prefill_combine8_kernel(const float* y, PfSlots sl, uint16_t* out, int H,
                                                               int top_k, int overwrite) {
  const int t = blockIdx.x;
  __shared__ int sok[kCombineSlots];
  __shared__ float swt[kCombineSlots];
  int okv = 0;
  float wvv = 0.f;
  if ((int)threadIdx.x < top_k) slot_of(sl, t * top_k + threadIdx.x, okv, wvv);
  const __amdgpu_buffer_rsrc_t ro = buffer_rsrc(out + (size_t)t * H, overwrite ? 0u : (uint32_t)H * 2u);
  constexpr int kStep = 256 * 4 * kCombineChunks;
  const int nit = (H + kStep - 1) / kStep;  // the same for every thread (the barrier below)
  int ok[kCombineSlots];
  float wv[kCombineSlots];
  for (int it = 0; it < nit; ++it) {
    const int c0 = threadIdx.x * 4 + it * kStep;
    u32x4_t v[kCombineChunks][kCombineSlots];
    u32x2_t o[kCombineChunks];
#pragma unroll
    for (int k = 0; k < kCombineSlots; ++k) {
      // a row's resource (its offsets stay below 2^32 whatever the row count)
      const __amdgpu_buffer_rsrc_t ry =
          buffer_rsrc(y + (size_t)(t * top_k + (k < top_k ? k : 0)) * H, k < top_k ? (uint32_t)H * 4u : 0u);
#pragma unroll
      for (int i = 0; i < kCombineChunks; ++i) {
        const int c = c0 + i * 1024;
        v[i][k] = __builtin_amdgcn_raw_buffer_load_b128(ry, c < H ? (uint32_t)c * 4u : kOob, 0, 0);
      }
    }
#pragma unroll
    for (int i = 0; i < kCombineChunks; ++i) {
      const int c = c0 + i * 1024;
      o[i] = __builtin_amdgcn_raw_buffer_load_b64(ro, c < H ? (uint32_t)c * 2u : kOob, 0, 0);
    }
    if (it == 0) {
      if (threadIdx.x < kCombineSlots) {
        sok[threadIdx.x] = okv;
        swt[threadIdx.x] = wvv;
      }
      lds_barrier();  // LDS only: the row loads stay in flight
#pragma unroll
      for (int k = 0; k < kCombineSlots; ++k) {
        ok[k] = __builtin_amdgcn_readfirstlane(sok[k]);
        wv[k] = swt[k];
      }
    }
#pragma unroll
    for (int i = 0; i < kCombineChunks; ++i) {
      const int c = c0 + i * 1024;
      if (c >= H) continue;
      float4 s = overwrite ? make_float4(0.f, 0.f, 0.f, 0.f)
                           : make_float4(bf16lo(o[i].x), bf16hi(o[i].x), bf16lo(o[i].y), bf16hi(o[i].y));
      float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
      for (int k = 0; k < kCombineSlots; ++k) {
        if (!ok[k]) continue;
        acc.x += wv[k] * __uint_as_float(v[i][k].x);
        acc.y += wv[k] * __uint_as_float(v[i][k].y);
        acc.z += wv[k] * __uint_as_float(v[i][k].z);
        acc.w += wv[k] * __uint_as_float(v[i][k].w);
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
}

constexpr size_t kPAlign = 256;
inline size_t pround(size_t v) { return (v + kPAlign - 1) / kPAlign * kPAlign; }

struct PfLayout {
  size_t idx, w, offsets, order, xk, act, y, total;
};
PfLayout pf_layout(int M, int top_k, int H, int I, int E) {
  const size_t P = (size_t)M * top_k;
  PfLayout l;
  l.idx = 0;
  l.w = pround(l.idx + P * 4);
  l.offsets = pround(l.w + P * 2);
  l.order = pround(l.offsets + (size_t)(E + 1) * 4);
  l.xk = pround(l.order + P * 4);
  l.act = pround(l.xk + (size_t)M * H * 2);
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
  if (h.H % 64 || h.I % 32) return false;
  if (h.gs % 32 || log2_exact(h.gs / 32) < 0 || kPChunk % (h.gs / 32)) return false;
  if (h.top_k > 64 || h.E > 1024) return false;
  // a workgroup's scales sit in LDS beside its static arrays (the gate/up sums
  // of a row tile, the staged A tiles): a launch past the CU's 160 KB fails
  constexpr size_t kLds = 160 * 1024, kDnStatic = 2 * kPChunk * kPRT * 64 * sizeof(uint4),
                   kGuStatic = 16 * 256 * sizeof(float) + kDnStatic;
  if ((size_t)h.Ggu * 64 * sizeof(uint2) + kGuStatic > kLds || (size_t)h.Gd * 64 * sizeof(uint2) + kDnStatic > kLds)
    return false;
  const long long P = (long long)h.M * h.top_k;
  // 32-bit buffer offsets (loads past K read an offset past the resource)
  if ((long long)h.E * (h.H / 8) * 2 * h.I * 4 >= (1LL << 32)) return false;
  if ((long long)h.E * (h.I / 8) * h.H * 4 >= (1LL << 32)) return false;
  if ((long long)h.M * h.H * 2 >= (1LL << 32) || P * h.I * 2 >= (1LL << 32)) return false;
  return P <= (1 << 20);
}

size_t moe_prefill_workspace_bytes(int M, int top_k, int H, int I, int E) {
  return pf_layout(M, top_k, H, I, E).total;
}

int launch_moe_prefill(const MoeHostArgs& h, void* workspace, size_t ws_bytes, int* arrive) {
  const PfLayout L = pf_layout(h.M, h.top_k, h.H, h.I, h.E);
  if (!workspace || ws_bytes < L.total)
    return fail(GI_ERR_WORKSPACE, "fused MoE: workspace missing or smaller than gi_fused_moe_workspace_bytes()");
  char* ws = (char*)workspace;
  const int P = h.M * h.top_k;
  PfFront f{};
  f.idx = h.idx;
  f.idx_is64 = h.idx_is64;
  const void* w = h.w;
  int w_dtype = h.w_dtype;
  if (h.logits) {
    // routing into the caller's report buffers when given, else the workspace
    // (the checks of the router-only entry point)
    if (h.E > moe::kRouteMaxExperts || h.top_k > h.E || h.top_k > 64)
      return fail(GI_ERR_UNSUPPORTED, "route: at most 1024 experts and top_k <= min(E, 64)");
    if (h.logits_dtype != GI_DTYPE_BF16 && h.logits_dtype != GI_DTYPE_FP32)
      return fail(GI_ERR_UNSUPPORTED, "route: logits must be bf16 or fp32");
    f.out_idx = h.out_idx ? h.out_idx : (int32_t*)(ws + L.idx);
    f.out_w = h.out_w ? (uint16_t*)h.out_w : (uint16_t*)(ws + L.w);
    f.r.logits = h.logits;
    f.r.logits_dtype = h.logits_dtype;
    f.r.expert_scale = h.expert_scale;
    f.nroute = (h.M + kAlignThreads / kWave - 1) / (kAlignThreads / kWave);
    f.idx = f.out_idx;
    f.idx_is64 = 0;
    w = f.out_w;
    w_dtype = GI_DTYPE_BF16;
  }
  f.r.M = h.M;
  f.r.E = h.E;
  f.r.top_k = h.top_k;
  f.P = P;
  int* offsets = (int*)(ws + L.offsets);
  int* order = (int*)(ws + L.order);
  f.offsets = offsets;
  f.order = order;
  f.arrive = arrive;
  f.x = (const uint4*)h.x;
  f.xk = (uint4*)(ws + L.xk);
  f.nx = h.M * h.H / 8;
  // one launch: routing (or the caller's ids), the align, the x reorder
  const int nlead = f.nroute > 0 ? f.nroute : 1;
  hipLaunchKernelGGL(prefill_front_kernel, dim3(nlead + (f.nx + kAlignThreads - 1) / kAlignThreads),
                     dim3(kAlignThreads), 0, h.stream, f);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return hip_fail(e, "prefill routing / align / x reorder launch");

  PfArgs k{};
  k.x = (const uint16_t*)h.x;
  k.xk = (uint16_t*)(ws + L.xk);
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
  const size_t gl = (size_t)h.Ggu * 64 * sizeof(uint2), dl = (size_t)h.Gd * 64 * sizeof(uint2);
  const dim3 ggrid((h.I + 127) / 128, h.E), dgrid((h.H + 255) / 256, h.E);
  switch (k.gsh) {
    case 0: hipLaunchKernelGGL(prefill_gu_kernel<0>, ggrid, dim3(kPThreads), gl, h.stream, k); break;
    case 1: hipLaunchKernelGGL(prefill_gu_kernel<1>, ggrid, dim3(kPThreads), gl, h.stream, k); break;
    case 2: hipLaunchKernelGGL(prefill_gu_kernel<2>, ggrid, dim3(kPThreads), gl, h.stream, k); break;
    default: hipLaunchKernelGGL(prefill_gu_kernel<3>, ggrid, dim3(kPThreads), gl, h.stream, k); break;
  }
  e = hipGetLastError();
  if (e != hipSuccess) return hip_fail(e, "prefill gate/up launch");
  switch (k.gsh) {
    case 0: hipLaunchKernelGGL(prefill_down_kernel<0>, dgrid, dim3(kPThreads), dl, h.stream, k); break;
    case 1: hipLaunchKernelGGL(prefill_down_kernel<1>, dgrid, dim3(kPThreads), dl, h.stream, k); break;
    case 2: hipLaunchKernelGGL(prefill_down_kernel<2>, dgrid, dim3(kPThreads), dl, h.stream, k); break;
    default: hipLaunchKernelGGL(prefill_down_kernel<3>, dgrid, dim3(kPThreads), dl, h.stream, k); break;
  }
  e = hipGetLastError();
  if (e != hipSuccess) return hip_fail(e, "prefill down launch");
  const PfSlots sl{f.idx, w, f.idx_is64, w_dtype, h.E};
  if (h.top_k <= kCombineSlots)
    hipLaunchKernelGGL(prefill_combine8_kernel, dim3(h.M), dim3(256), 0, h.stream, k.y, sl, (uint16_t*)h.out, h.H,
                       h.top_k, h.overwrite);
  else
    hipLaunchKernelGGL(prefill_combine_kernel, dim3(h.M), dim3(256), 0, h.stream, k.y, sl, (uint16_t*)h.out, h.H,
                       h.top_k, h.overwrite);
  e = hipGetLastError();
  if (e != hipSuccess) return hip_fail(e, "prefill combine launch");
  return GI_OK;
}

}  // namespace gi
