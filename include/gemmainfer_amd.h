/*
 * gemmainfer_amd.h -- C ABI of the MI355X (gfx950) Token-Union W4A16 MoE path.
 *
 * Plain C: pointers, sizes and int status codes; no torch or HIP types in the
 * signatures (a stream is passed as ``void*`` holding a hipStream_t, NULL =
 * the default stream).  Every entry point is asynchronous on that stream,
 * allocates no device memory and performs no host<->device synchronisation,
 * so it can be recorded into a HIP graph.  One exception, once per process:
 * the page of device error flags (64 ints per device, pinned host memory,
 * see gi_device_error_flags) is allocated by gi_device_error_flags or by the
 * first fused-MoE call whose stream is not capturing a graph; a launch under
 * capture before that has no host flag (its device status word still
 * records a failed wait).  Call gi_device_error_flags once at start-up to
 * allocate it at a time of your choosing.  Scratch memory is caller-owned
 * ("workspace"); it must be zero-filled once when first allocated and is
 * left zeroed by every successful call (the kernels reset their own
 * counters).  Calls that share one workspace must be ordered (same stream).
 *
 * Reference interfaces replaced (paths relative to the GemmaInfer repo):
 *   gi_fused_batched_moe        <- gemmainfer_csrc.fused_batched_moe
 *                                  csrc/pybind.cpp:247-271 -> csrc/marlin.cu:612-702
 *   gi_w4a16_linear             <- gemmainfer_csrc.marlin_w4a16
 *                                  csrc/pybind.cpp:182-196 -> csrc/marlin.cu:704-856
 *   gi_moe_route_topk_softmax   <- the router tail of GemmaBatchedMoE.forward
 *                                  gemmainfer/models/gemma.py:77-80 (torch ops there)
 *   gi_moe_align                <- the per-block dedup scan of the Token-Union kernels
 *                                  csrc/marlin.cu:285-335 and :453-505 (implicit there)
 *   gi_moe_layer_from_logits    <- gemma.py:77-98 (router tail + zeroed out + fused call)
 *   gi_moe_router_logits        <- gemma.py:75-76 (router norm, router_scale, gate linear;
 *                                  torch ops there, rmsnorm.cu:16-73 for the norm)
 *   gi_moe_layer_from_hidden    <- gemma.py:75-98 (the MoE block's forward)
 *   gi_w4a16_linear_multi       <- the q/k/v marlin_w4a16 calls of attention.py:115-122
 *   gi_w4a16_gated_mlp          <- GemmaMLP gate/up + gelu * up (activations.py:26-28)
 *   gi_w4a16_ingest(_batched)   <- gemmainfer/utils/weights.py:100-159 (checkpoint
 *                                  transposition of weight_packed / weight_scale)
 *   gi_softcap_inplace          <- gemmainfer_csrc.softcapping
 *                                  csrc/pybind.cpp:169-180 -> csrc/softcapping.cu:21-47
 *   gi_rmsnorm                  <- gemmainfer_csrc.rmsnorm
 *                                  csrc/pybind.cpp:137-151 -> csrc/rmsnorm.cu:75-114
 *   gi_rope_inplace             <- gemmainfer_csrc.fused_rope_inplace
 *                                  csrc/pybind.cpp:153-167 -> csrc/rmsnorm.cu:116-231
 *
 * Weight layouts are the reference's (gemmainfer/utils/weights.py:153-159,
 * gemmainfer/kernels/quant.py:12-46): int4 codes packed 8 per int32 along the
 * reduction dimension, nibble i of word [pk][n] = code of k = 8*pk+i, value
 * (code - 8) * scale[k / group_size][n].  A scales tensor with fewer groups
 * than ceil(K / group_size) drops the rows it does not cover, exactly as the
 * reference CUDA kernels do (marlin.cu:357,526).
 */
#ifndef GEMMAINFER_AMD_H
#define GEMMAINFER_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ------------------------------------------------------ */
#define GI_OK 0
#define GI_ERR_INVALID_ARG (-1)   /* bad pointer / shape / dtype combination   */
#define GI_ERR_UNSUPPORTED (-2)   /* valid but not implemented (e.g. fp32 x)   */
#define GI_ERR_WORKSPACE (-3)     /* workspace missing or too small            */
#define GI_ERR_HIP (-4)           /* a HIP runtime call failed                 */
#define GI_ERR_DEVICE (-5)        /* a kernel reported a device-side error     */

/* ---- dtype codes ------------------------------------------------------- */
#define GI_DTYPE_BF16 0
#define GI_DTYPE_FP16 1
#define GI_DTYPE_FP32 2
#define GI_DTYPE_INT32 3
#define GI_DTYPE_INT64 4

/* Device-side status bits written into a workspace's status word. */
#define GI_DEVICE_SPIN_TIMEOUT 1  /* a bounded wait gave up (never expected)  */

/* Message for the last non-OK status returned on this host thread. */
const char* gi_last_error(void);
/* ABI version (increments on any signature change). */
int gi_abi_version(void);

/* ---- a1: router tail ----------------------------------------------------
 * logits [M, E] (bf16 or fp32, row-major) -> out_idx int32 [M, top_k]
 * (descending logit; ties -> lower expert index; NaN ranks highest) and
 * out_w [M, top_k] = softmax_fp32(top logits) * expert_scale[idx], stored in
 * w_dtype (bf16/fp16/fp32).  expert_scale: fp32 [E] or NULL (= ones).
 * Limits: 1 <= top_k <= min(E, 64), E <= 1024.                              */
int gi_moe_route_topk_softmax(const void* logits, int logits_dtype,
                              const float* expert_scale, int M, int E, int top_k,
                              int32_t* out_idx, void* out_w, int w_dtype,
                              void* stream);

/* ---- a2: Token-Union alignment -----------------------------------------
 * idx [M*top_k] (int32 or int64; ids outside [0, E) are skipped) ->
 *   unique_experts int32 [min(S,E)]  first-occurrence slot order
 *   num_unique     int32 [1]
 *   slot_to_unique int32 [S]         -1 for skipped slots
 *   offsets        int32 [min(S,E)+1] CSR over unique experts
 *   slots          int32 [S]         slots of each unique expert, ascending
 * S = M*top_k <= 256, E <= 1024.  Entries past num_unique are left as is.  */
int gi_moe_align(const void* idx, int idx_dtype, int M, int top_k, int E,
                 int32_t* unique_experts, int32_t* num_unique,
                 int32_t* slot_to_unique, int32_t* offsets, int32_t* slots,
                 void* stream);

/* ---- a4-a7: fused Token-Union MoE ---------------------------------------
 * out[M, H] += sum_slots bf16(w[slot]) * down(gelu_tanh(gate) * up)(x[token])
 *   x          bf16 [M, H]
 *   gu_packed  int32 [E, H/8, 2I]     gate in columns [0, I), up in [I, 2I)
 *   gu_scales  T [E, gu_groups, 2I]
 *   d_packed   int32 [E, I/8, H]
 *   d_scales   T [E, d_groups, H]
 *   idx        int32|int64 [M*top_k]  w  bf16|fp16|fp32 [M*top_k]
 *   out        T [M, H]               accumulated into (caller zeroes it)
 * T = x_dtype: bf16, fp16 or fp32 (marlin.cu:694-700).  bf16 runs the paths
 * below; fp16 and fp32 run VALU kernels (fp32 arithmetic, the routing
 * weights cast to T, the activation stored in T, one rounding of the output
 * in T; the dequantised weights are never rounded; Token-Union in launches
 * of up to 64 slots, top_k <= 64: alignment, gate/up, down, combine).
 * One kernel launch per 256/top_k rows (8 rows on the decode kernel); from
 * 64 rows with top_k <= 64, a power-of-two multiple of 32 as group size,
 * H % 64 == 0 and I % 32 == 0, the grouped-GEMM prefill path (align with
 * the x reorder, gate/up, down, combine launches; each active expert read
 * once).
 * Requirements: H % 8 == 0,
 * I % 8 == 0, H, I multiples of 4 columns, group_size % 8 == 0, E <= 1024,
 * top_k <= 256.  Deterministic (fixed-order fp32 reductions, no float
 * atomics): the same inputs give bitwise-identical outputs.
 * spin_limit: bound on each inter-workgroup wait (0 = default).            */
size_t gi_fused_moe_workspace_bytes(int M, int top_k, int H, int I, int E);
int gi_fused_batched_moe(const void* x, int x_dtype,
                         const int32_t* gu_packed, const void* gu_scales, int gu_groups,
                         const int32_t* d_packed, const void* d_scales, int d_groups,
                         const void* idx, int idx_dtype,
                         const void* w, int w_dtype,
                         void* out,
                         int M, int H, int I, int E, int top_k, int group_size,
                         void* workspace, size_t workspace_bytes,
                         int spin_limit, void* stream);

/* gi_fused_batched_moe without a workspace argument: no counterpart in the
 * reference (which allocates scratch per call, csrc/marlin.cu:638).  For
 * callers that cannot allocate: code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc.  The scratch is a static 2 MiB
 * device array per GPU, held until the process ends (status word and the
 * decode kernel's exchange state); the call itself allocates nothing (the
 * first call on a device takes the array's address and zero-fills it with a
 * kernel on `stream`; make that first call outside graph capture).  Every
 * call on a GPU shares the array, so calls that overlap on one GPU (other
 * streams, other host threads) race.  Serves the decode kernel's shapes
 * (H, I multiples of 32, H <= 2816, I <= 768, group_size 64 * 2^k,
 * top_k <= 64; any M as launches of up to 8 rows); other shapes return
 * GI_ERR_WORKSPACE.  Results are bitwise those of gi_fused_batched_moe.
 * Errors: a bounded wait that gives up writes NaN into the outputs it could
 * not complete and sets the status word of this device's static scratch
 * (read it with gi_fused_batched_moe_static_status); it also sets the host
 * flag of gi_device_error_flags if that page already exists (this entry
 * never allocates it).                                                     */
int gi_fused_batched_moe_static(const void* x, int x_dtype,
                                const int32_t* gu_packed, const void* gu_scales, int gu_groups,
                                const int32_t* d_packed, const void* d_scales, int d_groups,
                                const void* idx, int idx_dtype,
                                const void* w, int w_dtype,
                                void* out,
                                int M, int H, int I, int E, int top_k, int group_size,
                                int spin_limit, void* stream);

/* Status word of the current device's static scratch (the device-side error
 * bits, GI_DEVICE_*, of gi_fused_batched_moe_static calls since the last
 * clearing read): copied to *host_status after the work queued on `stream`
 * (synchronises the stream); if it is non-zero and clear != 0, the whole
 * static scratch is then zero-filled by a kernel on `stream` (its first-use
 * state: status, launch epochs and exchange buffers).  No counterpart in the reference (its launches report
 * no errors, csrc/marlin.cu:699-701); for callers of the static entry.
 * 0 if no static call has run on this device.  Not for use under capture. */
int gi_fused_batched_moe_static_status(int32_t* host_status, int clear, void* stream);

/* Router + fused MoE: logits [M, E] (bf16/fp32) are routed as
 * gi_moe_route_topk_softmax does (weights rounded to bf16), out[M, H] is
 * OVERWRITTEN with the MoE output, and out_idx/out_w (may be NULL) receive
 * the routing.  Up to 8 rows per launch; from 64 rows (group size a power of
 * two times 32, H % 64 == 0, I % 32 == 0) the sorted-by-expert grouped-GEMM
 * prefill path replaces the 8-row slices of gemma.py:99-112 (routing with
 * the align and the x reorder, gate/up, down, combine launches).           */
int gi_moe_layer_from_logits(const void* x, int x_dtype,
                             const void* logits, int logits_dtype,
                             const float* expert_scale,
                             const int32_t* gu_packed, const void* gu_scales, int gu_groups,
                             const int32_t* d_packed, const void* d_scales, int d_groups,
                             void* out, int32_t* out_idx, void* out_w,
                             int M, int H, int I, int E, int top_k, int group_size,
                             void* workspace, size_t workspace_bytes,
                             int spin_limit, void* stream);

/* ---- f3: router front-end --------------------------------------------------
 * Replaces the torch statements of gemma.py:75-76 (GemmaRMSNorm without scale,
 * norm.py:28-40 -> rmsnorm.cu:16-73; router_scale * hidden_size**-0.5; the
 * bf16 nn.Linear gate) with one launch:
 *   logits[M, E] = bf16( bf16( bf16(x * rsqrt(mean(x^2) + eps))
 *                              * bf16(router_scale * H^-0.5) ) @ gate_w^T )
 * x bf16 [M, H], router_scale bf16 [H] (NULL = ones), gate_w bf16 [E, H] (the
 * nn.Linear weight), logits bf16 [M, E] (overwritten).  fp32 sums in a fixed
 * order: deterministic, and a logit may differ from a BLAS-computed one by one
 * bf16 ulp.  Requirements: H % 8 == 0, H <= 4096, E <= 65536.              */
int gi_moe_router_logits(const void* x, int x_dtype, const void* router_scale,
                         const void* gate_w, float eps, void* logits, int M, int H, int E,
                         void* stream);

/* The whole MoE block from the hidden state (gemma.py:75-98): the router
 * front-end above writes logits (bf16 [M, E], required), then
 * gi_moe_layer_from_logits runs on them.  Same workspace as
 * gi_moe_layer_from_logits; two launches at M <= 8.                        */
int gi_moe_layer_from_hidden(const void* x, int x_dtype, const void* router_scale,
                             const void* gate_w, float eps, void* logits,
                             const float* expert_scale,
                             const int32_t* gu_packed, const void* gu_scales, int gu_groups,
                             const int32_t* d_packed, const void* d_scales, int d_groups,
                             void* out, int32_t* out_idx, void* out_w,
                             int M, int H, int I, int E, int top_k, int group_size,
                             void* workspace, size_t workspace_bytes,
                             int spin_limit, void* stream);

/* Device-side error bits (GI_DEVICE_*) that kernels on `device` have raised
 * since the last clearing read, from a host-memory flag the kernels write
 * directly: no synchronisation, no device work.  A bit is visible once the
 * kernel that raised it has finished.  clear != 0 resets the flag.  A kernel
 * whose bounded wait gave up writes NaN into the outputs it could not
 * complete, so no wrong finite value is ever returned.  No counterpart in
 * the reference, whose launches report no errors (csrc/marlin.cu:699-701):
 * for callers that want such errors without a synchronisation of their own
 * (gemmainfer_csrc checks it before each MoE call).  The first call in a
 * process allocates the flag page (pinned host memory, 8 KiB) if no MoE
 * launch has yet; do that call outside graph capture.                     */
int gi_device_error_flags(int device, int clear);

/* Copies the workspace's device status word to *host_status (synchronises
 * the stream) and clears it.  0 = no device-side error since last read.    */
int gi_workspace_status(void* workspace, size_t workspace_bytes,
                        int32_t* host_status, void* stream);

/* ---- a8 / a11: W4A16 linear ---------------------------------------------
 * C[M, N] = A[M, K] @ dequant(B_packed[K/8, N], scales[n_groups, N]),
 * optionally followed by C = softcap*tanh(C/softcap) when softcap > 0 (the
 * lm_head epilogue, gemma.py:356-357).  A, scales, C of a_dtype: bf16, fp16
 * or fp32 (marlin.cu:764-842; fp16 and fp32 run a VALU kernel with fp32
 * arithmetic and one rounding of C).  C is overwritten.  Requirements:
 * K % 8 == 0, N % 4 == 0 (bf16), group_size % 8 == 0.                       */
size_t gi_w4a16_workspace_bytes(int M, int K, int N, int group_size);
int gi_w4a16_linear(const void* A, int a_dtype,
                    const int32_t* B_packed, const void* scales, int n_groups,
                    void* C, int M, int K, int N, int group_size, float softcap,
                    void* workspace, size_t workspace_bytes, void* stream);

/* ---- f4: dense callers ----------------------------------------------------
 * Several W4A16 projections of the same rows A[M, K] in one launch: the q, k
 * and v projections of attention.py:115-122 (three marlin_w4a16 calls on one
 * input there).  C[i][M, N[i]] = A @ dequant(B_packed[i], scales[i]) for
 * i < n_proj <= 4.  One launch for 1-2 rows (16-column tiles of every
 * projection in one grid) and for 3-16 rows on the matrix-core path (64-column
 * tiles); otherwise one gi_w4a16_linear per projection, in order.  Size the
 * workspace with gi_w4a16_linear_multi_workspace_bytes.  Arrays are host
 * memory.                                                                    */
size_t gi_w4a16_linear_multi_workspace_bytes(int n_proj, const int* N, int M, int K,
                                             int group_size);
int gi_w4a16_linear_multi(const void* A, int a_dtype, int n_proj,
                          const int32_t* const* B_packed, const void* const* scales,
                          const int* n_groups, void* const* C, const int* N,
                          int M, int K, int group_size,
                          void* workspace, size_t workspace_bytes, void* stream);

/* The gated MLP's first half (activations.py:26-28):
 *   out[M, N] = bf16( bf16(gelu_tanh(bf16(A @ Wg))) * bf16(A @ Wu) )
 * with the bf16 roundings of the torch statements.  One launch for 1-2 rows
 * (16-column tiles) and for 3-16 rows on the matrix-core path (both
 * projections per 64-column tile, the gelu and product in the epilogue).
 * Otherwise two linears into the workspace and an elementwise launch; size
 * the workspace with gi_w4a16_gated_mlp_workspace_bytes.                   */
size_t gi_w4a16_gated_mlp_workspace_bytes(int M, int K, int N, int group_size);
int gi_w4a16_gated_mlp(const void* A, int a_dtype,
                       const int32_t* gate_packed, const void* gate_scales, int gate_groups,
                       const int32_t* up_packed, const void* up_scales, int up_groups,
                       void* out, int M, int K, int N, int group_size,
                       void* workspace, size_t workspace_bytes, void* stream);

/* ---- f4: checkpoint ingest ------------------------------------------------
 * Replaces the `t.t()` + copy of weights.py:100-159 that turns a
 * compressed-tensors W4A16 linear into the layout the kernels read:
 *   weight_packed int32 [N, K/8]   ->  packed_out int32 [K/8, ld_out] (columns 0..N-1)
 *   weight_scale  [N, n_groups]    ->  scales_out bf16  [n_groups, ld_out]
 * (bf16/fp16/fp32 scales, rounded to bf16 to nearest even).  Words are moved
 * unchanged.  Pass pointers offset by I columns and ld_out = 2I to fill the up
 * half of an expert's gate_up (weights.py:152-159).  One tiled transpose
 * launch per tensor; n_groups = 0 or K = 0 skips that tensor.              */
int gi_w4a16_ingest(const int32_t* weight_packed, const void* weight_scale, int scale_dtype,
                    int N, int K, int n_groups, int32_t* packed_out, void* scales_out,
                    int64_t ld_out, void* stream);

/* The same for `batch` linears of one shape in one launch (the experts of a
 * layer): matrix b reads weight_packed + b*src_stride_packed and
 * weight_scale + b*src_stride_scale and writes packed_out +
 * b*dst_stride_packed and scales_out + b*dst_stride_scale (strides in
 * elements).  batch <= 65535.                                              */
int gi_w4a16_ingest_batched(const int32_t* weight_packed, const void* weight_scale, int scale_dtype,
                            int batch, int N, int K, int n_groups,
                            int64_t src_stride_packed, int64_t src_stride_scale,
                            int32_t* packed_out, void* scales_out, int64_t ld_out,
                            int64_t dst_stride_packed, int64_t dst_stride_scale, void* stream);

/* ---- drop-in companions (not on the MoE hot path) ----------------------- */
/* x <- cap * tanh(x / cap), n elements, bf16/fp16/fp32.                      */
int gi_softcap_inplace(void* x, int dtype, int64_t n, float cap, void* stream);
/* out[r, :] = in[r, :] * rsqrt(mean(in^2) + eps) * (weight or 1+weight);
 * weight may be NULL (no scale).  bf16/fp16/fp32, in/out/weight same dtype. */
int gi_rmsnorm(const void* in, const void* weight, void* out, int dtype,
               int64_t rows, int hidden, float eps, int add_unit_offset,
               void* stream);
/* Rotate-half RoPE in place: q [B, Hq, S, D], k [B, Hk, S, D] (k may be NULL),
 * last dimension contiguous, other strides in elements (q_sb/q_sh/q_ss and
 * k_sb/k_sh/k_ss for the B, head and S dimensions); cos/sin [P, D]
 * contiguous; position_ids int64 [B, S] contiguous.                          */
int gi_rope_inplace(void* q, void* k, const void* cos_t, const void* sin_t,
                    const int64_t* position_ids, int dtype,
                    int B, int Hq, int Hk, int S, int D,
                    int64_t q_sb, int64_t q_sh, int64_t q_ss,
                    int64_t k_sb, int64_t k_sh, int64_t k_ss, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* GEMMAINFER_AMD_H */
