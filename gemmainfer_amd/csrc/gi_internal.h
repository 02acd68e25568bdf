// Host-side declarations shared between the C-ABI layer (capi.cpp) and the
// kernel translation units.  Not part of the public ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <string>

namespace gi {

// Sets the thread-local error message and returns `code`.
int fail(int code, const std::string& msg);
int hip_fail(hipError_t e, const char* what);

// Multiprocessor count of the current device (cached per device).
int device_cu_count();

// Device address of the current device's error flag: an int in host memory
// mapped into the device, which kernels set when a bounded wait gives up
// (null if the mapping is unavailable).  Read and cleared by
// gi_device_error_flags without any device synchronisation.  The flags are
// allocated (pinned host memory) by gi_device_error_flags or by the first
// call with allocate = true whose stream is not capturing a graph;
// allocate = false only returns them once they exist.
int* device_error_flag(bool allocate, hipStream_t stream);
int read_device_error_flags(int device, int clear);

// ---- fused MoE --------------------------------------------------------------
struct MoeHostArgs {
  const void* x;
  const int32_t* gu_packed;
  const void* gu_scales;
  const int32_t* d_packed;
  const void* d_scales;
  const void* idx;
  int idx_is64;
  const void* w;
  int w_dtype;
  const void* logits;       // layer mode when non-null
  int logits_dtype;         // 0 bf16, 2 fp32
  const float* expert_scale;
  int32_t* out_idx;
  void* out_w;
  void* out;
  int M, H, I, E, top_k, gs, Ggu, Gd;
  int overwrite;
  void* workspace;
  size_t workspace_bytes;
  int spin_limit;
  hipStream_t stream;
  int no_alloc;             // the caller cannot allocate: no pinned-memory set-up either
  int x_dtype;              // activations, scales and out: GI_DTYPE_BF16 (0), FP16 or FP32
};

// Argument checks shared by every fused-MoE entry point (GI_OK or a failure code).
int check_moe_args(const MoeHostArgs& h);
// Byte offset of the decode kernel's state in a MoE workspace (the status word is at 0).
size_t moe_decode_scratch_offset();
// Largest number of token rows one fused launch handles (S = rows*top_k <= 256).
int moe_rows_per_launch(int top_k);
size_t moe_workspace_bytes(int rows, int top_k, int H, int I, int E);      // bf16 activations
size_t moe_workspace_bytes_any(int rows, int top_k, int H, int I, int E);  // any activation dtype
int launch_fused_moe(const MoeHostArgs& a);
// decode/verify kernel (moe_decode.hip): <= 8 rows per launch, no grid barrier
bool moe_decode_supported(const MoeHostArgs& h);
int moe_decode_rows_per_launch(int top_k);
size_t moe_decode_state_bytes();        // epochs + exchange buffers: kept between calls
int launch_moe_decode(const MoeHostArgs& h, void* state, int* status);
// timeline builds (-DGI_TIMELINE): per-workgroup phase stamps of every decode launch
int set_decode_timeline(void* buf, size_t bytes);
unsigned long long* decode_timeline_slot();  // null unless a timeline buffer is set
// one-token decode kernel (moe_decode1.hip): M == 1, one wait between workgroups;
// the same state (epochs, exchange buffers) as the decode kernel
bool moe_decode1_supported(const MoeHostArgs& h);
int launch_moe_decode1(const MoeHostArgs& h, void* state, int* status);
// the same launches with the library's static per-GPU scratch (moe_static.hip)
int launch_fused_moe_static(MoeHostArgs h);
// prefill (moe_prefill.hip): sorted-by-expert grouped GEMM for M >= kPrefillMinRows
constexpr int kPrefillMinRows = 64;
bool moe_prefill_supported(const MoeHostArgs& h);
size_t moe_prefill_workspace_bytes(int M, int top_k, int H, int I, int E);
// arrive: a counter word of the workspace that is zero between launches (the
// prefill's front launch counts its routing workgroups there)
int launch_moe_prefill(const MoeHostArgs& h, void* ws, size_t ws_bytes, int* arrive);
int launch_moe_align(const void* idx, int is64, int M, int top_k, int E, int32_t* uniq,
                     int32_t* nuniq, int32_t* s2u, int32_t* offsets, int32_t* slots,
                     hipStream_t stream);
int launch_route(const void* logits, int logits_dtype, const float* expert_scale, int M,
                 int E, int top_k, int32_t* out_idx, void* out_w, int w_dtype,
                 hipStream_t stream);
int read_workspace_status(void* workspace, int32_t* host_status, hipStream_t stream);
int launch_moe_router(const void* x, const void* router_scale, const void* gate, void* logits, int M,
                      int H, int E, float eps, hipStream_t stream);

// fp16 / fp32 activations (generic_dtype.hip): VALU kernels, fp32 arithmetic,
// the reference's rounding points in the activation dtype; the MoE runs in
// launches of up to 64 slots whose activations [S][I], slot outputs [S][H]
// (fp32) and Token-Union tables sit in the workspace
size_t moe_generic_workspace_bytes(int M, int top_k, int H, int I);
int launch_moe_generic(const MoeHostArgs& h, int x_dtype, void* act_ws, size_t act_bytes);
int launch_w4a16_generic(const void* A, int a_dtype, const int32_t* B, const void* scales, int n_groups, void* C,
                         int M, int K, int N, int gs, float softcap, hipStream_t stream);

// ---- W4A16 linear -------------------------------------------------------------
size_t w4a16_workspace_bytes(int M, int K, int N, int gs);
int launch_w4a16(const void* A, const int32_t* B, const void* scales, int n_groups, void* C,
                 int M, int K, int N, int gs, float softcap, void* workspace,
                 size_t workspace_bytes, hipStream_t stream);

int launch_w4a16_multi(const void* A, int n, const int32_t* const* B, const void* const* scales, const int* n_groups,
                       void* const* C, const int* N, int M, int K, int gs, void* workspace, size_t workspace_bytes,
                       hipStream_t stream);
size_t w4a16_gated_workspace_bytes(int M, int K, int N, int gs);
size_t w4a16_multi_workspace_bytes(int n, const int* N, int M, int K, int gs);
int launch_w4a16_gated(const void* A, const int32_t* gB, const void* gS, int gG, const int32_t* uB, const void* uS,
                       int uG, void* out, int M, int K, int N, int gs, void* workspace, size_t workspace_bytes,
                       hipStream_t stream);
int launch_w4a16_ingest_batched(const int32_t* weight_packed, const void* weight_scale, int scale_dtype, int batch,
                                int N, int K, int n_groups, int64_t src_stride_packed, int64_t src_stride_scale,
                                int32_t* packed_out, void* scales_out, int64_t ld_out, int64_t dst_stride_packed,
                                int64_t dst_stride_scale, hipStream_t stream);
int launch_w4a16_ingest(const int32_t* weight_packed, const void* weight_scale, int scale_dtype, int N,
                        int K, int n_groups, int32_t* packed_out, void* scales_out, int64_t ld_out,
                        hipStream_t stream);

// ---- companions -------------------------------------------------------------
int launch_softcap(void* x, int dtype, int64_t n, float cap, hipStream_t stream);
int launch_rmsnorm(const void* in, const void* weight, void* out, int dtype, int64_t rows,
                   int hidden, float eps, int add_unit_offset, hipStream_t stream);
int launch_rope(void* q, void* k, const void* cos_t, const void* sin_t,
                const int64_t* pos, int dtype, int B, int Hq, int Hk, int S, int D,
                const int64_t* q_strides, const int64_t* k_strides, hipStream_t stream);

}  // namespace gi
