// extern "C" entry points declared in include/gemmainfer_amd.h: argument
// checks, dtype dispatch and error reporting around the gfx950 kernels.

#include <mutex>
#include <string>

#include "../../include/gemmainfer_amd.h"
#include "gi_internal.h"

namespace gi {

namespace {
thread_local std::string g_last_error;
}

int fail(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

int hip_fail(hipError_t e, const char* what) {
  g_last_error = std::string(what) + ": " + hipGetErrorName(e) + " (" + hipGetErrorString(e) + ")";
  return GI_ERR_HIP;
}

int device_cu_count() {
  static int cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

// Error flags of up to 64 devices, one 128-byte line each, in host memory
// mapped into every device (coherent: a kernel's store is visible to the
// host without a synchronisation).  One pinned page per process, allocated
// by gi_device_error_flags or by the first MoE launch whose stream is not
// capturing a graph (an allocation there could invalidate the capture); a
// failed allocation is tried again on the next such call.
namespace {
constexpr int kFlagStride = 32;  // ints
std::mutex g_flag_mu;
int* g_flags = nullptr;

int* flags_host(bool allocate) {
  std::lock_guard<std::mutex> lk(g_flag_mu);
  if (allocate && !g_flags) {
    void* p = nullptr;
    if (hipHostMalloc(&p, 64 * kFlagStride * sizeof(int),
                      hipHostMallocMapped | hipHostMallocPortable | hipHostMallocCoherent) == hipSuccess && p) {
      for (int i = 0; i < 64 * kFlagStride; ++i) ((volatile int*)p)[i] = 0;
      g_flags = (int*)p;
    } else {
      (void)hipGetLastError();
    }
  }
  return g_flags;
}

bool capturing(hipStream_t stream) {
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(stream, &cs) != hipSuccess) {
    (void)hipGetLastError();
    return true;  // unknown: do not allocate
  }
  return cs != hipStreamCaptureStatusNone;
}
}  // namespace

int* device_error_flag(bool allocate, hipStream_t stream) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
  int* h = flags_host(allocate && !capturing(stream));
  if (!h) return nullptr;
  void* d = nullptr;
  if (hipHostGetDevicePointer(&d, h + dev * kFlagStride, 0) != hipSuccess) {
    (void)hipGetLastError();
    return nullptr;
  }
  return (int*)d;
}

int read_device_error_flags(int device, int clear) {
  if (device < 0 || device >= 64) return fail(GI_ERR_INVALID_ARG, "device_error_flags: device index out of range");
  int* h = flags_host(true);
  if (!h) return 0;
  volatile int* f = h + device * kFlagStride;
  const int v = *f;
  if (clear && v) *f = 0;
  return v;
}

}  // namespace gi

using gi::fail;

namespace {

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

int check_idx_dtype(int dt) {
  if (dt != GI_DTYPE_INT32 && dt != GI_DTYPE_INT64)
    return fail(GI_ERR_UNSUPPORTED, "expert ids must be int32 or int64");
  return GI_OK;
}

int check_bf16_x(int dt, const char* who) {
  if (dt != GI_DTYPE_BF16)
    return fail(GI_ERR_UNSUPPORTED,
                std::string(who) + ": only bf16 activations/scales are implemented on gfx950");
  return GI_OK;
}

}  // namespace

extern "C" {

const char* gi_last_error(void) { return gi::g_last_error.c_str(); }

int gi_abi_version(void) { return 1; }

int gi_moe_route_topk_softmax(const void* logits, int logits_dtype, const float* expert_scale,
                              int M, int E, int top_k, int32_t* out_idx, void* out_w,
                              int w_dtype, void* stream) {
  return gi::launch_route(logits, logits_dtype, expert_scale, M, E, top_k, out_idx, out_w,
                          w_dtype, as_stream(stream));
}

int gi_moe_align(const void* idx, int idx_dtype, int M, int top_k, int E,
                 int32_t* unique_experts, int32_t* num_unique, int32_t* slot_to_unique,
                 int32_t* offsets, int32_t* slots, void* stream) {
  int st = check_idx_dtype(idx_dtype);
  if (st != GI_OK) return st;
  return gi::launch_moe_align(idx, idx_dtype == GI_DTYPE_INT64, M, top_k, E, unique_experts,
                              num_unique, slot_to_unique, offsets, slots, as_stream(stream));
}

size_t gi_fused_moe_workspace_bytes(int M, int top_k, int H, int I, int E) {
  if (top_k <= 0 || H <= 0 || I <= 0 || E <= 0) return 0;
  return gi::moe_workspace_bytes_any(M, top_k, H, I, E);
}

int gi_fused_batched_moe(const void* x, int x_dtype, const int32_t* gu_packed,
                         const void* gu_scales, int gu_groups, const int32_t* d_packed,
                         const void* d_scales, int d_groups, const void* idx, int idx_dtype,
                         const void* w, int w_dtype, void* out, int M, int H, int I, int E,
                         int top_k, int group_size, void* workspace, size_t workspace_bytes,
                         int spin_limit, void* stream) {
  if (x_dtype != GI_DTYPE_BF16 && x_dtype != GI_DTYPE_FP16 && x_dtype != GI_DTYPE_FP32)
    return fail(GI_ERR_UNSUPPORTED, "fused_batched_moe: activations must be bf16, fp16 or fp32");
  int st = check_idx_dtype(idx_dtype);
  if (st != GI_OK) return st;
  if (w_dtype != GI_DTYPE_BF16 && w_dtype != GI_DTYPE_FP16 && w_dtype != GI_DTYPE_FP32)
    return fail(GI_ERR_UNSUPPORTED, "fused_batched_moe: expert weights must be bf16, fp16 or fp32");
  gi::MoeHostArgs a{};
  a.x = x;
  a.gu_packed = gu_packed;
  a.gu_scales = gu_scales;
  a.d_packed = d_packed;
  a.d_scales = d_scales;
  a.idx = idx;
  a.idx_is64 = idx_dtype == GI_DTYPE_INT64;
  a.w = w;
  a.w_dtype = w_dtype;
  a.out = out;
  a.M = M;
  a.H = H;
  a.I = I;
  a.E = E;
  a.top_k = top_k;
  a.gs = group_size;
  a.Ggu = gu_groups;
  a.Gd = d_groups;
  a.overwrite = 0;
  a.workspace = workspace;
  a.workspace_bytes = workspace_bytes;
  a.spin_limit = spin_limit;
  a.stream = as_stream(stream);
  a.x_dtype = x_dtype;
  return gi::launch_fused_moe(a);
}

int gi_moe_layer_from_logits(const void* x, int x_dtype, const void* logits, int logits_dtype,
                             const float* expert_scale, const int32_t* gu_packed,
                             const void* gu_scales, int gu_groups, const int32_t* d_packed,
                             const void* d_scales, int d_groups, void* out, int32_t* out_idx,
                             void* out_w, int M, int H, int I, int E, int top_k,
                             int group_size, void* workspace, size_t workspace_bytes,
                             int spin_limit, void* stream) {
  int st = check_bf16_x(x_dtype, "moe_layer_from_logits");
  if (st != GI_OK) return st;
  if (logits_dtype != GI_DTYPE_BF16 && logits_dtype != GI_DTYPE_FP32)
    return fail(GI_ERR_UNSUPPORTED, "moe_layer_from_logits: logits must be bf16 or fp32");
  if (!logits) return fail(GI_ERR_INVALID_ARG, "moe_layer_from_logits: null logits");
  if (top_k > E) return fail(GI_ERR_INVALID_ARG, "moe_layer_from_logits: top_k > number of experts");
  gi::MoeHostArgs a{};
  a.x = x;
  a.gu_packed = gu_packed;
  a.gu_scales = gu_scales;
  a.d_packed = d_packed;
  a.d_scales = d_scales;
  a.logits = logits;
  a.logits_dtype = logits_dtype;
  a.expert_scale = expert_scale;
  a.out_idx = out_idx;
  a.out_w = out_w;
  a.out = out;
  a.M = M;
  a.H = H;
  a.I = I;
  a.E = E;
  a.top_k = top_k;
  a.gs = group_size;
  a.Ggu = gu_groups;
  a.Gd = d_groups;
  a.overwrite = 1;
  a.workspace = workspace;
  a.workspace_bytes = workspace_bytes;
  a.spin_limit = spin_limit;
  a.stream = as_stream(stream);
  return gi::launch_fused_moe(a);
}

int gi_moe_router_logits(const void* x, int x_dtype, const void* router_scale,
                         const void* gate_w, float eps, void* logits, int M, int H, int E,
                         void* stream) {
  int st = check_bf16_x(x_dtype, "moe_router_logits");
  if (st != GI_OK) return st;
  return gi::launch_moe_router(x, router_scale, gate_w, logits, M, H, E, eps, as_stream(stream));
}

int gi_moe_layer_from_hidden(const void* x, int x_dtype, const void* router_scale,
                             const void* gate_w, float eps, void* logits,
                             const float* expert_scale, const int32_t* gu_packed,
                             const void* gu_scales, int gu_groups, const int32_t* d_packed,
                             const void* d_scales, int d_groups, void* out, int32_t* out_idx,
                             void* out_w, int M, int H, int I, int E, int top_k,
                             int group_size, void* workspace, size_t workspace_bytes,
                             int spin_limit, void* stream) {
  int st = check_bf16_x(x_dtype, "moe_layer_from_hidden");
  if (st != GI_OK) return st;
  if (!logits && M > 0) return fail(GI_ERR_INVALID_ARG, "moe_layer_from_hidden: null logits");
  if (top_k <= 0 || top_k > E)
    return fail(GI_ERR_INVALID_ARG, "moe_layer_from_hidden: top_k must be in [1, E]");
  st = gi::launch_moe_router(x, router_scale, gate_w, logits, M, H, E, eps, as_stream(stream));
  if (st != GI_OK) return st;
  return gi_moe_layer_from_logits(x, x_dtype, logits, GI_DTYPE_BF16, expert_scale, gu_packed,
                                  gu_scales, gu_groups, d_packed, d_scales, d_groups, out,
                                  out_idx, out_w, M, H, I, E, top_k, group_size, workspace,
                                  workspace_bytes, spin_limit, stream);
}

int gi_device_error_flags(int device, int clear) { return gi::read_device_error_flags(device, clear); }

int gi_workspace_status(void* workspace, size_t workspace_bytes, int32_t* host_status,
                        void* stream) {
  if (workspace_bytes < sizeof(int32_t))
    return fail(GI_ERR_WORKSPACE, "workspace_status: workspace too small");
  return gi::read_workspace_status(workspace, host_status, as_stream(stream));
}

size_t gi_w4a16_workspace_bytes(int M, int K, int N, int group_size) {
  return gi::w4a16_workspace_bytes(M, K, N, group_size);
}

int gi_w4a16_linear(const void* A, int a_dtype, const int32_t* B_packed, const void* scales,
                    int n_groups, void* C, int M, int K, int N, int group_size, float softcap,
                    void* workspace, size_t workspace_bytes, void* stream) {
  if (a_dtype == GI_DTYPE_FP16 || a_dtype == GI_DTYPE_FP32)
    return gi::launch_w4a16_generic(A, a_dtype, B_packed, scales, n_groups, C, M, K, N, group_size, softcap,
                                    as_stream(stream));
  int st = check_bf16_x(a_dtype, "w4a16_linear");
  if (st != GI_OK) return st;
  return gi::launch_w4a16(A, B_packed, scales, n_groups, C, M, K, N, group_size, softcap,
                          workspace, workspace_bytes, as_stream(stream));
}

int gi_w4a16_linear_multi(const void* A, int a_dtype, int n_proj, const int32_t* const* B_packed,
                          const void* const* scales, const int* n_groups, void* const* C, const int* N, int M,
                          int K, int group_size, void* workspace, size_t workspace_bytes, void* stream) {
  int st = check_bf16_x(a_dtype, "w4a16_linear_multi");
  if (st != GI_OK) return st;
  return gi::launch_w4a16_multi(A, n_proj, B_packed, scales, n_groups, C, N, M, K, group_size, workspace,
                                workspace_bytes, as_stream(stream));
}

size_t gi_w4a16_linear_multi_workspace_bytes(int n_proj, const int* N, int M, int K, int group_size) {
  return gi::w4a16_multi_workspace_bytes(n_proj, N, M, K, group_size);
}

size_t gi_w4a16_gated_mlp_workspace_bytes(int M, int K, int N, int group_size) {
  return gi::w4a16_gated_workspace_bytes(M, K, N, group_size);
}

int gi_w4a16_gated_mlp(const void* A, int a_dtype, const int32_t* gate_packed, const void* gate_scales,
                       int gate_groups, const int32_t* up_packed, const void* up_scales, int up_groups, void* out,
                       int M, int K, int N, int group_size, void* workspace, size_t workspace_bytes,
                       void* stream) {
  int st = check_bf16_x(a_dtype, "w4a16_gated_mlp");
  if (st != GI_OK) return st;
  return gi::launch_w4a16_gated(A, gate_packed, gate_scales, gate_groups, up_packed, up_scales, up_groups, out, M,
                                K, N, group_size, workspace, workspace_bytes, as_stream(stream));
}

int gi_w4a16_ingest(const int32_t* weight_packed, const void* weight_scale, int scale_dtype, int N,
                    int K, int n_groups, int32_t* packed_out, void* scales_out, int64_t ld_out,
                    void* stream) {
  return gi::launch_w4a16_ingest(weight_packed, weight_scale, scale_dtype, N, K, n_groups, packed_out,
                                 scales_out, ld_out, as_stream(stream));
}

int gi_w4a16_ingest_batched(const int32_t* weight_packed, const void* weight_scale, int scale_dtype, int batch,
                            int N, int K, int n_groups, int64_t src_stride_packed, int64_t src_stride_scale,
                            int32_t* packed_out, void* scales_out, int64_t ld_out, int64_t dst_stride_packed,
                            int64_t dst_stride_scale, void* stream) {
  return gi::launch_w4a16_ingest_batched(weight_packed, weight_scale, scale_dtype, batch, N, K, n_groups,
                                         src_stride_packed, src_stride_scale, packed_out, scales_out, ld_out,
                                         dst_stride_packed, dst_stride_scale, as_stream(stream));
}

int gi_softcap_inplace(void* x, int dtype, int64_t n, float cap, void* stream) {
  return gi::launch_softcap(x, dtype, n, cap, as_stream(stream));
}

int gi_rmsnorm(const void* in, const void* weight, void* out, int dtype, int64_t rows,
               int hidden, float eps, int add_unit_offset, void* stream) {
  return gi::launch_rmsnorm(in, weight, out, dtype, rows, hidden, eps, add_unit_offset,
                            as_stream(stream));
}

int gi_rope_inplace(void* q, void* k, const void* cos_t, const void* sin_t,
                    const int64_t* position_ids, int dtype, int B, int Hq, int Hk, int S, int D,
                    int64_t q_sb, int64_t q_sh, int64_t q_ss, int64_t k_sb, int64_t k_sh,
                    int64_t k_ss, void* stream) {
  const int64_t qs[3] = {q_sb, q_sh, q_ss};
  const int64_t ks[3] = {k_sb, k_sh, k_ss};
  return gi::launch_rope(q, k, cos_t, sin_t, position_ids, dtype, B, Hq, Hk, S, D, qs, ks,
                         as_stream(stream));
}

}  // extern "C"
