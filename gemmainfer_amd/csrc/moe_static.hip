// gi_fused_batched_moe_static: the fused MoE (gi_fused_batched_moe) for
// callers that cannot allocate -- code under HIP graph capture, tight
// serving loops, harnesses that forbid hipMalloc.  Its scratch memory is a
// file-scope device array (one per GPU, held until the process ends) instead
// of a caller workspace: the status word and the decode kernel's exchange
// state (launch epochs, activation and partial-sum buffers).  No counterpart
// in the reference, which allocates its scratch per call
// (csrc/marlin.cu:638, torch::empty).
//
// The array's host-side name is not a device address: the set-up (first call
// on each device, that device current) takes its address with
// hipGetSymbolAddress and every later use goes through that pointer.  The
// first call on a device also zero-fills the array with a kernel on the
// caller's stream; after that every launch leaves the state ready for the
// next one (the exchange buffers of the next launch's parity cleared, the
// epochs advanced), so nothing else must start at zero.  All calls on one GPU
// share the array: calls that overlap on one GPU (other streams, other host
// threads) race.
//
// Only the decode kernel's shapes run here (any number of rows, as launches
// of up to 8 rows; no grouped-GEMM prefill and no general fused path, whose
// partial slabs grow with the shape): other shapes are rejected.

#include <mutex>

#include "../../include/gemmainfer_amd.h"
#include "gi_internal.h"

namespace gi {

// The scratch of every call on one GPU (see the header comment).
static __device__ __align__(256) unsigned char scratch[(size_t)2 << 20];

namespace {

constexpr size_t kStaticScratchBytes = (size_t)2 << 20;  // 2 MiB per GPU
constexpr int kMaxDevices = 64;

std::mutex g_mu;
unsigned char* g_scratch[kMaxDevices];  // device address of `scratch` on each device
bool g_zeroed[kMaxDevices];

__global__ __launch_bounds__(256) void zero_fill_kernel(uint4* p, size_t n16) {
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n16; i += (size_t)gridDim.x * 256)
    p[i] = make_uint4(0u, 0u, 0u, 0u);
}

// Address of this device's array (set-up on first use) and, on the first
// call, its zero fill on `stream`.
int static_scratch(hipStream_t stream, unsigned char** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  if (dev < 0 || dev >= kMaxDevices) return fail(GI_ERR_UNSUPPORTED, "fused MoE (static): device index >= 64");
  std::lock_guard<std::mutex> lk(g_mu);
  if (!g_scratch[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) return hip_fail(e, "hipGetSymbolAddress(scratch)");
    g_scratch[dev] = (unsigned char*)p;
  }
  if (!g_zeroed[dev]) {
    hipLaunchKernelGGL(zero_fill_kernel, dim3(256), dim3(256), 0, stream, (uint4*)g_scratch[dev],
                       kStaticScratchBytes / 16);
    e = hipGetLastError();
    if (e != hipSuccess) return hip_fail(e, "fused MoE (static): zero fill launch");
    g_zeroed[dev] = true;
  }
  *out = g_scratch[dev];
  return GI_OK;
}

}  // namespace

int read_static_status(int32_t* host_status, int clear, hipStream_t stream) {
  if (!host_status) return fail(GI_ERR_INVALID_ARG, "fused MoE static status: null pointer");
  *host_status = 0;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  if (dev < 0 || dev >= kMaxDevices) return fail(GI_ERR_UNSUPPORTED, "fused MoE (static): device index >= 64");
  unsigned char* base = nullptr;
  {
    std::lock_guard<std::mutex> lk(g_mu);
    if (!g_zeroed[dev]) return GI_OK;  // no static call has run on this device
    base = g_scratch[dev];
  }
  int32_t v = 0;
  e = hipMemcpyAsync(&v, base, sizeof(int32_t), hipMemcpyDeviceToHost, stream);
  if (e != hipSuccess) return hip_fail(e, "fused MoE static status copy");
  e = hipStreamSynchronize(stream);
  if (e != hipSuccess) return hip_fail(e, "fused MoE static status sync");
  *host_status = v;
  if (clear && v) {
    // after a failed wait the whole scratch goes back to its first-use state
    // (status, epochs and exchange buffers zero), as a fresh workspace would
    hipLaunchKernelGGL(zero_fill_kernel, dim3(256), dim3(256), 0, stream, (uint4*)base, kStaticScratchBytes / 16);
    e = hipGetLastError();
    if (e != hipSuccess) return hip_fail(e, "fused MoE static status clear");
  }
  return GI_OK;
}

int launch_fused_moe_static(MoeHostArgs h) {
  int st = check_moe_args(h);
  if (st != GI_OK) return st;
  h.no_alloc = 1;
  h.workspace = nullptr;
  h.workspace_bytes = 0;
  const bool one = h.M == 1 && moe_decode1_supported(h);
  if (!one && !moe_decode_supported(h))
    return fail(GI_ERR_WORKSPACE,
                "fused MoE (static): this shape needs a caller workspace (gi_fused_batched_moe); the static "
                "2 MiB scratch serves the decode kernel's shapes only (hidden and intermediate sizes multiples "
                "of 32, hidden <= 2816, intermediate <= 768, group size 64 * 2^k, top_k <= 64)");
  const size_t off = moe_decode_scratch_offset();
  if (off + moe_decode_state_bytes() > kStaticScratchBytes)
    return fail(GI_ERR_WORKSPACE, "fused MoE (static): decode state larger than the static scratch");
  if (h.M == 0) return GI_OK;
  unsigned char* base = nullptr;
  st = static_scratch(h.stream, &base);
  if (st != GI_OK) return st;
  if (one) return launch_moe_decode1(h, base + off, (int*)base);
  return launch_moe_decode(h, base + off, (int*)base);
}

}  // namespace gi

extern "C" int gi_fused_batched_moe_static(const void* x, int x_dtype, const int32_t* gu_packed,
                                           const void* gu_scales, int gu_groups, const int32_t* d_packed,
                                           const void* d_scales, int d_groups, const void* idx, int idx_dtype,
                                           const void* w, int w_dtype, void* out, int M, int H, int I, int E,
                                           int top_k, int group_size, int spin_limit, void* stream) {
  if (x_dtype != GI_DTYPE_BF16)
    return gi::fail(GI_ERR_UNSUPPORTED, "fused_batched_moe_static: bf16 activations only");
  if (idx_dtype != GI_DTYPE_INT32 && idx_dtype != GI_DTYPE_INT64)
    return gi::fail(GI_ERR_UNSUPPORTED, "fused_batched_moe_static: expert ids must be int32 or int64");
  if (w_dtype != GI_DTYPE_BF16 && w_dtype != GI_DTYPE_FP16 && w_dtype != GI_DTYPE_FP32)
    return gi::fail(GI_ERR_UNSUPPORTED, "fused_batched_moe_static: expert weights must be bf16, fp16 or fp32");
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
  a.spin_limit = spin_limit;
  a.stream = reinterpret_cast<hipStream_t>(stream);
  return gi::launch_fused_moe_static(a);
}

extern "C" int gi_fused_batched_moe_static_status(int32_t* host_status, int clear, void* stream) {
  return gi::read_static_status(host_status, clear, reinterpret_cast<hipStream_t>(stream));
}
