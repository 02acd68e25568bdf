"""torch-facing wrappers over the C ABI (device tensors only).

Every function here takes tensors on a ROCm device, checks shapes/dtypes the
way the reference's call sites imply, passes raw pointers plus torch's current
HIP stream to libgemmainfer_amd.so, and never synchronises.  Scratch
("workspace") memory is allocated once per (device, stream) through torch's
caching allocator, zero-filled once, and reused: the kernels leave it zeroed.

Reference entry points mirrored (GemmaInfer paths):
  fused_batched_moe   csrc/pybind.cpp:247-271 -> csrc/marlin.cu:612-702
  marlin_w4a16        csrc/pybind.cpp:182-196 -> csrc/marlin.cu:704-856
  route_topk_softmax  gemmainfer/models/gemma.py:77-80
  softcapping         csrc/pybind.cpp:169-180 -> csrc/softcapping.cu:21-47
  rmsnorm             csrc/pybind.cpp:137-151 -> csrc/rmsnorm.cu:75-114
  fused_rope_inplace  csrc/pybind.cpp:153-167 -> csrc/rmsnorm.cu:166-231
"""
from __future__ import annotations

import ctypes
import threading
from typing import Optional

import torch

from . import _lib as L

_DTYPE_CODE = {
    torch.bfloat16: L.DTYPE_BF16,
    torch.float16: L.DTYPE_FP16,
    torch.float32: L.DTYPE_FP32,
    torch.int32: L.DTYPE_INT32,
    torch.int64: L.DTYPE_INT64,
}


def _ptr(t: Optional[torch.Tensor]):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(device: torch.device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _require(cond: bool, msg: str, exc=ValueError) -> None:
    if not cond:
        raise exc(msg)


def _on_device(*tensors: torch.Tensor) -> torch.device:
    dev = tensors[0].device
    for t in tensors:
        _require(t.is_cuda, "gemmainfer_amd ops take ROCm device tensors only", TypeError)
        _require(t.device == dev, f"all tensors must be on {dev}, got {t.device}")
    return dev


# ---------------------------------------------------------------------------
# workspaces
# ---------------------------------------------------------------------------
class _WorkspacePool:
    """One zero-filled uint8 buffer per (kind, device, stream), grown on demand."""

    def __init__(self):
        self._bufs: dict[tuple, torch.Tensor] = {}
        self._lock = threading.Lock()

    def get(self, kind: str, device: torch.device, nbytes: int) -> torch.Tensor:
        stream = torch.cuda.current_stream(device).cuda_stream
        key = (kind, device.index, stream)
        with self._lock:
            buf = self._bufs.get(key)
            if buf is None or buf.numel() < nbytes:
                size = max(nbytes, 1 << 16)
                size = (size + 4095) // 4096 * 4096
                buf = torch.zeros(size, dtype=torch.uint8, device=device)
                self._bufs[key] = buf
            return buf

    def all(self, kind: str, device: torch.device):
        with self._lock:
            return [b for (k, d, _), b in self._bufs.items() if k == kind and d == device.index]


_WS = _WorkspacePool()


def _device_index(device) -> int:
    if device is None:
        return torch.cuda.current_device()
    d = torch.device(device)
    return torch.cuda.current_device() if d.index is None else d.index


def workspace_status(device=None) -> int:
    """OR of the device status words of every MoE workspace on ``device`` and
    of the device's host-visible error flag, clearing them (synchronises).
    0 means no kernel reported an error (``gemmainfer_amd._lib.DEVICE_SPIN_TIMEOUT``
    = a bounded wait gave up)."""
    device = torch.device("cuda", _device_index(device))
    lib = L.load()
    out = 0
    for buf in _WS.all("moe", device):
        st = ctypes.c_int32(0)
        L.check(lib.gi_workspace_status(_ptr(buf), buf.numel(), ctypes.byref(st), _stream(device)),
                "workspace_status")
        out |= st.value
    flags = lib.gi_device_error_flags(device.index, 1)
    return out | max(flags, 0)


def raise_pending_device_error(device=None) -> None:
    """Raise GIError(GI_ERR_DEVICE) if a kernel on ``device`` reported an error
    since the last check.  Reads a host-memory flag the kernels write: no
    synchronisation.  The MoE entry points call it before launching, so a
    failure surfaces at the next call (the failed call's outputs that could
    not be completed hold NaN).  The device's MoE workspaces are re-zeroed."""
    idx = _device_index(device)
    flags = L.load().gi_device_error_flags(idx, 1)
    if flags > 0:
        for buf in _WS.all("moe", torch.device("cuda", idx)):
            buf.zero_()
        raise L.GIError(L.GI_ERR_DEVICE,
                        f"a MoE kernel on cuda:{idx} reported device error bits {flags:#x} "
                        "(a bounded wait gave up; the outputs it could not complete hold NaN)")


# ---------------------------------------------------------------------------
# MoE
# ---------------------------------------------------------------------------
def _moe_weight_shapes(x, gu_packed, gu_scales, d_packed, d_scales):
    _require(x.dim() == 2, f"x must be [M, H], got {tuple(x.shape)}")
    m, h = x.shape
    _require(gu_packed.dim() == 3 and gu_packed.dtype == torch.int32,
             "gate_up_packed must be int32 [E, H/8, 2I]")
    e, hp, two_i = gu_packed.shape
    _require(hp * 8 == h, f"gate_up_packed.shape[1]*8 ({hp * 8}) must equal H ({h})")
    _require(two_i % 2 == 0, "gate_up_packed last dim must be 2*I")
    i = two_i // 2
    _require(gu_scales.dim() == 3 and gu_scales.shape[0] == e and gu_scales.shape[2] == two_i,
             f"gate_up_scales must be [E, groups, 2I], got {tuple(gu_scales.shape)}")
    _require(d_packed.dim() == 3 and d_packed.dtype == torch.int32 and
             tuple(d_packed.shape) == (e, i // 8, h),
             f"down_packed must be int32 [E, I/8, H] = {(e, i // 8, h)}, got {tuple(d_packed.shape)}")
    _require(d_scales.dim() == 3 and d_scales.shape[0] == e and d_scales.shape[2] == h,
             f"down_scales must be [E, groups, H], got {tuple(d_scales.shape)}")
    for name, t in (("gate_up_scales", gu_scales), ("down_scales", d_scales)):
        _require(t.dtype == x.dtype, f"{name} dtype {t.dtype} must match x dtype {x.dtype}", TypeError)
    for name, t in (("gate_up_packed", gu_packed), ("gate_up_scales", gu_scales),
                    ("down_packed", d_packed), ("down_scales", d_scales)):
        _require(t.is_contiguous(), f"{name} must be contiguous")
    return m, h, i, e


def _require_bf16(x: torch.Tensor, who: str) -> None:
    if x.dtype != torch.bfloat16:
        raise NotImplementedError(
            f"{who}: the gfx950 kernels implement bf16 activations; got {x.dtype}")


_ACT_DTYPES = (torch.bfloat16, torch.float16, torch.float32)


def _require_act_dtype(x: torch.Tensor, who: str) -> None:
    """bf16, fp16 or fp32 activations (the reference's dispatch, marlin.cu:694-700,
    :764-842): bf16 runs the tuned kernels, fp16 and fp32 VALU kernels."""
    if x.dtype not in _ACT_DTYPES:
        raise TypeError(f"{who}: activations must be bf16, fp16 or fp32; got {x.dtype}")


def fused_batched_moe(x, gate_up_packed, gate_up_scales, down_packed, down_scales,
                      expert_indices, expert_weights, out, group_size, *, spin_limit: int = 0):
    """out += sum over slots of w * expert(x)  (drop-in for gemmainfer_csrc.fused_batched_moe).

    Semantics of the reference (csrc/marlin.cu:612-702): M = x.size(0),
    top_k = numel(expert_indices) / M, ids outside [0, E) are skipped, the
    weights are cast to x's dtype, and the result is ADDED to ``out`` (the
    caller zeroes it, gemma.py:82).  Unlike the reference there is no cap on
    how many slots share an expert (marlin.cu:325) and no 128-slot limit
    (:300); the combine is a fixed-order fp32 sum with one rounding to x's
    dtype.  x, the scales and out are bf16, fp16 or fp32 (all the same).
    """
    dev = _on_device(x, gate_up_packed, gate_up_scales, down_packed, down_scales,
                     expert_indices, expert_weights, out)
    raise_pending_device_error(dev)
    _require_act_dtype(x, "fused_batched_moe")
    m, h, i, e = _moe_weight_shapes(x, gate_up_packed, gate_up_scales, down_packed, down_scales)
    _require(isinstance(group_size, int) and group_size > 0 and group_size % 8 == 0,
             f"group_size must be a positive multiple of 8, got {group_size}")
    _require(tuple(out.shape) == (m, h), f"out must be [M, H] = {(m, h)}, got {tuple(out.shape)}")
    _require(out.dtype == x.dtype, "out dtype must match x", TypeError)
    if m == 0:
        return
    n_slots = expert_indices.numel()
    _require(n_slots % m == 0 and n_slots > 0,
             f"numel(expert_indices) ({n_slots}) must be a positive multiple of M ({m})")
    top_k = n_slots // m
    _require(expert_weights.numel() == n_slots,
             f"expert_weights has {expert_weights.numel()} elements, expected {n_slots}")
    idx = expert_indices
    if idx.dtype not in (torch.int32, torch.int64):
        idx = idx.to(torch.int32)
    idx = idx.contiguous()
    w = expert_weights
    if w.dtype not in (torch.bfloat16, torch.float16, torch.float32):
        w = w.to(torch.float32)
    w = w.contiguous()
    xc = x.contiguous()
    oc = out if out.is_contiguous() else out.contiguous()
    lib = L.load()
    nbytes = lib.gi_fused_moe_workspace_bytes(m, top_k, h, i, e)
    ws = _WS.get("moe", dev, nbytes)
    L.check(lib.gi_fused_batched_moe(
        _ptr(xc), _DTYPE_CODE[x.dtype], _ptr(gate_up_packed), _ptr(gate_up_scales),
        gate_up_scales.shape[1], _ptr(down_packed), _ptr(down_scales), down_scales.shape[1],
        _ptr(idx), _DTYPE_CODE[idx.dtype], _ptr(w), _DTYPE_CODE[w.dtype], _ptr(oc),
        m, h, i, e, top_k, int(group_size), _ptr(ws), ws.numel(), int(spin_limit),
        _stream(dev)), "fused_batched_moe")
    if oc is not out:
        out.copy_(oc)


def moe_layer(x, router_logits, gate_up_packed, gate_up_scales, down_packed, down_scales,
              top_k, group_size, expert_scale=None, out=None, *, spin_limit: int = 0):
    """Router tail + fused MoE (gemma.py:77-98): one launch per 8 rows up to
    63 rows, and from 64 rows the grouped-GEMM prefill path (routing, align,
    gate/up, down and combine launches).

    Returns (out [M, H] bf16 -- overwritten, idx int32 [M, top_k],
    weights bf16 [M, top_k]).
    """
    dev = _on_device(x, router_logits, gate_up_packed, gate_up_scales, down_packed, down_scales)
    raise_pending_device_error(dev)
    _require_bf16(x, "moe_layer")
    m, h, i, e = _moe_weight_shapes(x, gate_up_packed, gate_up_scales, down_packed, down_scales)
    _require(router_logits.dim() == 2 and tuple(router_logits.shape) == (m, e),
             f"router_logits must be [M, E] = {(m, e)}, got {tuple(router_logits.shape)}")
    _require(router_logits.dtype in (torch.bfloat16, torch.float32),
             "router_logits must be bf16 or fp32", TypeError)
    _require(0 < top_k <= min(e, 64), f"top_k must be in [1, min(E, 64)], got {top_k}")
    if expert_scale is not None:
        _on_device(x, expert_scale)
        _require(expert_scale.numel() == e, "expert_scale must have E elements")
        expert_scale = expert_scale.to(torch.float32).contiguous()
    if out is None:
        out = torch.empty_like(x)
    _require(tuple(out.shape) == (m, h) and out.dtype == x.dtype and out.is_contiguous(),
             "out must be a contiguous bf16 [M, H] tensor")
    idx = torch.empty((m, top_k), dtype=torch.int32, device=dev)
    w = torch.empty((m, top_k), dtype=torch.bfloat16, device=dev)
    if m == 0:
        return out, idx, w
    logits = router_logits.contiguous()
    lib = L.load()
    nbytes = lib.gi_fused_moe_workspace_bytes(m, top_k, h, i, e)
    ws = _WS.get("moe", dev, nbytes)
    L.check(lib.gi_moe_layer_from_logits(
        _ptr(x.contiguous()), L.DTYPE_BF16, _ptr(logits), _DTYPE_CODE[logits.dtype],
        _ptr(expert_scale), _ptr(gate_up_packed), _ptr(gate_up_scales), gate_up_scales.shape[1],
        _ptr(down_packed), _ptr(down_scales), down_scales.shape[1], _ptr(out), _ptr(idx),
        _ptr(w), m, h, i, e, int(top_k), int(group_size), _ptr(ws), ws.numel(),
        int(spin_limit), _stream(dev)), "moe_layer")
    return out, idx, w


def _router_inputs(x, router_scale, gate_weight, who):
    dev = _on_device(x, gate_weight)
    _require_bf16(x, who)
    _require(x.dim() == 2, f"{who}: x must be [M, H]")
    m, h = x.shape
    _require(gate_weight.dim() == 2 and gate_weight.shape[1] == h,
             f"{who}: gate weight must be [E, H={h}], got {tuple(gate_weight.shape)}")
    _require(gate_weight.dtype == torch.bfloat16, f"{who}: gate weight must be bf16", TypeError)
    if router_scale is not None:
        _on_device(x, router_scale)
        _require(router_scale.numel() == h and router_scale.dtype == torch.bfloat16,
                 f"{who}: router_scale must be a bf16 tensor of H={h} elements")
        router_scale = router_scale.contiguous()
    return dev, m, h, gate_weight.shape[0], router_scale


def moe_router_logits(x, router_scale, gate_weight, eps: float = 1e-6):
    """Router front-end of GemmaBatchedMoE.forward (gemma.py:75-76) in one launch:
    bf16 logits [M, E] of the gate linear applied to
    router_norm(x) * (router_scale * H**-0.5), with the bf16 roundings of the
    bf16 model (norm output, scaled router_scale, their product, the logits).
    ``router_scale`` may be None (ones); ``gate_weight`` is the nn.Linear weight
    [E, H]."""
    dev, m, h, e, rs = _router_inputs(x, router_scale, gate_weight, "moe_router_logits")
    logits = torch.empty((m, e), dtype=torch.bfloat16, device=dev)
    if m == 0:
        return logits
    L.check(L.load().gi_moe_router_logits(
        _ptr(x.contiguous()), L.DTYPE_BF16, _ptr(rs), _ptr(gate_weight.contiguous()), float(eps),
        _ptr(logits), m, h, e, _stream(dev)), "moe_router_logits")
    return logits


def moe_layer_from_hidden(x, router_scale, gate_weight, gate_up_packed, gate_up_scales,
                          down_packed, down_scales, top_k, group_size, expert_scale=None,
                          eps: float = 1e-6, out=None, *, spin_limit: int = 0):
    """GemmaBatchedMoE.forward (gemma.py:75-98) from the hidden state: the router
    front-end (one launch) feeding ``moe_layer`` on the logits it writes.

    Returns (out [M, H] bf16 -- overwritten, idx int32 [M, top_k],
    weights bf16 [M, top_k], logits bf16 [M, E]).
    """
    dev, m, h, e, rs = _router_inputs(x, router_scale, gate_weight, "moe_layer_from_hidden")
    raise_pending_device_error(dev)
    _on_device(x, gate_up_packed, gate_up_scales, down_packed, down_scales)
    m2, h2, i, e2 = _moe_weight_shapes(x, gate_up_packed, gate_up_scales, down_packed, down_scales)
    _require(e2 == e, f"gate weight has {e} experts, the expert weights {e2}")
    _require(0 < top_k <= min(e, 64), f"top_k must be in [1, min(E, 64)], got {top_k}")
    if expert_scale is not None:
        _on_device(x, expert_scale)
        _require(expert_scale.numel() == e, "expert_scale must have E elements")
        expert_scale = expert_scale.to(torch.float32).contiguous()
    if out is None:
        out = torch.empty_like(x)
    _require(tuple(out.shape) == (m, h) and out.dtype == x.dtype and out.is_contiguous(),
             "out must be a contiguous bf16 [M, H] tensor")
    idx = torch.empty((m, top_k), dtype=torch.int32, device=dev)
    w = torch.empty((m, top_k), dtype=torch.bfloat16, device=dev)
    logits = torch.empty((m, e), dtype=torch.bfloat16, device=dev)
    if m == 0:
        return out, idx, w, logits
    lib = L.load()
    nbytes = lib.gi_fused_moe_workspace_bytes(m, top_k, h, i, e)
    ws = _WS.get("moe", dev, nbytes)
    L.check(lib.gi_moe_layer_from_hidden(
        _ptr(x.contiguous()), L.DTYPE_BF16, _ptr(rs), _ptr(gate_weight.contiguous()), float(eps),
        _ptr(logits), _ptr(expert_scale), _ptr(gate_up_packed), _ptr(gate_up_scales),
        gate_up_scales.shape[1], _ptr(down_packed), _ptr(down_scales), down_scales.shape[1],
        _ptr(out), _ptr(idx), _ptr(w), m, h, i, e, int(top_k), int(group_size), _ptr(ws),
        ws.numel(), int(spin_limit), _stream(dev)), "moe_layer_from_hidden")
    return out, idx, w, logits


def route_topk_softmax(router_logits, top_k, expert_scale=None, out_dtype=torch.bfloat16):
    """idx int32 [M, k], w [M, k] = softmax_fp32(topk(logits)) * expert_scale, cast
    to out_dtype (gemma.py:77-80; ties -> lower expert index)."""
    dev = _on_device(router_logits)
    _require(router_logits.dim() == 2, "router_logits must be [M, E]")
    _require(router_logits.dtype in (torch.bfloat16, torch.float32),
             "router_logits must be bf16 or fp32", TypeError)
    m, e = router_logits.shape
    _require(0 < top_k <= min(e, 64), f"top_k must be in [1, min(E, 64)], got {top_k}")
    if expert_scale is not None:
        _on_device(router_logits, expert_scale)
        expert_scale = expert_scale.to(torch.float32).contiguous()
    idx = torch.empty((m, top_k), dtype=torch.int32, device=dev)
    w = torch.empty((m, top_k), dtype=out_dtype, device=dev)
    logits = router_logits.contiguous()
    L.check(L.load().gi_moe_route_topk_softmax(
        _ptr(logits), _DTYPE_CODE[logits.dtype], _ptr(expert_scale), m, e, int(top_k), _ptr(idx),
        _ptr(w), _DTYPE_CODE[out_dtype], _stream(dev)), "route_topk_softmax")
    return idx, w


def moe_align(expert_indices, num_experts):
    """Token-Union alignment of a [M, top_k] id tensor: dict of unique_experts,
    num_unique, slot_to_unique, offsets, slots (int32 device tensors; entries
    past num_unique are unspecified)."""
    dev = _on_device(expert_indices)
    _require(expert_indices.dim() == 2, "expert_indices must be [M, top_k]")
    m, k = expert_indices.shape
    idx = expert_indices
    if idx.dtype not in (torch.int32, torch.int64):
        idx = idx.to(torch.int32)
    idx = idx.contiguous()
    s = m * k
    umax = min(s, num_experts)
    res = {
        "unique_experts": torch.full((umax,), -1, dtype=torch.int32, device=dev),
        "num_unique": torch.zeros((1,), dtype=torch.int32, device=dev),
        "slot_to_unique": torch.empty((s,), dtype=torch.int32, device=dev),
        "offsets": torch.zeros((umax + 1,), dtype=torch.int32, device=dev),
        "slots": torch.full((s,), -1, dtype=torch.int32, device=dev),
    }
    L.check(L.load().gi_moe_align(
        _ptr(idx), _DTYPE_CODE[idx.dtype], m, k, int(num_experts), _ptr(res["unique_experts"]),
        _ptr(res["num_unique"]), _ptr(res["slot_to_unique"]), _ptr(res["offsets"]),
        _ptr(res["slots"]), _stream(dev)), "moe_align")
    return res


# ---------------------------------------------------------------------------
# W4A16 linear
# ---------------------------------------------------------------------------
def marlin_w4a16(A, B_packed, scales, C, group_size, softcap: float = 0.0):
    """C = A @ dequant(B_packed, scales)  (drop-in for gemmainfer_csrc.marlin_w4a16).

    Overwrites C (reference marlin.cu:704-856).  ``softcap > 0`` fuses the
    final-logit softcap cap*tanh(C/cap) (gemma.py:356-357).
    """
    dev = _on_device(A, B_packed, scales, C)
    _require_act_dtype(A, "marlin_w4a16")
    _require(A.dim() == 2, f"A must be [M, K], got {tuple(A.shape)}")
    m, k = A.shape
    _require(B_packed.dim() == 2 and B_packed.dtype == torch.int32 and B_packed.shape[0] * 8 == k,
             f"B_packed must be int32 [K/8, N] with K={k}, got {tuple(B_packed.shape)}")
    n = B_packed.shape[1]
    _require(scales.dim() == 2 and scales.shape[1] == n and scales.dtype == A.dtype,
             f"scales must be [groups, N={n}] of A's dtype")
    _require(tuple(C.shape) == (m, n) and C.dtype == A.dtype,
             f"C must be [M, N] = {(m, n)} of A's dtype")
    _require(B_packed.is_contiguous() and scales.is_contiguous(), "B_packed/scales must be contiguous")
    _require(isinstance(group_size, int) and group_size > 0 and group_size % 8 == 0,
             f"group_size must be a positive multiple of 8, got {group_size}")
    if m == 0:
        return
    Ac = A.contiguous()
    Cc = C if C.is_contiguous() else torch.empty_like(C, memory_format=torch.contiguous_format)
    lib = L.load()
    nbytes = lib.gi_w4a16_workspace_bytes(m, k, n, group_size)
    ws = _WS.get("w4a16", dev, nbytes) if nbytes else None
    L.check(lib.gi_w4a16_linear(
        _ptr(Ac), _DTYPE_CODE[A.dtype], _ptr(B_packed), _ptr(scales), scales.shape[0], _ptr(Cc), m, k, n,
        int(group_size), float(softcap), _ptr(ws), 0 if ws is None else ws.numel(), _stream(dev)),
        "marlin_w4a16")
    if Cc is not C:
        C.copy_(Cc)


def w4a16_linear(A, B_packed, scales, group_size, softcap: Optional[float] = None):
    """Allocating form of marlin_w4a16; ``softcap`` fuses cap*tanh(y/cap)."""
    C = torch.empty((A.shape[0], B_packed.shape[1]), dtype=A.dtype, device=A.device)
    marlin_w4a16(A, B_packed, scales, C, group_size, softcap=float(softcap or 0.0))
    return C


def _linear_operands(A, B_packed, scales, who):
    _require(B_packed.dim() == 2 and B_packed.dtype == torch.int32 and B_packed.shape[0] * 8 == A.shape[1],
             f"{who}: B_packed must be int32 [K/8, N] with K={A.shape[1]}, got {tuple(B_packed.shape)}")
    _require(scales.dim() == 2 and scales.shape[1] == B_packed.shape[1] and scales.dtype == A.dtype,
             f"{who}: scales must be [groups, N] of A's dtype")
    _require(B_packed.is_contiguous() and scales.is_contiguous(), f"{who}: B_packed/scales must be contiguous")


def w4a16_linear_multi(A, weights, group_size):
    """Several W4A16 projections of the same rows (the q, k, v marlin_w4a16 calls
    of attention.py:115-122) in one call: one launch for one or two rows.
    ``weights`` is a list of up to 4 (B_packed, scales); returns the outputs."""
    dev = _on_device(A, *[t for w in weights for t in w])
    _require_bf16(A, "w4a16_linear_multi")
    _require(A.dim() == 2, "A must be [M, K]")
    _require(1 <= len(weights) <= 4, "1 to 4 projections")
    m, k = A.shape
    for B, S in weights:
        _linear_operands(A, B, S, "w4a16_linear_multi")
    outs = [torch.empty((m, B.shape[1]), dtype=A.dtype, device=dev) for B, _ in weights]
    if m == 0:
        return outs
    lib = L.load()
    n = len(weights)
    nbytes = lib.gi_w4a16_linear_multi_workspace_bytes(n, (ctypes.c_int * n)(*[B.shape[1] for B, _ in weights]),
                                                       m, k, int(group_size))
    ws = _WS.get("w4a16", dev, nbytes) if nbytes else None
    arr = lambda vals: (ctypes.c_void_p * n)(*[v.data_ptr() for v in vals])  # noqa: E731
    L.check(lib.gi_w4a16_linear_multi(
        _ptr(A.contiguous()), L.DTYPE_BF16, n, arr([B for B, _ in weights]), arr([S for _, S in weights]),
        (ctypes.c_int * n)(*[S.shape[0] for _, S in weights]), arr(outs),
        (ctypes.c_int * n)(*[B.shape[1] for B, _ in weights]), m, k, int(group_size), _ptr(ws),
        0 if ws is None else ws.numel(), _stream(dev)), "w4a16_linear_multi")
    return outs


def gated_mlp_act(A, gate, up, group_size):
    """GemmaMLP's ``gelu_tanh(gate_proj(x)) * up_proj(x)`` (activations.py:26-28)
    with the bf16 roundings of those torch statements; one launch for one or
    two rows.  ``gate`` and ``up`` are (B_packed, scales); returns bf16 [M, N]."""
    dev = _on_device(A, *gate, *up)
    _require_bf16(A, "gated_mlp_act")
    _require(A.dim() == 2, "A must be [M, K]")
    _linear_operands(A, *gate, "gated_mlp_act")
    _linear_operands(A, *up, "gated_mlp_act")
    _require(gate[0].shape == up[0].shape, "gate and up projections must have the same shape")
    m, k = A.shape
    n = gate[0].shape[1]
    out = torch.empty((m, n), dtype=A.dtype, device=dev)
    if m == 0:
        return out
    lib = L.load()
    nbytes = lib.gi_w4a16_gated_mlp_workspace_bytes(m, k, n, group_size)
    ws = _WS.get("w4a16", dev, nbytes) if nbytes else None
    L.check(lib.gi_w4a16_gated_mlp(
        _ptr(A.contiguous()), L.DTYPE_BF16, _ptr(gate[0]), _ptr(gate[1]), gate[1].shape[0], _ptr(up[0]),
        _ptr(up[1]), up[1].shape[0], _ptr(out), m, k, n, int(group_size), _ptr(ws),
        0 if ws is None else ws.numel(), _stream(dev)), "gated_mlp_act")
    return out


# ---------------------------------------------------------------------------
# companions
# ---------------------------------------------------------------------------
def softcapping(logits, cap: float):
    dev = _on_device(logits)
    _require(logits.dtype in (torch.bfloat16, torch.float16, torch.float32),
             "softcapping: bf16/fp16/fp32 only", TypeError)
    t = logits if logits.is_contiguous() else logits.contiguous()
    L.check(L.load().gi_softcap_inplace(_ptr(t), _DTYPE_CODE[t.dtype], t.numel(), float(cap),
                                        _stream(dev)), "softcapping")
    if t is not logits:
        logits.copy_(t)


def rmsnorm(input, weight, output, eps: float, add_unit_offset: bool):
    dev = _on_device(input, output)
    _require(input.dtype in (torch.bfloat16, torch.float16, torch.float32),
             "rmsnorm: bf16/fp16/fp32 only", TypeError)
    _require(output.shape == input.shape and output.dtype == input.dtype, "rmsnorm: output mismatch")
    hidden = input.shape[-1]
    x = input.contiguous()
    has_w = weight is not None and weight.numel() > 0
    w = None
    if has_w:
        _on_device(input, weight)
        _require(weight.numel() == hidden, "rmsnorm: weight must have hidden elements")
        w = weight.to(input.dtype).contiguous()
    o = output if output.is_contiguous() else torch.empty_like(output, memory_format=torch.contiguous_format)
    L.check(L.load().gi_rmsnorm(_ptr(x), _ptr(w), _ptr(o), _DTYPE_CODE[x.dtype],
                                x.numel() // hidden if hidden else 0, hidden, float(eps),
                                int(bool(add_unit_offset)), _stream(dev)), "rmsnorm")
    if o is not output:
        output.copy_(o)


def fused_rope_inplace(q, k, cos, sin, position_ids):
    dev = _on_device(q, cos, sin, position_ids)
    _require(q.dim() == 4, "q must be [B, Hq, S, D]")
    _require(q.stride(-1) == 1, "q's last dimension must be contiguous")
    b, hq, s, d = q.shape
    has_k = k is not None and k.numel() > 0
    if has_k:
        _on_device(q, k)
        _require(k.dim() == 4 and k.shape[0] == b and k.shape[2] == s and k.shape[3] == d
                 and k.dtype == q.dtype and k.stride(-1) == 1, "k must be [B, Hk, S, D] like q")
    c = cos.to(q.dtype).contiguous()
    sn = sin.to(q.dtype).contiguous()
    pos = position_ids.to(torch.int64).contiguous()
    _require(pos.numel() == b * s, "position_ids must have B*S elements")
    ks = k.stride()[:3] if has_k else (0, 0, 0)
    L.check(L.load().gi_rope_inplace(
        _ptr(q), _ptr(k) if has_k else None, _ptr(c), _ptr(sn), _ptr(pos), _DTYPE_CODE[q.dtype],
        b, hq, k.shape[1] if has_k else 0, s, d, q.stride(0), q.stride(1), q.stride(2),
        ks[0], ks[1], ks[2], _stream(dev)), "fused_rope_inplace")
