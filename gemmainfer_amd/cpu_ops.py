"""CPU-tensor behaviour of the reference extension (host tensors ONLY).

The reference's ``gemmainfer_csrc`` dispatches on ``tensor.is_cuda()``: CPU
tensors go to scalar C++ fallbacks in csrc/pybind.cpp, and its CPU test-suite
and engine rely on that (e.g. GemmaBatchedMoE calls fused_batched_moe on CPU
tensors, gemma.py:85-98).  This module restates those fallbacks with torch CPU
ops so the drop-in keeps working for host tensors.  It is never used for
device tensors: ``gemmainfer_csrc`` routes a ROCm tensor to the HIP library
or raises.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F


def _dequant_f32(packed: torch.Tensor, scales: torch.Tensor, group_size: int) -> torch.Tensor:
    """fp32 [K, N] weights (code-8)*scale, scale row = (8*pk)//group_size
    (pybind.cpp:67-79 indexes the group by the word's first k)."""
    kp, n = packed.shape
    s = scales.to(torch.float32)
    grp = (torch.arange(kp) * 8) // group_size
    if kp and int(grp[-1]) >= s.shape[0]:
        raise IndexError(
            f"scales has {s.shape[0]} groups but K={8 * kp} with group_size={group_size} needs "
            f"{int(grp[-1]) + 1}")
    s_rows = s[grp]  # [kp, N]
    shifts = torch.arange(8, dtype=torch.int32) * 4
    codes = (packed.unsqueeze(1) >> shifts.view(1, 8, 1)) & 0xF  # [kp, 8, N]
    w = (codes.to(torch.float32) - 8.0) * s_rows.unsqueeze(1)
    return w.reshape(kp * 8, n)


def marlin_w4a16(A, B_packed, scales, C, group_size):
    """pybind.cpp:46-85: fp32 dequant-and-accumulate, then C.copy_(result)."""
    y = A.to(torch.float32) @ _dequant_f32(B_packed, scales, group_size)
    C.copy_(y.to(C.dtype))


def fused_batched_moe(x, gate_up_packed, gate_up_scales, down_packed, down_scales,
                      expert_indices, expert_weights, out, group_size):
    """pybind.cpp:198-245: per slot, gate_up -> gelu_tanh(gate)*up -> down,
    then out[token].add_(y, alpha=w) in slot order."""
    m = x.shape[0]
    two_i = gate_up_packed.shape[2]
    n_inter = two_i // 2
    flat = expert_indices.reshape(-1).to(torch.int64)
    w = expert_weights.reshape(-1).to(torch.float32)
    top_k = flat.numel() // m
    cache = {}
    for t in range(m):
        for k in range(top_k):
            s = t * top_k + k
            e = int(flat[s])
            if e not in cache:
                cache[e] = (_dequant_f32(gate_up_packed[e], gate_up_scales[e], group_size),
                            _dequant_f32(down_packed[e], down_scales[e], group_size))
            wgu, wd = cache[e]
            gu = (x[t:t + 1].to(torch.float32) @ wgu).to(x.dtype)
            act = F.gelu(gu[:, :n_inter], approximate="tanh") * gu[:, n_inter:two_i]
            y = (act.to(torch.float32) @ wd).to(x.dtype)
            out[t:t + 1].add_(y, alpha=float(w[s]))


def rmsnorm(input, weight, output, eps, add_unit_offset):
    """pybind.cpp:87-104."""
    x = input.reshape(-1, input.shape[-1]).to(torch.float32)
    r = torch.rsqrt((x * x).mean(-1, keepdim=True) + eps)
    y = x * r
    if weight is not None and weight.numel() > 0:
        wf = weight.to(torch.float32)
        y = y * ((1.0 + wf) if add_unit_offset else wf)
    output.copy_(y.view_as(output))


def fused_rope_inplace(q, k, cos, sin, position_ids):
    """pybind.cpp:106-128 (rotate-half)."""
    half = q.shape[-1] // 2
    c = cos[position_ids].unsqueeze(1)
    s = sin[position_ids].unsqueeze(1)

    def rot(t):
        return torch.cat((-t[..., half:], t[..., :half]), dim=-1)

    q.copy_(q * c + rot(q) * s)
    if k is not None and k.numel() > 0:
        k.copy_(k * c + rot(k) * s)


def softcapping(logits, cap):
    """pybind.cpp:130-135."""
    logits.copy_(cap * torch.tanh(logits / cap))
