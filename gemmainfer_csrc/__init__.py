"""Drop-in ``gemmainfer_csrc`` module backed by the gfx950 HIP library.

GemmaInfer imports this module by name (``import gemmainfer_csrc`` in
gemmainfer/kernels/{quant,norm,activations,attention}.py, models/gemma.py and
speculative/dspark.py) and calls the five functions its pybind module defines
(csrc/pybind.cpp:273-279) with the same positional arguments.  All return
None and write into caller-owned tensors.

Dispatch matches the reference's ``tensor.is_cuda()`` test: ROCm tensors run
the hand-written HIP kernels through libgemmainfer_amd.so (and raise if it is
missing -- there is no silent fallback), host tensors run the restated CPU
semantics of pybind.cpp.
"""
from __future__ import annotations

from gemmainfer_amd import cpu_ops as _cpu
from gemmainfer_amd import ops as _gpu

__all__ = ["rmsnorm", "fused_rope_inplace", "softcapping", "marlin_w4a16", "fused_batched_moe"]


def rmsnorm(input, weight, output, eps, add_unit_offset):
    """pybind.cpp:137-151 (rmsnorm_dispatch)."""
    if input.is_cuda:
        _gpu.rmsnorm(input, weight, output, eps, add_unit_offset)
    else:
        _cpu.rmsnorm(input, weight, output, eps, add_unit_offset)


def fused_rope_inplace(q, k, cos, sin, position_ids):
    """pybind.cpp:153-167 (fused_rope_inplace_dispatch)."""
    if q.is_cuda:
        _gpu.fused_rope_inplace(q, k, cos, sin, position_ids)
    else:
        _cpu.fused_rope_inplace(q, k, cos, sin, position_ids)


def softcapping(logits, cap):
    """pybind.cpp:169-180 (softcapping_dispatch)."""
    if logits.is_cuda:
        _gpu.softcapping(logits, cap)
    else:
        _cpu.softcapping(logits, cap)


def marlin_w4a16(A, B_packed, scales, C, group_size):
    """pybind.cpp:182-196 (marlin_w4a16_dispatch): C = A @ dequant(B)."""
    if A.is_cuda:
        _gpu.marlin_w4a16(A, B_packed, scales, C, group_size)
    else:
        _cpu.marlin_w4a16(A, B_packed, scales, C, group_size)


def fused_batched_moe(x, gate_up_packed, gate_up_scales, down_packed, down_scales,
                      expert_indices, expert_weights, out, group_size):
    """pybind.cpp:247-271 (fused_batched_moe_dispatch): out += MoE(x)."""
    if x.is_cuda:
        _gpu.fused_batched_moe(x, gate_up_packed, gate_up_scales, down_packed, down_scales,
                               expert_indices, expert_weights, out, group_size)
    else:
        _cpu.fused_batched_moe(x, gate_up_packed, gate_up_scales, down_packed, down_scales,
                               expert_indices, expert_weights, out, group_size)
