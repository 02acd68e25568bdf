"""Timed CPU baseline: the reference's PyTorch CPU dequant+matmul path (TEST INFRASTRUCTURE).

Restates, with torch CPU ops and the same sequence of steps, the path the
reference takes when tensors are on the CPU / the extension is absent:

  * W4A16 linear, quant.py:67-75: eight strided passes that dequantise the
    packed weight into a bf16 [K, N] matrix (code - 8, cast, times the scale
    row gathered by group index), then one bf16 ``torch.matmul``.
  * MoE, gemma.py:115-147: for every distinct expert id (``torch.unique``,
    sorted), gather its tokens, gate_up linear, ``chunk(2)``,
    ``F.gelu(tanh) * up``, down linear, ``index_add_`` of ``expert_out * w``.
  * lm_head, gemma.py:351-357 + activations.py:42: linear then cap*tanh(y/cap).

Used only by bench.py's ``cpu_baseline`` leg (and its own test).  It is never
on the product path.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F


def dequant_matmul(x, packed, scales, group_size, out_features):
    """quant.py:67-75 restated: bf16 dequant of the whole weight, then matmul."""
    k = x.shape[1]
    w = torch.empty((k, out_features), dtype=x.dtype)
    rows = torch.arange(k // 8)
    for i in range(8):
        code = ((packed >> (4 * i)) & 0xF) - 8
        grp = (rows * 8 + i) // group_size
        w[i::8, :] = code.to(x.dtype) * scales[grp, :]
    return torch.matmul(x, w)


def moe_forward(x, idx, w, gu_packed, gu_scales, d_packed, d_scales, group_size):
    """gemma.py:115-147 restated (per unique expert, sorted ids)."""
    n_tok, top_k = idx.shape
    n_inter = gu_packed.shape[2] // 2
    hidden = x.shape[1]
    flat = idx.reshape(-1)
    tok_of_slot = torch.arange(n_tok).unsqueeze(1).expand(-1, top_k).reshape(-1)
    w_col = w.reshape(-1, 1)
    out = torch.zeros_like(x)
    for e in torch.unique(flat).tolist():
        sel = flat == e
        toks = tok_of_slot[sel]
        gu = dequant_matmul(x[toks], gu_packed[e], gu_scales[e], group_size, 2 * n_inter)
        gate, up = gu.chunk(2, dim=-1)
        act = F.gelu(gate, approximate="tanh") * up
        y = dequant_matmul(act, d_packed[e], d_scales[e], group_size, hidden)
        out.index_add_(0, toks, y * w_col[sel])
    return out


def lm_head_softcap(x, packed, scales, group_size, cap=30.0):
    """gemma.py:351-357: W4A16 lm_head then the final logit softcap."""
    y = dequant_matmul(x, packed, scales, group_size, packed.shape[1])
    return cap * torch.tanh(y / cap)
