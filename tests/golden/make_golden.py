"""Writes tests/golden/*.npz: input/output vectors of the reference's own CPU
C++ fallback (csrc/pybind.cpp, compiled from the reference tree into
oracle/_ref by oracle/Makefile).

The reference's test-suite holds no golden vectors for this path, so these
fixtures are the reference-produced known answers the oracle and the HIP
kernels are checked against.  Run in the build container (where the
reference tree exists):  make -C oracle && python tests/golden/make_golden.py

bf16 tensors are stored as their uint16 bit patterns (``*_bf16`` keys).
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT / "oracle" / "_ref"))
sys.path.insert(0, str(ROOT))

import gemmainfer_csrc_ref as R  # noqa: E402  (reference CPU fallback, built from source)

from gemmainfer_amd import synth  # noqa: E402

OUT = Path(__file__).resolve().parent


def bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def linear_case(name, m, k, n, gs, seed):
    B, S = synth.linear_weights(k, n, gs, seed=seed)
    A = synth.activations(m, k, seed=seed)
    C = torch.empty(m, n, dtype=torch.bfloat16)
    R.marlin_w4a16(A, B, S, C, gs)  # pybind.cpp:46-85
    np.savez_compressed(OUT / f"{name}.npz", A_bf16=bits(A), B_packed=B.numpy(), scales_bf16=bits(S),
                        C_bf16=bits(C), group_size=np.int32(gs))


def moe_case(name, m, h, i, e, top_k, gs, seed, idx=None):
    W = synth.moe_weights(e, h, i, gs, seed=seed)
    x = synth.activations(m, h, seed=seed)
    if idx is None:
        logits = synth.router_logits(m, e, seed=seed)
        top, idx = torch.topk(logits, top_k, dim=-1)
        w = torch.softmax(top, dim=-1, dtype=torch.float32).to(torch.bfloat16)
    else:
        idx = torch.tensor(idx, dtype=torch.int64)
        w = torch.softmax(torch.randn(idx.shape, generator=torch.Generator().manual_seed(seed)),
                          dim=-1).to(torch.bfloat16)
    idx32 = idx.to(torch.int32)
    out = torch.zeros(m, h, dtype=torch.bfloat16)
    R.fused_batched_moe(x, W["gate_up_packed"], W["gate_up_scales"], W["down_packed"],
                        W["down_scales"], idx32, w, out, gs)  # pybind.cpp:198-245
    np.savez_compressed(
        OUT / f"{name}.npz", x_bf16=bits(x), gate_up_packed=W["gate_up_packed"].numpy(),
        gate_up_scales_bf16=bits(W["gate_up_scales"]), down_packed=W["down_packed"].numpy(),
        down_scales_bf16=bits(W["down_scales"]), idx=idx32.numpy(), w_bf16=bits(w),
        out_bf16=bits(out), group_size=np.int32(gs))


def dtype_cases():
    """fp16 and fp32 activations (the reference dispatches all three dtypes,
    marlin.cu:694-700 and :764-842; its CPU fallback computes in float32 and
    stores in the tensors' dtype, pybind.cpp:46-85,198-245): one linear and
    one MoE call with duplicate ids per dtype, stored as float16 / float32
    arrays."""
    for dt, tag in ((torch.float16, "fp16"), (torch.float32, "fp32")):
        B, S = synth.linear_weights(512, 128, 128, seed=11)
        A = synth.activations(3, 512, seed=11).to(dt)
        S = S.to(dt)
        C = torch.empty(3, 128, dtype=dt)
        R.marlin_w4a16(A, B, S, C, 128)
        np.savez_compressed(OUT / f"linear_m3_k512_n128_gs128_{tag}.npz", A=A.numpy(), B_packed=B.numpy(),
                            scales=S.numpy(), C=C.numpy(), group_size=np.int32(128))
        W = synth.moe_weights(8, 256, 128, 64, seed=12)
        x = synth.activations(3, 256, seed=12).to(dt)
        idx = torch.tensor([[1, 1, 2, 3], [2, 5, 5, 5], [0, 7, 1, 2]], dtype=torch.int32)
        w = torch.softmax(torch.randn(idx.shape, generator=torch.Generator().manual_seed(12)), dim=-1).to(dt)
        gus, dns = W["gate_up_scales"].to(dt), W["down_scales"].to(dt)
        out = torch.zeros(3, 256, dtype=dt)
        R.fused_batched_moe(x, W["gate_up_packed"], gus, W["down_packed"], dns, idx, w, out, 64)
        np.savez_compressed(OUT / f"moe_m3_dups_gs64_{tag}.npz", x=x.numpy(), gate_up_packed=W["gate_up_packed"].numpy(),
                            gate_up_scales=gus.numpy(), down_packed=W["down_packed"].numpy(), down_scales=dns.numpy(),
                            idx=idx.numpy(), w=w.numpy(), out=out.numpy(), group_size=np.int32(64))


def elementwise_case():
    g = torch.Generator().manual_seed(5)
    x = (torch.randn(3, 256, generator=g) * 3).to(torch.bfloat16)
    wt = (torch.randn(256, generator=g) * 0.5).to(torch.bfloat16)
    y0 = torch.empty_like(x)
    y1 = torch.empty_like(x)
    R.rmsnorm(x, wt, y0, 1e-6, False)
    R.rmsnorm(x, wt, y1, 1e-6, True)
    logits = (torch.randn(2, 512, generator=g) * 40).to(torch.bfloat16)
    capped = logits.clone()
    R.softcapping(capped, 30.0)
    np.savez_compressed(OUT / "elementwise.npz", x_bf16=bits(x), w_bf16=bits(wt),
                        rms_bf16=bits(y0), rms_unit_bf16=bits(y1), logits_bf16=bits(logits),
                        capped_bf16=bits(capped))


def router_case(name, m, h, e, seed):
    """Router front-end (gemma.py:75-76): the norm through the reference's CPU
    fallback rmsnorm with no weight (pybind.cpp:87-103), the rest as the
    module's own torch statements on bf16 CPU tensors."""
    x = synth.activations(m, h, seed=seed)
    x[0] *= 20.0   # rows of very different RMS
    if m > 1:
        x[1] *= 0.05
    W = synth.router_weights(e, h, seed=seed)
    y = torch.empty_like(x)
    R.rmsnorm(x, torch.empty(0), y, 1e-6, False)
    xr = y * (W["router_scale"] * (h ** -0.5))
    logits = torch.nn.functional.linear(xr, W["gate"])
    np.savez_compressed(OUT / f"{name}.npz", x_bf16=bits(x), router_scale_bf16=bits(W["router_scale"]),
                        gate_bf16=bits(W["gate"]), norm_bf16=bits(y), x_normed_bf16=bits(xr),
                        logits_bf16=bits(logits), eps=np.float32(1e-6))


def main():
    linear_case("linear_m1_k256_n96_gs64", 1, 256, 96, 64, seed=1)
    linear_case("linear_m5_k512_n128_gs128", 5, 512, 128, 128, seed=2)
    linear_case("linear_m3_k2816_n64_gs128", 3, 2816, 64, 128, seed=3)
    moe_case("moe_m5_small_top2_gs64", 5, 256, 128, 8, 2, 64, seed=4)
    moe_case("moe_m1_small_top2_gs64", 1, 256, 128, 8, 2, 64, seed=6)
    # duplicate ids across and within tokens (the reference test's randint(0,16) pattern)
    moe_case("moe_m3_dups_gs64", 3, 256, 128, 8, 4, 64, seed=7,
             idx=[[1, 1, 2, 3], [2, 5, 5, 5], [0, 7, 1, 2]])
    elementwise_case()
    router_case("router_m3_h512_e16", 3, 512, 16, seed=8)
    dtype_cases()
    for p in sorted(OUT.glob("*.npz")):
        print(p.name, p.stat().st_size)


if __name__ == "__main__":
    main()
