"""CPU tests of the drop-in boundary: the C-ABI library and the gemmainfer_csrc module.

No GPU work happens here: only library loading, symbol export, host-side
argument validation (which returns before any HIP call), and the CPU-tensor
semantics the drop-in module keeps from the reference (pybind.cpp CPU paths).
"""
from __future__ import annotations

import ctypes
import re
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

import gemmainfer_csrc
from gemmainfer_amd import _lib as L
from gemmainfer_amd import cpu_ops, ops, synth
from oracle import cpu_baseline as CB
from oracle import moe_oracle as O

ROOT = Path(__file__).resolve().parents[1]
HEADERS = sorted((ROOT / "include").glob("*.h"))
REF_DIR = ROOT / "oracle" / "_ref"


@pytest.fixture(scope="module")
def lib():
    if not L.LIB_PATH.exists():
        from gemmainfer_amd import build
        build.build(verbose=False)
    return L.load()


def header_functions():
    names = set()
    for h in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names.update(re.findall(r"\b(gi_[a-z0-9_]+)\s*\(", text))
    return sorted(names)


def test_library_exports_every_declared_symbol(lib):
    declared = header_functions()
    assert len(declared) >= 12
    assert set(declared) == set(L.SIGNATURES), "ctypes table and header disagree"
    for name in declared:
        assert hasattr(lib, name), f"{name} not exported"
    assert lib.gi_abi_version() == 1


def test_workspace_queries_are_host_only(lib):
    # 7 tokens x top-8 = 56 slots, 22 intermediate tiles of 32, 2816 fp32 each
    need = lib.gi_fused_moe_workspace_bytes(7, 8, 2816, 704, 128)
    assert need >= 56 * 22 * 2816 * 4
    assert lib.gi_fused_moe_workspace_bytes(0, 8, 2816, 704, 128) > 0
    assert lib.gi_fused_moe_workspace_bytes(1, 0, 2816, 704, 128) == 0
    assert lib.gi_w4a16_workspace_bytes(6, 2816, 262144, 128) == 0      # wide N: matrix cores, no K split
    assert lib.gi_w4a16_workspace_bytes(1, 2816, 2816, 128) == 0         # 1-2 rows: 16-column tiles, no K split
    assert lib.gi_w4a16_workspace_bytes(4, 2816, 2816, 128) > 0          # 3-16 rows: matrix cores, K split
    assert lib.gi_w4a16_workspace_bytes(4, 16384, 2816, 128) > 0         # long K: VALU split-K partials


def _moe_call(lib, **over):
    a = dict(x=ctypes.c_void_p(16), xd=L.DTYPE_BF16, gu=ctypes.c_void_p(16), gus=ctypes.c_void_p(16), ggu=22,
             dp=ctypes.c_void_p(16), ds=ctypes.c_void_p(16), gd=6, idx=ctypes.c_void_p(16), idt=L.DTYPE_INT32,
             w=ctypes.c_void_p(16), wd=L.DTYPE_BF16, out=ctypes.c_void_p(16), M=1, H=2816, I=704, E=128,
             top_k=8, gs=128, ws=None, wsb=0)
    a.update(over)
    st = lib.gi_fused_batched_moe(a["x"], a["xd"], a["gu"], a["gus"], a["ggu"], a["dp"], a["ds"], a["gd"],
                                  a["idx"], a["idt"], a["w"], a["wd"], a["out"], a["M"], a["H"], a["I"],
                                  a["E"], a["top_k"], a["gs"], a["ws"], a["wsb"], 0, None)
    return st, lib.gi_last_error().decode()


@pytest.mark.parametrize("over,code,frag", [
    (dict(xd=L.DTYPE_INT32), L.GI_ERR_UNSUPPORTED, "bf16, fp16 or fp32"),
    (dict(idt=L.DTYPE_FP32), L.GI_ERR_UNSUPPORTED, "int32 or int64"),
    (dict(H=2820), L.GI_ERR_INVALID_ARG, "multiples of 8"),
    (dict(gs=12), L.GI_ERR_INVALID_ARG, "group_size"),
    (dict(E=2048), L.GI_ERR_UNSUPPORTED, "1024 experts"),
    (dict(x=None), L.GI_ERR_INVALID_ARG, "null"),
    (dict(x=ctypes.c_void_p(8)), L.GI_ERR_INVALID_ARG, "16-byte"),
    (dict(gd=0), L.GI_ERR_INVALID_ARG, "group"),
    (dict(), L.GI_ERR_WORKSPACE, "workspace"),
])
def test_fused_moe_rejects_bad_arguments_without_touching_the_gpu(lib, over, code, frag):
    st, msg = _moe_call(lib, **over)
    assert st == code, msg
    assert frag in msg


def test_other_entry_points_validate(lib):
    assert lib.gi_w4a16_linear(None, L.DTYPE_BF16, None, None, 1, None, 1, 2816, 2816, 128, 0.0,
                               None, 0, None) == L.GI_ERR_INVALID_ARG
    assert lib.gi_w4a16_linear(None, L.DTYPE_BF16, None, None, 1, None, 1, 2812, 2816, 128, 0.0,
                               None, 0, None) == L.GI_ERR_INVALID_ARG       # K % 8
    assert lib.gi_w4a16_linear(None, L.DTYPE_FP16, None, None, 1, None, 1, 2816, 2816, 128, 0.0,
                               None, 0, None) == L.GI_ERR_INVALID_ARG       # fp16: null pointers
    assert lib.gi_w4a16_linear(None, L.DTYPE_INT32, None, None, 1, None, 1, 2816, 2816, 128, 0.0,
                               None, 0, None) == L.GI_ERR_UNSUPPORTED       # int32 activations
    assert lib.gi_moe_route_topk_softmax(None, L.DTYPE_FP32, None, 1, 128, 65, None, None, 0,
                                         None) == L.GI_ERR_UNSUPPORTED      # top_k > 64
    assert lib.gi_moe_align(None, L.DTYPE_INT32, 40, 8, 128, None, None, None, None, None,
                            None) == L.GI_ERR_UNSUPPORTED                   # 320 slots
    assert lib.gi_softcap_inplace(None, L.DTYPE_BF16, 10, 0.0, None) == L.GI_ERR_INVALID_ARG
    with pytest.raises(L.GIError) as ei:
        L.check(L.GI_ERR_INVALID_ARG, "probe")
    assert ei.value.code == L.GI_ERR_INVALID_ARG


def test_router_ingest_and_dense_entry_points_validate(lib):
    """The entry points added for the router front-end, checkpoint ingest and
    the dense callers reject bad arguments on the host, before any launch."""
    vp = ctypes.c_void_p(16)
    R = lib.gi_moe_router_logits
    assert R(vp, L.DTYPE_FP32, None, vp, 1e-6, vp, 1, 2816, 128, None) == L.GI_ERR_UNSUPPORTED  # fp32 x
    assert R(vp, L.DTYPE_BF16, None, vp, 1e-6, vp, 1, 2812, 128, None) == L.GI_ERR_UNSUPPORTED  # H % 8
    assert R(vp, L.DTYPE_BF16, None, vp, 1e-6, vp, 1, 8192, 128, None) == L.GI_ERR_UNSUPPORTED  # H > 4096
    assert R(vp, L.DTYPE_BF16, None, None, 1e-6, vp, 1, 2816, 128, None) == L.GI_ERR_INVALID_ARG  # no gate
    assert R(vp, L.DTYPE_BF16, None, vp, -1.0, vp, 1, 2816, 128, None) == L.GI_ERR_INVALID_ARG  # eps < 0
    assert R(None, L.DTYPE_BF16, None, None, 1e-6, None, 0, 2816, 128, None) == L.GI_OK          # M = 0
    lh = lib.gi_moe_layer_from_hidden
    args = [vp, L.DTYPE_BF16, None, vp, 1e-6, None, None, vp, vp, 22, vp, vp, 6, vp, None, None,
            1, 2816, 704, 128, 8, 128, vp, 1 << 20, 0, None]
    assert lh(*args) == L.GI_ERR_INVALID_ARG                                  # no logits buffer
    args[5], args[20] = vp, 129
    assert lh(*args) == L.GI_ERR_INVALID_ARG                                  # top_k > E
    I = lib.gi_w4a16_ingest
    assert I(vp, vp, L.DTYPE_BF16, 64, 100, 1, vp, vp, 64, None) == L.GI_ERR_INVALID_ARG  # K % 8
    assert I(vp, vp, L.DTYPE_BF16, 64, 128, 2, vp, vp, 32, None) == L.GI_ERR_INVALID_ARG  # ld < N
    assert I(vp, vp, L.DTYPE_INT32, 64, 128, 2, vp, vp, 64, None) == L.GI_ERR_UNSUPPORTED  # scale dtype
    assert I(None, None, L.DTYPE_BF16, 0, 128, 2, None, None, 0, None) == L.GI_OK          # N = 0
    assert I(None, vp, L.DTYPE_BF16, 64, 128, 2, vp, vp, 64, None) == L.GI_ERR_INVALID_ARG  # null words
    IB = lib.gi_w4a16_ingest_batched
    assert IB(vp, vp, L.DTYPE_BF16, 70000, 64, 128, 2, 0, 0, vp, vp, 64, 0, 0, None) == L.GI_ERR_INVALID_ARG
    assert IB(None, None, L.DTYPE_BF16, 0, 64, 128, 2, 0, 0, None, None, 64, 0, 0, None) == L.GI_OK  # empty
    assert IB(vp, None, L.DTYPE_BF16, 4, 64, 128, 2, 0, 0, vp, vp, 64, 0, 0, None) == L.GI_ERR_INVALID_ARG
    n5 = (ctypes.c_int * 5)(*[64] * 5)
    p5 = (ctypes.c_void_p * 5)(*[16] * 5)
    assert lib.gi_w4a16_linear_multi(vp, L.DTYPE_BF16, 5, p5, p5, n5, p5, n5, 1, 256, 64, None, 0,
                                     None) == L.GI_ERR_INVALID_ARG            # more than 4 projections
    n2 = (ctypes.c_int * 2)(64, 66)
    assert lib.gi_w4a16_linear_multi(vp, L.DTYPE_BF16, 2, p5, p5, n2, p5, n2, 1, 256, 64, None, 0,
                                     None) == L.GI_ERR_INVALID_ARG            # N % 4
    assert lib.gi_w4a16_gated_mlp(vp, L.DTYPE_BF16, vp, vp, 4, vp, vp, 4, vp, 1, 256, 66, 64, None, 0,
                                  None) == L.GI_ERR_INVALID_ARG               # N % 4
    assert lib.gi_w4a16_gated_mlp(vp, L.DTYPE_FP16, vp, vp, 4, vp, vp, 4, vp, 1, 256, 64, 64, None, 0,
                                  None) == L.GI_ERR_UNSUPPORTED               # fp16 activations
    # workspace queries of the new calls are host-only
    assert lib.gi_w4a16_gated_mlp_workspace_bytes(1, 2816, 2112, 64) == 0    # one launch, none
    assert lib.gi_w4a16_gated_mlp_workspace_bytes(7, 2816, 2112, 64) > 0     # matrix cores, K split
    assert lib.gi_w4a16_linear_multi_workspace_bytes(3, (ctypes.c_int * 3)(4096, 2048, 2048), 1, 2816,
                                                     64) == 0


def test_missing_library_raises_no_fallback(monkeypatch, tmp_path):
    monkeypatch.setattr(L, "LIB_PATH", tmp_path / "absent.so")
    monkeypatch.setattr(L, "_lib", None)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        L.load()


def test_device_ops_reject_host_tensors():
    x = torch.zeros(1, 256, dtype=torch.bfloat16)
    with pytest.raises(TypeError, match="device tensors"):
        ops.marlin_w4a16(x, torch.zeros(32, 8, dtype=torch.int32), torch.zeros(4, 8, dtype=torch.bfloat16),
                         torch.zeros(1, 8, dtype=torch.bfloat16), 64)


# ----------------------------------------------------------------- CPU-tensor semantics
def _ref():
    if not any(REF_DIR.glob("gemmainfer_csrc_ref*.so")):
        pytest.skip("oracle/_ref not built (reference tree absent)")
    sys.path.insert(0, str(REF_DIR))
    import gemmainfer_csrc_ref  # noqa: PLC0415
    return gemmainfer_csrc_ref


def test_dropin_module_surface():
    assert set(gemmainfer_csrc.__all__) == {"rmsnorm", "fused_rope_inplace", "softcapping",
                                            "marlin_w4a16", "fused_batched_moe"}


def test_dropin_cpu_moe_and_linear_match_reference_fallback():
    R = _ref()
    W = synth.moe_weights(8, 256, 128, 64, seed=31)
    x = synth.activations(5, 256, seed=31)
    idx = torch.tensor([[1, 3], [3, 3], [0, 7], [2, 5], [6, 1]], dtype=torch.int32)
    w = torch.softmax(torch.randn(5, 2, generator=torch.Generator().manual_seed(0)), -1).to(torch.bfloat16)
    args = (W["gate_up_packed"], W["gate_up_scales"], W["down_packed"], W["down_scales"], idx, w)
    ours = torch.zeros(5, 256, dtype=torch.bfloat16)
    theirs = torch.zeros(5, 256, dtype=torch.bfloat16)
    gemmainfer_csrc.fused_batched_moe(x, *args, ours, 64)
    R.fused_batched_moe(x, *args, theirs, 64)
    torch.testing.assert_close(ours.float(), theirs.float(), rtol=2 ** -6, atol=2e-2)
    A = synth.activations(3, 512, seed=2)
    B, S = synth.linear_weights(512, 96, 128, seed=2)
    C1 = torch.empty(3, 96, dtype=torch.bfloat16)
    C2 = torch.empty(3, 96, dtype=torch.bfloat16)
    gemmainfer_csrc.marlin_w4a16(A, B, S, C1, 128)
    R.marlin_w4a16(A, B, S, C2, 128)
    torch.testing.assert_close(C1.float(), C2.float(), rtol=2 ** -7, atol=1e-2)


def test_dropin_cpu_companions_match_reference_fallback():
    R = _ref()
    x = torch.randn(2, 3, 256).to(torch.bfloat16)
    wt = torch.randn(256).to(torch.bfloat16)
    for unit in (False, True):
        a, b = torch.empty_like(x), torch.empty_like(x)
        gemmainfer_csrc.rmsnorm(x, wt, a, 1e-6, unit)
        R.rmsnorm(x, wt, b, 1e-6, unit)
        torch.testing.assert_close(a.float(), b.float(), rtol=2 ** -7, atol=1e-3)
    logits = (torch.randn(4, 100) * 50).to(torch.bfloat16)
    a, b = logits.clone(), logits.clone()
    gemmainfer_csrc.softcapping(a, 30.0)
    R.softcapping(b, 30.0)
    torch.testing.assert_close(a.float(), b.float(), rtol=2 ** -6, atol=1e-3)
    q = torch.randn(1, 2, 3, 8)
    k = torch.randn(1, 1, 3, 8)
    cos, sin = torch.randn(5, 8), torch.randn(5, 8)
    pos = torch.tensor([[0, 2, 4]])
    q1, k1, q2, k2 = q.clone(), k.clone(), q.clone(), k.clone()
    gemmainfer_csrc.fused_rope_inplace(q1, k1, cos, sin, pos)
    R.fused_rope_inplace(q2, k2, cos, sin, pos)
    torch.testing.assert_close(q1, q2)
    torch.testing.assert_close(k1, k2)


def test_cpu_ops_raise_like_the_reference_python_path_on_missing_groups():
    # K=704 with group 128 needs 6 scale rows; 5 (K//gs) is out of range
    A = torch.zeros(1, 704, dtype=torch.bfloat16)
    B = torch.zeros(88, 16, dtype=torch.int32)
    with pytest.raises(IndexError):
        cpu_ops.marlin_w4a16(A, B, torch.zeros(5, 16, dtype=torch.bfloat16),
                             torch.empty(1, 16, dtype=torch.bfloat16), 128)


# ----------------------------------------------------------------- CPU baseline
def test_cpu_baseline_restatement_agrees_with_oracle():
    W = synth.moe_weights(8, 256, 128, 64, seed=41)
    x = synth.activations(3, 256, seed=41)
    logits = synth.router_logits(3, 8, seed=41)
    top, idx = torch.topk(logits, 2, dim=-1)
    w = torch.softmax(top, -1).to(torch.bfloat16)
    got = CB.moe_forward(x, idx, w, W["gate_up_packed"], W["gate_up_scales"], W["down_packed"],
                         W["down_scales"], 64)
    f = lambda t: t.float().numpy().astype(np.float64)  # noqa: E731
    ref, _ = O.fused_batched_moe(f(x), W["gate_up_packed"].numpy(), f(W["gate_up_scales"]),
                                 W["down_packed"].numpy(), f(W["down_scales"]), idx.numpy(), f(w),
                                 np.zeros((3, 256)), 64)
    assert O.error_stats(f(got), ref)["rel_l2"] < 2e-2
    B, S = synth.linear_weights(256, 64, 64, seed=1)
    y = CB.lm_head_softcap(synth.activations(2, 256), B, S, 64)
    assert float(y.float().abs().max()) <= 30.0
