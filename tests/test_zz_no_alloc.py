"""gi_fused_batched_moe_static (no workspace argument, static per-GPU scratch)
against gi_fused_batched_moe (caller workspace), both through the C ABI.

Two calls in a row, the second with fewer rows, each compared bitwise with
the workspace entry point on the same inputs (the same kernels run, and their
sums have a fixed order); then a shape the static scratch cannot serve is
rejected with GI_ERR_WORKSPACE.
"""
import ctypes

import pytest
import torch

from gemmainfer_amd import _lib as L
from gemmainfer_amd import synth

pytestmark = pytest.mark.gpu
DEV = "cuda"
E, H, I, TOP_K = 128, 2816, 704, 8


def _p(t):
    return ctypes.c_void_p(t.data_ptr())


def _args(W, x, idx, w, out, m, gs):
    return (_p(x), L.DTYPE_BF16, _p(W["gate_up_packed"]), _p(W["gate_up_scales"]), W["gate_up_scales"].shape[1],
            _p(W["down_packed"]), _p(W["down_scales"]), W["down_scales"].shape[1], _p(idx), L.DTYPE_INT32,
            _p(w), L.DTYPE_BF16, _p(out), m, H, I, E, TOP_K, gs)


@pytest.mark.parametrize("gs", [64, 128])
def test_static_scratch_matches_workspace_entry_point(gs):
    lib = L.load()
    W = synth.device_moe_weights(E, H, I, gs, DEV, seed=800 + gs)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    ws = torch.zeros(lib.gi_fused_moe_workspace_bytes(8, TOP_K, H, I, E), dtype=torch.uint8, device=DEV)
    for call, (m, noise) in enumerate(((7, 0.5), (1, 0.0))):
        print(f"static scratch gs={gs} call={call} m={m}", flush=True)
        x = synth.activations(m, H, seed=810 + m).to(DEV)
        logits = synth.router_logits(m, E, seed=810 + m, verify_noise=noise)
        top, idx = torch.topk(logits, TOP_K, dim=-1)
        w = torch.softmax(top, dim=-1, dtype=torch.float32).to(torch.bfloat16).to(DEV)
        idx = idx.to(torch.int32).to(DEV)
        out_in = (torch.randn(m, H) * 0.1).to(torch.bfloat16).to(DEV)   # both accumulate into out
        ref = out_in.clone()
        got = out_in.clone()
        L.check(lib.gi_fused_batched_moe(*_args(W, x, idx, w, ref, m, gs), _p(ws), ws.numel(), 0, stream),
                "gi_fused_batched_moe")
        L.check(lib.gi_fused_batched_moe_static(*_args(W, x, idx, w, got, m, gs), 0, stream),
                "gi_fused_batched_moe_static")
        torch.cuda.synchronize()
        assert torch.isfinite(got.float()).all()
        assert torch.equal(got, ref), f"call {call} (m={m}): static-scratch output differs"
    assert lib.gi_device_error_flags(torch.cuda.current_device(), 0) == 0


def test_static_scratch_rejects_shapes_it_cannot_serve():
    lib = L.load()
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    buf = torch.zeros(16, dtype=torch.int32, device=DEV)
    p = _p(buf)
    # group size 24: the general fused path, whose partial slabs need a caller workspace
    st = lib.gi_fused_batched_moe_static(p, L.DTYPE_BF16, p, p, 11, p, p, 30, p, L.DTYPE_INT32, p, L.DTYPE_BF16,
                                         p, 1, 256, 128, 8, 2, 24, 0, stream)
    assert st == L.GI_ERR_WORKSPACE
    assert "caller workspace" in lib.gi_last_error().decode()


@pytest.mark.parametrize("m", [1, 7])
def test_static_entry_wait_timeout_is_reported(m):
    """spin_limit=1 makes the static entry's bounded waits give up from the
    host (every kernel still ends): outputs are then bitwise those of the
    workspace entry point or NaN, never a wrong finite value;
    gi_fused_batched_moe_static_status reports the timeout exactly when an
    output is NaN, and its clearing read resets the static scratch, after
    which a call is right again and the status reads 0."""
    lib = L.load()
    gs = 128
    dev = torch.cuda.current_device()
    W = synth.device_moe_weights(E, H, I, gs, DEV, seed=830)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    ws = torch.zeros(lib.gi_fused_moe_workspace_bytes(8, TOP_K, H, I, E), dtype=torch.uint8, device=DEV)
    x = synth.activations(m, H, seed=840 + m).to(DEV)
    logits = synth.router_logits(m, E, seed=840 + m, verify_noise=0.5)
    top, idx = torch.topk(logits, TOP_K, dim=-1)
    w = torch.softmax(top, dim=-1, dtype=torch.float32).to(torch.bfloat16).to(DEV)
    idx = idx.to(torch.int32).to(DEV)
    out_in = (torch.randn(m, H) * 0.1).to(torch.bfloat16).to(DEV)
    ref = out_in.clone()
    L.check(lib.gi_fused_batched_moe(*_args(W, x, idx, w, ref, m, gs), _p(ws), ws.numel(), 0, stream),
            "gi_fused_batched_moe")
    print(f"static timeout m={m}", flush=True)
    got = out_in.clone()
    L.check(lib.gi_fused_batched_moe_static(*_args(W, x, idx, w, got, m, gs), 1, stream), "static spin 1")
    torch.cuda.synchronize()
    finite = torch.isfinite(got.float())
    print(f"  {int((~finite).sum())} NaN outputs of {got.numel()}", flush=True)
    assert torch.equal(got[finite], ref[finite]), "a finite output is wrong after a timeout"
    st = ctypes.c_int32(-1)
    L.check(lib.gi_fused_batched_moe_static_status(ctypes.byref(st), 1, stream), "static status")
    assert st.value == (0 if bool(finite.all()) else L.DEVICE_SPIN_TIMEOUT)
    lib.gi_device_error_flags(dev, 1)  # the host flag this timeout may have set
    again = out_in.clone()
    L.check(lib.gi_fused_batched_moe_static(*_args(W, x, idx, w, again, m, gs), 0, stream), "static after")
    torch.cuda.synchronize()
    assert torch.equal(again, ref)
    L.check(lib.gi_fused_batched_moe_static_status(ctypes.byref(st), 1, stream), "static status")
    assert st.value == 0
    assert lib.gi_device_error_flags(dev, 1) == 0
