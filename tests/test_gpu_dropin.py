"""The engine's real configuration on the GPU, called exactly as the reference calls it.

GemmaBatchedMoE.forward (gemmainfer/models/gemma.py:82-111) calls
``gemmainfer_csrc.fused_batched_moe`` with the whole batch when it has at most
8 rows and with 8-row slices ``x_flat[start:end]``, ``idx_i32[start:end]``,
``weights[start:end]``, ``out[start:end]`` (views at non-zero offsets) above
that, on the real checkpoint's group size 64 (gemmainfer/models/config.py:40,
gemmainfer/utils/weights.py:47).  The reference's own GPU test of the kernel
(tests/test_cuda_kernels_sanitizer.py:60-83) uses E=128, H=2816, I=704,
group 64, packed words from randint(-1e5, 1e5), signed randn scales and ids
from randint(0, 16) (duplicates inside a token).  Every case here is checked
against the float64 oracle to the tolerance gate of tests/helpers.py.
"""
import ctypes

import numpy as np
import pytest
import torch

import gemmainfer_csrc
from gemmainfer_amd import _lib as L
from gemmainfer_amd import ops, synth
from oracle import moe_oracle as O
from tests.helpers import assert_bf16_close, assert_close_rms, np64

pytestmark = pytest.mark.gpu
DEV = "cuda"
E, H, I, TOP_K = 128, 2816, 704, 8


def _sanitizer_weights(gs, seed):
    """The inputs of test_cuda_kernels_sanitizer.py:66-72 (seeded, on the CPU)."""
    g = torch.Generator().manual_seed(seed)
    return {
        "gate_up_packed": torch.randint(-100000, 100000, (E, H // 8, 2 * I), generator=g, dtype=torch.int32),
        "gate_up_scales": torch.randn((E, H // gs, 2 * I), generator=g).to(torch.bfloat16),
        "down_packed": torch.randint(-100000, 100000, (E, I // 8, H), generator=g, dtype=torch.int32),
        "down_scales": torch.randn((E, -(-I // gs), H), generator=g).to(torch.bfloat16),
    }


def _signed_weights(gs, seed):
    """Uniform int4 codes with signed scales N(0, 0.02^2): the value range of a
    real checkpoint, both signs of scale."""
    W = synth.moe_weights(E, H, I, gs, seed=seed)
    g = torch.Generator().manual_seed(seed + 7)
    for k in ("gate_up_scales", "down_scales"):
        W[k] = (torch.randn(W[k].shape, generator=g) * 0.02).to(torch.bfloat16)
    return W


def _dev(W):
    return {k: v.to(DEV) for k, v in W.items()}


@pytest.fixture(scope="module")
def sanitizer64():
    W = _sanitizer_weights(64, seed=60)
    return W, _dev(W)


@pytest.fixture(scope="module")
def signed64():
    W = _signed_weights(64, seed=61)
    return W, _dev(W)


@pytest.fixture(scope="module")
def signed128():
    W = _signed_weights(128, seed=62)
    return W, _dev(W)


def _oracle(W, x, idx, w, out_in, gs):
    ref, al = O.fused_batched_moe(np64(x), W["gate_up_packed"].numpy(), np64(W["gate_up_scales"]),
                                  W["down_packed"].numpy(), np64(W["down_scales"]), idx.cpu().numpy(),
                                  np64(w), np64(out_in), gs)
    return ref, al


def _routing(m, seed, noise=0.0):
    logits = synth.router_logits(m, E, seed=seed, verify_noise=noise)
    top, idx = torch.topk(logits, TOP_K, dim=-1)                 # gemma.py:77
    w = torch.softmax(top, dim=-1, dtype=torch.float32)            # gemma.py:78
    return idx.to(torch.int32), w.to(torch.bfloat16)               # gemma.py:80, :85


@pytest.mark.parametrize("m", [1, 5, 7, 8])
def test_sanitizer_inputs_gs64(sanitizer64, m):
    """test_cuda_kernels_sanitizer.py:74-83 with values checked: ids from
    randint(0, 16) (duplicates within a token), softmax weights in bf16.
    Outputs reach RMS ~1e7 here; see assert_close_rms for the gate."""
    W, Wd = sanitizer64
    g = torch.Generator().manual_seed(100 + m)
    x = torch.randn((m, H), generator=g).to(torch.bfloat16)
    idx = torch.randint(0, 16, (m, TOP_K), generator=g, dtype=torch.int32)
    w = torch.softmax(torch.randn((m, TOP_K), generator=g), dim=-1).to(torch.bfloat16)
    print(f"sanitizer gs=64 m={m}", flush=True)
    out = torch.zeros((m, H), dtype=torch.bfloat16, device=DEV)
    gemmainfer_csrc.fused_batched_moe(x.to(DEV), Wd["gate_up_packed"], Wd["gate_up_scales"], Wd["down_packed"],
                                      Wd["down_scales"], idx.to(DEV), w.to(DEV), out, 64)
    ref, al = _oracle(W, x, idx, w, torch.zeros(m, H), 64)
    stats = assert_close_rms(out, ref, f"sanitizer gs=64 m={m}")
    print(f"  U={al.num_unique} {stats}")


@pytest.mark.parametrize("m,noise", [(1, 0.0), (5, 0.5), (7, 0.5), (8, 0.5)])
@pytest.mark.parametrize("gs", [64, 128])
def test_signed_scales_gemma(signed64, signed128, m, noise, gs):
    """Router-shaped ids (distinct within a token), signed scales, both group sizes."""
    W, Wd = signed64 if gs == 64 else signed128
    x = synth.activations(m, H, seed=200 + m)
    idx, w = _routing(m, seed=200 + m, noise=noise)
    print(f"signed gs={gs} m={m}", flush=True)
    out = torch.zeros((m, H), dtype=torch.bfloat16, device=DEV)
    gemmainfer_csrc.fused_batched_moe(x.to(DEV), Wd["gate_up_packed"], Wd["gate_up_scales"], Wd["down_packed"],
                                      Wd["down_scales"], idx.to(DEV), w.to(DEV), out, gs)
    ref, al = _oracle(W, x, idx, w, torch.zeros(m, H), gs)
    stats = assert_bf16_close(out, ref, f"signed gs={gs} m={m}")
    print(f"  U={al.num_unique} {stats}")


@pytest.mark.parametrize("m", [12, 23, 64, 100])
def test_caller_chunk_loop_gs64(signed64, m):
    """gemma.py:99-111 verbatim: 8-row slices of x_flat, idx_i32, weights and
    out (views at non-zero offsets) through the drop-in module."""
    W, Wd = signed64
    x = synth.activations(m, H, seed=300 + m)
    idx, w = _routing(m, seed=300 + m)
    x_flat, idx_i32, weights = x.to(DEV), idx.to(DEV), w.to(DEV)
    out = torch.zeros_like(x_flat)
    print(f"chunk loop gs=64 m={m}", flush=True)
    for start in range(0, m, 8):
        end = min(start + 8, m)
        gemmainfer_csrc.fused_batched_moe(x_flat[start:end], Wd["gate_up_packed"], Wd["gate_up_scales"],
                                          Wd["down_packed"], Wd["down_scales"], idx_i32[start:end],
                                          weights[start:end], out[start:end], 64)
    ref, _ = _oracle(W, x, idx, w, torch.zeros(m, H), 64)
    assert_bf16_close(out, ref, f"chunk loop m={m}")


def test_layer_gs64_matches_drop_in(signed64):
    """The layer entry point (routing in the kernel) at group 64 gives the same
    ids as torch.topk and the same output as the drop-in call on those ids."""
    W, Wd = signed64
    for m, noise in ((1, 0.0), (7, 0.5)):
        x = synth.activations(m, H, seed=400 + m).to(DEV)
        logits = synth.router_logits(m, E, seed=400 + m, verify_noise=noise)
        out, idx, w = ops.moe_layer(x, logits.to(DEV), Wd["gate_up_packed"], Wd["gate_up_scales"],
                                    Wd["down_packed"], Wd["down_scales"], TOP_K, 64)
        ref_idx, _ = _routing(m, seed=400 + m, noise=noise)
        np.testing.assert_array_equal(idx.cpu().numpy(), ref_idx.numpy())
        out2 = torch.zeros_like(x)
        gemmainfer_csrc.fused_batched_moe(x, Wd["gate_up_packed"], Wd["gate_up_scales"], Wd["down_packed"],
                                          Wd["down_scales"], idx, w, out2, 64)
        assert torch.equal(out, out2), f"m={m}"
        ref, _ = _oracle(W, x.cpu(), idx.cpu(), w.cpu(), torch.zeros(m, H), 64)
        assert_bf16_close(out, ref, f"layer gs=64 m={m}")


@pytest.mark.parametrize("gs", [64, 128])
@pytest.mark.parametrize("m", [1, 2, 7])
def test_decode_kernel_small_hidden(gs, m):
    """H <= 512 runs the decode kernel's two-k-block gate/up variant."""
    e, h, i = 16, 512, 256
    Wc = synth.moe_weights(e, h, i, gs, seed=500 + gs)
    Wd = _dev(Wc)
    x = synth.activations(m, h, seed=510 + m)
    logits = synth.router_logits(m, e, seed=510 + m, verify_noise=0.5)
    top, idx = torch.topk(logits, 4, dim=-1)
    w = torch.softmax(top, dim=-1, dtype=torch.float32).to(torch.bfloat16)
    idx = idx.to(torch.int32)
    out_in = (torch.randn(m, h) * 0.1).to(torch.bfloat16)
    out = out_in.to(DEV).clone()
    gemmainfer_csrc.fused_batched_moe(x.to(DEV), Wd["gate_up_packed"], Wd["gate_up_scales"], Wd["down_packed"],
                                      Wd["down_scales"], idx.to(DEV), w.to(DEV), out, gs)
    ref, _ = O.fused_batched_moe(np64(x), Wc["gate_up_packed"].numpy(), np64(Wc["gate_up_scales"]),
                                 Wc["down_packed"].numpy(), np64(Wc["down_scales"]), idx.numpy(), np64(w),
                                 np64(out_in), gs)
    assert_bf16_close(out, ref, f"small hidden gs={gs} m={m}")


@pytest.mark.parametrize("m", [1, 7])
def test_decode_kernel_wait_timeout_surfaces(signed128, m):
    """spin_limit=1 makes the decode kernels' own bounded waits give up from the
    host (every kernel still ends): the one-token kernel at M=1 (activation and
    folded-unit waits), the 8-row kernel at M=7.  Outputs are then either right
    or NaN, never a wrong finite value; the next call through the drop-in
    raises the device error once (no synchronisation of its own), and the
    call after it is right without any explicit status read or clear."""
    W, Wd = signed128
    x = synth.activations(m, H, seed=600)
    idx, w = _routing(m, seed=600, noise=0.5)
    ref, _ = _oracle(W, x, idx, w, torch.zeros(m, H), 128)
    xd, idd, wd = x.to(DEV), idx.to(DEV), w.to(DEV)
    out = torch.zeros((m, H), dtype=torch.bfloat16, device=DEV)
    ops.fused_batched_moe(xd, Wd["gate_up_packed"], Wd["gate_up_scales"], Wd["down_packed"], Wd["down_scales"],
                          idd, wd, out, 128, spin_limit=1)
    torch.cuda.synchronize()
    got = np64(out)
    finite = np.isfinite(got)
    print(f"timeout run: {int((~finite).sum())} NaN outputs of {got.size}", flush=True)
    if finite.any():
        bound = 2e-2 + 2.0 ** -7 * np.abs(ref[finite])
        assert np.all(np.abs(got[finite] - ref[finite]) <= bound), "a finite output is wrong after a timeout"
    raised = 0
    for _ in range(2):
        out2 = torch.zeros((m, H), dtype=torch.bfloat16, device=DEV)
        try:
            gemmainfer_csrc.fused_batched_moe(xd, Wd["gate_up_packed"], Wd["gate_up_scales"], Wd["down_packed"],
                                              Wd["down_scales"], idd, wd, out2, 128)
        except L.GIError as exc:
            assert exc.code == L.GI_ERR_DEVICE
            raised += 1
            continue
        break
    assert raised == (0 if finite.all() else 1)
    torch.cuda.synchronize()
    assert_bf16_close(out2, ref, "after the timeout")


def test_prefill_without_routing_outputs_keeps_general_path_counters():
    """A layer call of 64+ rows with out_idx/out_w NULL (the grouped-GEMM path
    then writes the routing into its own workspace buffers), followed on the
    same workspace by calls on the general fused path (group 32): the general
    path's barrier counters must be untouched by the prefill buffers."""
    e, h, i, k, gs = 8, 256, 128, 2, 32
    Wc = synth.moe_weights(e, h, i, gs, seed=700)
    Wd = _dev(Wc)
    lib = L.load()
    ws = torch.zeros(lib.gi_fused_moe_workspace_bytes(64, k, h, i, e), dtype=torch.uint8, device=DEV)
    p = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    x64 = synth.activations(64, h, seed=701).to(DEV)
    logits = synth.router_logits(64, e, seed=701).to(DEV)
    out64 = torch.empty_like(x64)
    L.check(lib.gi_moe_layer_from_logits(
        p(x64), L.DTYPE_BF16, p(logits), L.DTYPE_FP32, None, p(Wd["gate_up_packed"]), p(Wd["gate_up_scales"]),
        Wd["gate_up_scales"].shape[1], p(Wd["down_packed"]), p(Wd["down_scales"]), Wd["down_scales"].shape[1],
        p(out64), None, None, 64, h, i, e, k, gs, p(ws), ws.numel(), 0, stream), "layer m=64")
    for m in (4, 3):
        x = synth.activations(m, h, seed=710 + m)
        lg = synth.router_logits(m, e, seed=710 + m)
        idx, _, wv = O.route_topk_softmax(np64(lg), k)
        idx_t = torch.from_numpy(idx).to(torch.int32)
        w_t = torch.from_numpy(wv).to(torch.bfloat16)
        out = torch.zeros((m, h), dtype=torch.bfloat16, device=DEV)
        xd, idd, wd = x.to(DEV), idx_t.to(DEV), w_t.to(DEV)  # alive until the kernel has run
        L.check(lib.gi_fused_batched_moe(
            p(xd), L.DTYPE_BF16, p(Wd["gate_up_packed"]), p(Wd["gate_up_scales"]),
            Wd["gate_up_scales"].shape[1], p(Wd["down_packed"]), p(Wd["down_scales"]), Wd["down_scales"].shape[1],
            p(idd), L.DTYPE_INT32, p(wd), L.DTYPE_BF16, p(out), m, h, i, e, k, gs,
            p(ws), ws.numel(), 0, stream), f"fused m={m}")
        torch.cuda.synchronize()
        ref, _ = O.fused_batched_moe(np64(x), Wc["gate_up_packed"].numpy(), np64(Wc["gate_up_scales"]),
                                     Wc["down_packed"].numpy(), np64(Wc["down_scales"]), idx, np64(w_t),
                                     np.zeros((m, h)), gs)
        assert_bf16_close(out, ref, f"general path after prefill m={m}")
    st = ctypes.c_int32(0)
    L.check(lib.gi_workspace_status(p(ws), ws.numel(), ctypes.byref(st), stream), "status")
    assert st.value == 0


def _routing_logits(case, e, seed):
    g = torch.Generator().manual_seed(seed)
    if case == "ties":
        # half-integers: many equal values, ties across the top-k boundary
        return (torch.round(torch.randn(1, e, generator=g) * 2.0) / 2.0)
    logits = torch.randn(1, e, generator=g)
    if case == "nan":
        logits[0, e // 3] = float("nan")
    return logits.to(torch.bfloat16) if case == "bf16" else logits


@pytest.mark.parametrize("e", [36, 128, 200])
@pytest.mark.parametrize("case", ["fp32", "bf16", "ties", "nan", "scale"])
def test_one_token_layer_routing(e, case):
    """The one-token kernel's in-kernel routing (M=1 layer call): ranks of all
    threads up to 128 experts, the radix select above.  ids bit-exact against
    the oracle's top-k (value descending, lower index first, NaN highest),
    weights within one bf16 ulp, the output within the gate; with a NaN logit
    only the ids and the finite weights are compared."""
    h, i, gs = 256, 128, 64
    Wc = synth.moe_weights(e, h, i, gs, seed=700 + e)
    Wd = _dev(Wc)
    x = synth.activations(1, h, seed=701)
    logits = _routing_logits(case, e, seed=702 + e)
    es = torch.linspace(0.5, 1.5, e) if case == "scale" else None
    out, idx, w = ops.moe_layer(x.to(DEV), logits.to(DEV), Wd["gate_up_packed"], Wd["gate_up_scales"],
                                Wd["down_packed"], Wd["down_scales"], TOP_K, gs,
                                expert_scale=None if es is None else es.to(DEV))
    ref_out, ref_idx, ref_w, _ = O.moe_layer_from_logits(
        np64(x), np64(logits), Wc["gate_up_packed"].numpy(), np64(Wc["gate_up_scales"]),
        Wc["down_packed"].numpy(), np64(Wc["down_scales"]), TOP_K, gs,
        expert_scale=None if es is None else es.numpy())
    np.testing.assert_array_equal(idx.cpu().numpy(), ref_idx, err_msg=f"{case} E={e}")
    finite = np.isfinite(ref_w)
    np.testing.assert_allclose(np64(w)[finite], ref_w[finite], rtol=2.0 ** -7)
    if case != "nan":
        assert_bf16_close(out, ref_out, f"routing {case} E={e}")


def _one_token_case(case, idx, w, g):
    """ids/weights of one token for the edge cases of the reference's
    launch_fused_batched_moe at M=1 (csrc/marlin.cu:286-296: the MAX_MATCH=1
    path skips ids outside [0, E); :631-636: ids cast to int32, weights to the
    activation dtype)."""
    if case == "invalid_mix":
        idx[0, 1], idx[0, 4], idx[0, 6] = -1, E, 4096
    elif case == "all_invalid":
        idx[0] = torch.tensor([-1, E, -7, 4096, E + 1, -1, 99999, -100], dtype=idx.dtype)
    elif case == "int64":
        idx = idx.to(torch.int64)
    elif case == "w_fp32":
        w = torch.rand(1, TOP_K, generator=g) + 0.05        # not bf16-representable: cast in the kernel
    elif case == "w_fp16":
        w = (torch.rand(1, TOP_K, generator=g) + 0.05).to(torch.float16)
    elif case == "dups":
        idx[0, 3] = idx[0, 0]
        idx[0, 5] = idx[0, 0]
        idx[0, 7] = idx[0, 2]
        w = (torch.rand(1, TOP_K, generator=g) + 0.05).to(torch.bfloat16)
    elif case == "dups_invalid":
        idx[0] = torch.tensor([9, -1, 9, 9, E, 9, 9, -3], dtype=idx.dtype)   # U = 1
    return idx, w


@pytest.mark.parametrize("gs", [64, 128])
@pytest.mark.parametrize("case", ["invalid_mix", "all_invalid", "int64", "w_fp32", "w_fp16", "dups",
                                  "dups_invalid"])
def test_one_token_kernel_reference_edge_cases(signed64, signed128, gs, case):
    """The one-token kernel (every M=1 call at the Gemma shapes) on the
    reference's edge cases, through the drop-in module, accumulating into a
    non-zero out: ids outside [0, E) mixed in or all of them (U = 0: out is
    left as it was), int64 ids, fp32 and fp16 routing weights, one expert in
    several slots with different weights."""
    W, Wd = signed64 if gs == 64 else signed128
    g = torch.Generator().manual_seed(900)
    x = synth.activations(1, H, seed=900)
    idx, w = _routing(1, seed=900)
    idx, w = _one_token_case(case, idx, w, g)
    out_in = (torch.randn(1, H, generator=g) * 0.5).to(torch.bfloat16)
    out = out_in.to(DEV).clone()
    print(f"one-token edge case {case} gs={gs} ids={idx.tolist()}", flush=True)
    gemmainfer_csrc.fused_batched_moe(x.to(DEV), Wd["gate_up_packed"], Wd["gate_up_scales"], Wd["down_packed"],
                                      Wd["down_scales"], idx.to(DEV), w.to(DEV), out, gs)
    ref, al = _oracle(W, x, idx, w, out_in, gs)
    if case == "all_invalid":
        assert al.num_unique == 0
        assert torch.equal(out.cpu(), out_in)
    assert_bf16_close(out, ref, f"one-token {case} gs={gs}")
    assert ops.workspace_status() == 0


@pytest.mark.parametrize("i,gs", [(704, 256), (768, 128), (768, 64)])
def test_one_token_kernel_other_variants(i, gs):
    """The one-token kernel's variants with the group size read at run time
    (group 256 at I = 704) and with 12 unit steps (I = 768), at H = 2816,
    E = 32, top-8, against the oracle, from ids and from logits."""
    e = 32
    Wc = _signed_weights_shape(e, H, i, gs, seed=910 + i + gs)
    Wd = _dev(Wc)
    x = synth.activations(1, H, seed=911)
    logits = synth.router_logits(1, e, seed=912)
    top, idx = torch.topk(logits, TOP_K, dim=-1)
    w = torch.softmax(top, dim=-1, dtype=torch.float32).to(torch.bfloat16)
    idx = idx.to(torch.int32)
    out_in = (torch.randn(1, H) * 0.1).to(torch.bfloat16)
    out = out_in.to(DEV).clone()
    print(f"one-token variant I={i} gs={gs}", flush=True)
    gemmainfer_csrc.fused_batched_moe(x.to(DEV), Wd["gate_up_packed"], Wd["gate_up_scales"], Wd["down_packed"],
                                      Wd["down_scales"], idx.to(DEV), w.to(DEV), out, gs)
    ref, _ = _oracle(Wc, x, idx, w, out_in, gs)
    assert_bf16_close(out, ref, f"one-token I={i} gs={gs}")
    lo, lidx, lw = ops.moe_layer(x.to(DEV), logits.to(DEV), Wd["gate_up_packed"], Wd["gate_up_scales"],
                                 Wd["down_packed"], Wd["down_scales"], TOP_K, gs)
    np.testing.assert_array_equal(lidx.cpu().numpy(), idx.numpy())
    ref0, _ = _oracle(Wc, x, idx, lw.cpu(), torch.zeros(1, H), gs)
    assert_bf16_close(lo, ref0, f"one-token layer I={i} gs={gs}")


def _signed_weights_shape(e, h, i, gs, seed):
    W = synth.moe_weights(e, h, i, gs, seed=seed)
    g = torch.Generator().manual_seed(seed + 7)
    for k in ("gate_up_scales", "down_scales"):
        W[k] = (torch.randn(W[k].shape, generator=g) * 0.02).to(torch.bfloat16)
    return W
