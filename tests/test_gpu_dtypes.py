"""fp16 and fp32 activations through the drop-in module on the GPU.

The reference dispatches all three activation dtypes for the MoE
(csrc/marlin.cu:694-700) and the linear (:764-770, :816-822, :831-842), and
its CLIs offer them (scripts/chat.py:53, scripts/serve.py:293).  x (A), the
scales and out (C) share the dtype; the routing weights are cast to it.
Checked against the float64 oracle with the reference's rounding points in
that dtype (oracle/moe_oracle.py round_to) and against the golden vectors of
the reference's own CPU fallback in fp16 and fp32 (tests/golden).
"""
import numpy as np
import pytest
import torch

import gemmainfer_csrc
from gemmainfer_amd import ops, synth
from oracle import moe_oracle as O
from tests.helpers import assert_dtype_close, np64

pytestmark = pytest.mark.gpu
DEV = "cuda"
DT = {"fp16": torch.float16, "fp32": torch.float32}
GOLDEN = __import__("pathlib").Path(__file__).resolve().parent / "golden"
E, H, I = 128, 2816, 704


def _moe_weights(e, h, i, gs, seed, dt):
    W = synth.moe_weights(e, h, i, gs, seed=seed)
    g = torch.Generator().manual_seed(seed + 3)
    for k in ("gate_up_scales", "down_scales"):   # signed scales of a checkpoint's size
        W[k] = (torch.randn(W[k].shape, generator=g) * 0.02).to(dt)
    return W


def _oracle(W, x, idx, w, out_in, gs, tag):
    ref, _ = O.fused_batched_moe(np64(x), W["gate_up_packed"].numpy(), np64(W["gate_up_scales"]),
                                 W["down_packed"].numpy(), np64(W["down_scales"]), idx.numpy(), np64(w),
                                 np64(out_in), gs, dtype=tag)
    return ref


@pytest.fixture(scope="module", params=[(64, "fp16"), (128, "fp16"), (64, "fp32"), (128, "fp32")],
                ids=lambda p: f"gs{p[0]}-{p[1]}")
def gemma(request):
    gs, tag = request.param
    W = _moe_weights(E, H, I, gs, seed=800 + gs, dt=DT[tag])
    return gs, tag, W, {k: v.to(DEV) for k, v in W.items()}


@pytest.mark.parametrize("m,noise", [(1, 0.0), (7, 0.5), (9, 0.5)])
def test_moe_gemma_shape(gemma, m, noise):
    gs, tag, W, Wd = gemma
    dt = DT[tag]
    x = synth.activations(m, H, seed=810 + m).to(dt)
    logits = synth.router_logits(m, E, seed=810 + m, verify_noise=noise)
    top, idx = torch.topk(logits, 8, dim=-1)
    w = torch.softmax(top, dim=-1, dtype=torch.float32).to(dt)   # gemma.py:78-80, .type_as(x)
    idx = idx.to(torch.int32)
    out_in = (torch.randn(m, H, generator=torch.Generator().manual_seed(m)) * 0.1).to(dt)
    out = out_in.to(DEV).clone()
    gemmainfer_csrc.fused_batched_moe(x.to(DEV), Wd["gate_up_packed"], Wd["gate_up_scales"], Wd["down_packed"],
                                      Wd["down_scales"], idx.to(DEV), w.to(DEV), out, gs)
    torch.cuda.synchronize()
    assert out.dtype == dt
    assert_dtype_close(out, _oracle(W, x, idx, w, out_in, gs, tag), tag, f"moe {tag} gs={gs} m={m}")


@pytest.mark.parametrize("gs", [64, 128])
def test_moe_fp16_one_token_edge_cases(gs):
    """fp16 at one token runs the one-token kernel's fp16 variant (its items
    split each fp16 value of x exactly into bf16 hi + lo operand rows, its
    units take fp16 products on exact q - 8 operands): ids outside [0, E)
    skipped (marlin.cu:304, :473), one expert in several slots with different
    weights, int64 ids and fp32 weights cast to fp16 (marlin.cu:631-636),
    activations spread over fp16's whole range (every significand bit and
    subnormals in use), accumulation into a non-zero out, and all ids
    invalid (out unchanged)."""
    dt = torch.float16
    W = _moe_weights(E, H, I, gs, seed=900 + gs, dt=dt)
    Wd = {n: v.to(DEV) for n, v in W.items()}
    g = torch.Generator().manual_seed(901)
    mag = torch.exp(torch.randn(1, H, generator=g)).clamp(max=20.0)
    x = (synth.activations(1, H, seed=902) * mag).to(dt)
    x[0, :8] = torch.tensor([6e-8, -6e-8, 1e-6, -3e-5, 0.0, 17.0078125, -1.0009765625, 0.33325195]).to(dt)
    cases = [
        (torch.tensor([[5, -1, 5, 127, 128, 99, 0, 3]], dtype=torch.int64), torch.rand(1, 8, generator=g)),
        (torch.tensor([[3, 3, 3, 3, 3, 3, 3, 3]], dtype=torch.int32), torch.rand(1, 8, generator=g).to(dt)),
        (torch.tensor([[17, 42, 9, 120, 77, 1, 64, 33]], dtype=torch.int32),
         torch.softmax(torch.randn(1, 8, generator=g), dim=-1).to(torch.bfloat16)),
    ]
    for n, (idx, w) in enumerate(cases):
        out_in = (torch.randn(1, H, generator=g) * 0.1).to(dt)
        out = out_in.to(DEV).clone()
        gemmainfer_csrc.fused_batched_moe(x.to(DEV), Wd["gate_up_packed"], Wd["gate_up_scales"],
                                          Wd["down_packed"], Wd["down_scales"], idx.to(DEV), w.to(DEV), out, gs)
        torch.cuda.synchronize()
        ref = _oracle(W, x, idx, w.to(dt), out_in, gs, "fp16")
        assert_dtype_close(out, ref, "fp16", f"fp16 one token gs={gs} case {n}")
    # no valid id: out unchanged
    idx = torch.tensor([[-1, 128, 200, -5, 1000, -1, 128, 129]], dtype=torch.int32)
    out_in = (torch.randn(1, H, generator=g) * 0.1).to(dt).to(DEV)
    out = out_in.clone()
    gemmainfer_csrc.fused_batched_moe(x.to(DEV), Wd["gate_up_packed"], Wd["gate_up_scales"], Wd["down_packed"],
                                      Wd["down_scales"], idx.to(DEV), torch.ones(1, 8, dtype=dt).to(DEV), out, gs)
    torch.cuda.synchronize()
    assert torch.equal(out, out_in)


@pytest.mark.parametrize("gs", [64, 128])
@pytest.mark.parametrize("m", [2, 5, 8])
def test_moe_fp16_rows_edge_cases(gs, m):
    """fp16 at 2-8 rows runs the 8-row kernel's fp16 variant (fp16 products
    with the int4 codes unpacked exactly to q - 8): the two-token dot-product
    path (m=2) and the matrix-core path (m=5, 8), ids outside [0, E) skipped
    (marlin.cu:304, :473), one expert in several slots of a token, every
    token on one expert, int64 ids and fp32 weights cast to fp16
    (marlin.cu:631-636), activations spread over 1/16 .. 4 times their
    scale plus subnormals and full-significand values, accumulation into a
    non-zero out, and all ids invalid (out unchanged).  The magnitudes keep
    outputs in the hundreds: in the thousands, one-ulp flips of the fp16
    activation rounding (marlin.cu:421-423) under any fp32 sum order exceed
    one output ulp (a float32 evaluation of the same semantics fails the
    bound there too); on these inputs it stays within 0.75 of it."""
    dt = torch.float16
    W = _moe_weights(E, H, I, gs, seed=930 + gs, dt=dt)
    Wd = {n: v.to(DEV) for n, v in W.items()}
    g = torch.Generator().manual_seed(931 + m)
    mag = torch.exp(0.5 * torch.randn(m, H, generator=g)).clamp(max=4.0)
    x = (synth.activations(m, H, seed=932 + m) * mag).to(dt)
    x[0, :8] = torch.tensor([6e-8, -6e-8, 1e-6, -3e-5, 0.0, 17.0078125, -1.0009765625, 0.33325195]).to(dt)
    ids = torch.stack([torch.randperm(E, generator=g)[:8] for _ in range(m)])
    ids[0, 1], ids[0, 4], ids[m - 1, 2] = -1, E, ids[m - 1, 6]       # invalid ids, a repeated expert
    cases = [
        (ids.to(torch.int64), torch.rand(m, 8, generator=g)),
        (torch.full((m, 8), 3, dtype=torch.int32), (torch.rand(m, 8, generator=g) / 4).to(dt)),
        (ids.clamp(0, E - 1).to(torch.int32), torch.softmax(torch.randn(m, 8, generator=g), dim=-1).to(torch.bfloat16)),
    ]
    for n, (idx, w) in enumerate(cases):
        out_in = (torch.randn(m, H, generator=g) * 0.1).to(dt)
        out = out_in.to(DEV).clone()
        gemmainfer_csrc.fused_batched_moe(x.to(DEV), Wd["gate_up_packed"], Wd["gate_up_scales"],
                                          Wd["down_packed"], Wd["down_scales"], idx.to(DEV), w.to(DEV), out, gs)
        torch.cuda.synchronize()
        ref = _oracle(W, x, idx, w.to(dt), out_in, gs, "fp16")
        assert_dtype_close(out, ref, "fp16", f"fp16 rows m={m} gs={gs} case {n}")
    idx = torch.full((m, 8), -1, dtype=torch.int32)
    idx[:, ::2] = E
    out_in = (torch.randn(m, H, generator=g) * 0.1).to(dt).to(DEV)
    out = out_in.clone()
    gemmainfer_csrc.fused_batched_moe(x.to(DEV), Wd["gate_up_packed"], Wd["gate_up_scales"], Wd["down_packed"],
                                      Wd["down_scales"], idx.to(DEV), torch.ones(m, 8, dtype=dt).to(DEV), out, gs)
    torch.cuda.synchronize()
    assert torch.equal(out, out_in)


@pytest.mark.parametrize("h,i,e,gs", [(256, 128, 32, 64), (2816, 704, 128, 128), (2816, 704, 32, 256)])
@pytest.mark.parametrize("m", [1, 2, 4])
def test_moe_fp16_eight_row_modes(h, i, e, gs, m):
    """top_k = 16, more experts per token than the one-token kernel holds:
    every call of 1-4 rows is one launch of the 8-row kernel's fp16 variant,
    in its one-row (m=1) and two-row (m=2) dot-product modes and its
    matrix-core mode (m=4), at a hidden size of at most 512 and at the Gemma
    size (group size 256: the scale groups read at run time); an id outside
    [0, E) and a repeated expert in a token (marlin.cu:304, :473)."""
    dt, k = torch.float16, 16
    W = _moe_weights(e, h, i, gs, seed=950 + m, dt=dt)
    Wd = {n: v.to(DEV) for n, v in W.items()}
    g = torch.Generator().manual_seed(951 + m)
    idx = torch.stack([torch.randperm(e, generator=g)[:k] for _ in range(m)]).to(torch.int32)
    idx[0, 3], idx[m - 1, 5] = -1, idx[m - 1, 9]
    w = torch.softmax(torch.randn(m, k, generator=g), dim=-1).to(dt)
    x = synth.activations(m, h, seed=952 + m).to(dt)
    out_in = (torch.randn(m, h, generator=g) * 0.1).to(dt)
    out = out_in.to(DEV).clone()
    gemmainfer_csrc.fused_batched_moe(x.to(DEV), Wd["gate_up_packed"], Wd["gate_up_scales"], Wd["down_packed"],
                                      Wd["down_scales"], idx.to(DEV), w.to(DEV), out, gs)
    torch.cuda.synchronize()
    assert_dtype_close(out, _oracle(W, x, idx, w, out_in, gs, "fp16"), "fp16", f"fp16 top-16 h={h} m={m}")


@pytest.mark.parametrize("i,gs", [(704, 256), (768, 128), (768, 64)])
def test_moe_fp16_one_token_other_variants(i, gs):
    """The one-token kernel's fp16 variants with the group size read at run
    time (group 256 at I = 704) and with 12 unit steps (I = 768), at H = 2816,
    E = 32, top-8, from ids, against the oracle."""
    dt, e = torch.float16, 32
    W = _moe_weights(e, H, i, gs, seed=990 + i + gs, dt=dt)
    Wd = {n: v.to(DEV) for n, v in W.items()}
    x = synth.activations(1, H, seed=991).to(dt)
    logits = synth.router_logits(1, e, seed=992)
    top, idx = torch.topk(logits, 8, dim=-1)
    w = torch.softmax(top, dim=-1, dtype=torch.float32).to(dt)
    idx = idx.to(torch.int32)
    out_in = (torch.randn(1, H, generator=torch.Generator().manual_seed(993)) * 0.1).to(dt)
    out = out_in.to(DEV).clone()
    gemmainfer_csrc.fused_batched_moe(x.to(DEV), Wd["gate_up_packed"], Wd["gate_up_scales"], Wd["down_packed"],
                                      Wd["down_scales"], idx.to(DEV), w.to(DEV), out, gs)
    torch.cuda.synchronize()
    assert_dtype_close(out, _oracle(W, x, idx, w, out_in, gs, "fp16"), "fp16", f"fp16 one-token I={i} gs={gs}")


@pytest.mark.parametrize("m", [7, 12])
def test_moe_fp16_deterministic_and_multi_launch(m):
    """fp16 on the 8-row kernel: one launch (m=7) and two launches of 8 and 4
    rows (m=12), against the oracle, and bitwise the same result on a second
    call (every sum has a fixed order)."""
    dt, gs = torch.float16, 128
    W = _moe_weights(E, H, I, gs, seed=970 + m, dt=dt)
    Wd = {n: v.to(DEV) for n, v in W.items()}
    x = synth.activations(m, H, seed=971 + m).to(dt)
    logits = synth.router_logits(m, E, seed=972 + m, verify_noise=0.5)
    top, idx = torch.topk(logits, 8, dim=-1)
    w = torch.softmax(top, dim=-1, dtype=torch.float32).to(dt)
    idx = idx.to(torch.int32)
    outs = []
    for _ in range(2):
        out = torch.zeros(m, H, dtype=dt, device=DEV)
        gemmainfer_csrc.fused_batched_moe(x.to(DEV), Wd["gate_up_packed"], Wd["gate_up_scales"], Wd["down_packed"],
                                          Wd["down_scales"], idx.to(DEV), w.to(DEV), out, gs)
        torch.cuda.synchronize()
        outs.append(out)
    assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16))
    assert_dtype_close(outs[0], _oracle(W, x, idx, w, torch.zeros(m, H), gs, "fp16"), "fp16", f"fp16 m={m}")


@pytest.mark.parametrize("tag", ["fp16", "fp32"])
def test_moe_duplicates_invalid_ids_and_many_rows(tag):
    dt = DT[tag]
    e, h, i, k, gs = 8, 256, 128, 4, 64
    W = _moe_weights(e, h, i, gs, seed=820, dt=dt)
    Wd = {n: v.to(DEV) for n, v in W.items()}
    for m in (3, 64):
        g = torch.Generator().manual_seed(821 + m)
        idx = torch.randint(-1, e + 1, (m, k), generator=g, dtype=torch.int64)   # duplicates, -1 and E
        w = torch.rand((m, k), generator=g).to(dt)
        x = synth.activations(m, h, seed=822 + m).to(dt)
        out = torch.zeros(m, h, dtype=dt, device=DEV)
        gemmainfer_csrc.fused_batched_moe(x.to(DEV), Wd["gate_up_packed"], Wd["gate_up_scales"],
                                          Wd["down_packed"], Wd["down_scales"], idx.to(DEV), w.to(DEV), out, gs)
        torch.cuda.synchronize()
        assert_dtype_close(out, _oracle(W, x, idx, w, torch.zeros(m, h), gs, tag), tag, f"dups {tag} m={m}")


@pytest.mark.parametrize("tag", ["fp16", "fp32"])
@pytest.mark.parametrize("m,k,e", [(20, 2, 4), (3, 64, 80)])
def test_moe_skewed_and_wide_top_k(tag, m, k, e):
    """One expert taking most slots of a launch (several passes of 8 slots
    over its words; a 20-row call is one launch of 40 slots at top_k 2), and
    top_k = 64 (one row, 64 slots, per launch)."""
    dt = DT[tag]
    h, i, gs = 256, 128, 64
    W = _moe_weights(e, h, i, gs, seed=840 + k, dt=dt)
    Wd = {n: v.to(DEV) for n, v in W.items()}
    g = torch.Generator().manual_seed(841 + k)
    if k == 2:
        idx = torch.ones((m, k), dtype=torch.int32)
        idx[::5, 1] = 3
        idx[2, 0] = -1
    else:
        idx = torch.stack([torch.randperm(e, generator=g)[:k] for _ in range(m)]).to(torch.int32)
    w = torch.softmax(torch.randn((m, k), generator=g), dim=-1).to(dt)
    x = synth.activations(m, h, seed=842 + k).to(dt)
    out_in = (torch.randn(m, h, generator=g) * 0.1).to(dt)
    out = out_in.to(DEV).clone()
    gemmainfer_csrc.fused_batched_moe(x.to(DEV), Wd["gate_up_packed"], Wd["gate_up_scales"], Wd["down_packed"],
                                      Wd["down_scales"], idx.to(DEV), w.to(DEV), out, gs)
    torch.cuda.synchronize()
    assert_dtype_close(out, _oracle(W, x, idx, w, out_in, gs, tag), tag, f"skewed {tag} m={m} top_k={k}")


@pytest.mark.parametrize("tag", ["fp16", "fp32"])
def test_moe_reference_golden(tag):
    g = np.load(GOLDEN / f"moe_m3_dups_gs64_{tag}.npz")
    dt = DT[tag]
    t = lambda k: torch.from_numpy(g[k]).to(DEV)  # noqa: E731
    out = torch.zeros(g["x"].shape, dtype=dt, device=DEV)
    gemmainfer_csrc.fused_batched_moe(t("x"), t("gate_up_packed"), t("gate_up_scales"), t("down_packed"),
                                      t("down_scales"), t("idx"), t("w"), out, int(g["group_size"]))
    torch.cuda.synchronize()
    ref = g["out"].astype(np.float64)
    st = O.error_stats(np64(out), ref)
    # the reference rounds gate/up, each expert output and each accumulation to the dtype
    assert st["rel_l2"] < (1e-5 if tag == "fp32" else 3e-3), st
    assert st["max_abs_over_rms"] < (1e-4 if tag == "fp32" else 2e-2), st


@pytest.mark.parametrize("tag", ["fp16", "fp32"])
@pytest.mark.parametrize("m,k,n,gs", [(1, 2816, 2816, 128), (6, 2816, 4096, 64), (33, 512, 200, 64),
                                      (3, 2816, 64, 128)])
def test_linear(tag, m, k, n, gs):
    dt = DT[tag]
    B, S = synth.linear_weights(k, n, gs, seed=830 + m)
    A = synth.activations(m, k, seed=831 + m).to(dt)
    S = S.to(dt)
    C = torch.full((m, n), float("nan"), dtype=dt, device=DEV)   # overwritten
    gemmainfer_csrc.marlin_w4a16(A.to(DEV), B.to(DEV), S.to(DEV), C, gs)
    torch.cuda.synchronize()
    ref = O.w4a16_linear(np64(A), B.numpy(), np64(S), gs)
    assert_dtype_close(C, ref, tag, f"linear {tag} m={m} k={k} n={n} gs={gs}")


@pytest.mark.parametrize("tag", ["fp16", "fp32"])
def test_linear_reference_golden_and_softcap(tag):
    g = np.load(GOLDEN / f"linear_m3_k512_n128_gs128_{tag}.npz")
    dt = DT[tag]
    A, B, S = (torch.from_numpy(g[k]).to(DEV) for k in ("A", "B_packed", "scales"))
    C = torch.empty(g["C"].shape, dtype=dt, device=DEV)
    gemmainfer_csrc.marlin_w4a16(A, B, S, C, int(g["group_size"]))
    torch.cuda.synchronize()
    ref = g["C"].astype(np.float64)
    got = np64(C)
    if tag == "fp32":
        np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-5 * np.abs(ref).max())
    else:
        ulp = np.ldexp(1.0, np.frexp(np.maximum(np.abs(ref), 2.0 ** -14))[1] - 11)
        assert np.all(np.abs(got - ref) <= ulp), "more than one fp16 ulp from the reference"
    # the lm_head epilogue cap * tanh(y / cap) (gemma.py:356-357) in the same dtype
    y = ops.w4a16_linear(A * 8, B, S, int(g["group_size"]), softcap=30.0)
    ref_c = O.softcap(O.w4a16_linear(np64(A * 8), g["B_packed"], g["scales"].astype(np.float64),
                                     int(g["group_size"])), 30.0)
    assert y.dtype == dt and float(y.abs().max()) <= 30.0
    assert_dtype_close(y, ref_c, tag, f"softcap {tag}")
