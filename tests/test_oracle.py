"""Pins the CPU oracle (oracle/moe_oracle.py) -- CPU only.

Each check is chosen so a plausible mistake (a dropped term, a wrong nibble
order or sign, a transposed operand, a wrong group index, a mis-ordered
unique list) fails it:
  * golden vectors produced by the reference's own CPU C++ fallback
    (tests/golden, written from oracle/_ref by tests/golden/make_golden.py);
  * the reference fallback itself when oracle/_ref is built (this container);
  * library routines the reference calls (torch.topk / softmax / gelu / tanh);
  * closed forms, brute force on tiny inputs, invariants.
"""
from __future__ import annotations

import itertools
import sys
from pathlib import Path

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from gemmainfer_amd import synth
from oracle import moe_oracle as O

GOLDEN = Path(__file__).resolve().parent / "golden"
REF_DIR = Path(__file__).resolve().parents[1] / "oracle" / "_ref"


def f64(bits_u16) -> np.ndarray:
    return O.bf16_bits_to_f64(bits_u16)


def t64(t: torch.Tensor) -> np.ndarray:
    return t.float().numpy().astype(np.float64)


def load(name):
    return dict(np.load(GOLDEN / f"{name}.npz"))


def ref_module():
    if not any(REF_DIR.glob("gemmainfer_csrc_ref*.so")):
        pytest.skip("oracle/_ref not built (reference tree absent)")
    sys.path.insert(0, str(REF_DIR))
    import gemmainfer_csrc_ref  # noqa: PLC0415
    return gemmainfer_csrc_ref


# --------------------------------------------------------------------------- bf16
def test_bf16_round_matches_torch_cast():
    rng = np.random.default_rng(0)
    vals = np.concatenate([
        rng.standard_normal(200_000) * 10.0 ** rng.integers(-40, 39, 200_000),
        # exact ties between two bf16 values (round half to even)
        (np.arange(-5000, 5000) + 0.5).astype(np.float64) * 2.0 ** -7,
        np.array([0.0, -0.0, 1e-45, -1e-45, 2.0 ** -130, 3.4e38, -3.4e38, np.inf, -np.inf]),
    ])
    vals = vals[np.abs(vals) < 3.4e38].astype(np.float32).astype(np.float64)
    vals = np.concatenate([vals, [np.inf, -np.inf]])
    ours = O.bf16_round(vals)
    theirs = torch.from_numpy(vals.astype(np.float32)).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(ours, theirs.astype(np.float64))
    assert np.isnan(O.bf16_round(np.array([np.nan])))[0]


# --------------------------------------------------------------------------- int4
def test_unpack_exhaustive_codes_positions_and_scale_sign():
    # every code 0..15 at every nibble position 0..7
    for q, pos in itertools.product(range(16), range(8)):
        word = np.array([[(q << (4 * pos)) | (0x8 << (4 * ((pos + 1) % 8)))]], dtype=np.int64)
        word = word.astype(np.uint32).view(np.int32)
        codes = O.unpack_int4(word)[:, 0]
        assert codes[pos] == q
        assert codes[(pos + 1) % 8] == 8
        for s in (0.5, -0.25):
            w = O.dequant(word, np.array([[s]]), 8)[:, 0]
            assert w[pos] == (q - 8) * s
            assert w[(pos + 1) % 8] == 0.0


def test_pack_quantize_round_trip():
    rng = np.random.default_rng(1)
    q = rng.integers(0, 16, size=(64, 12))
    np.testing.assert_array_equal(O.unpack_int4(O.pack_int4(q)), q)
    w = rng.standard_normal((12, 64)) * 0.05
    packed, s = O.quantize_w4(w, 32)
    codes = O.unpack_int4(packed)
    assert codes.min() >= 1 and codes.max() <= 15  # symmetric: round(w/s) in [-7, 7]
    deq = O.dequant(packed, s, 32).T
    # quantisation error bounded by half a step per group
    err = np.abs(deq - w).reshape(12, 2, 32)
    assert np.all(err <= 0.5 * s.T[:, :, None] + 1e-12)


def test_dequant_drops_rows_past_the_last_scale_group():
    rng = np.random.default_rng(2)
    packed = rng.integers(-2**31, 2**31, size=(88, 16)).astype(np.int32)  # K = 704
    s6 = rng.random((6, 16))
    w6 = O.dequant(packed, s6, 128)
    w5 = O.dequant(packed, s6[:5], 128)        # reference-style K//gs groups
    np.testing.assert_array_equal(w5[:640], w6[:640])
    assert np.all(w5[640:] == 0.0)


def test_w4a16_brute_force_and_integer_case():
    rng = np.random.default_rng(3)
    m, k, n, gs = 3, 64, 5, 16
    packed = rng.integers(-2**31, 2**31, size=(k // 8, n)).astype(np.int32)
    scales = rng.standard_normal((k // gs, n))
    a = rng.standard_normal((m, k))
    brute = np.zeros((m, n))
    for i in range(m):
        for j in range(n):
            for kk in range(k):
                word = int(packed[kk // 8, j]) & 0xFFFFFFFF
                q = (word >> (4 * (kk % 8))) & 0xF
                brute[i, j] += a[i, kk] * (q - 8) * scales[kk // gs, j]
    np.testing.assert_allclose(O.w4a16_linear(a, packed, scales, gs), brute, rtol=1e-12, atol=1e-12)
    # scale = 1, integer activations: exact integer matmul of (q - 8)
    ai = rng.integers(-3, 4, size=(m, k)).astype(np.float64)
    q = O.unpack_int4(packed)
    np.testing.assert_array_equal(O.w4a16_linear(ai, packed, np.ones((k // gs, n)), gs),
                                  ai @ (q - 8).astype(np.float64))


@pytest.mark.parametrize("name", ["linear_m1_k256_n96_gs64", "linear_m5_k512_n128_gs128",
                                  "linear_m3_k2816_n64_gs128"])
def test_linear_matches_reference_golden(name):
    g = load(name)
    ref = f64(g["C_bf16"])
    ours = O.w4a16_linear(f64(g["A_bf16"]), g["B_packed"], f64(g["scales_bf16"]), int(g["group_size"]))
    # the reference accumulates (a*w*s) per element in fp32 then rounds to bf16
    st = O.error_stats(ref, ours)
    assert st["rel_l2"] < 4e-3, st
    assert np.all(np.abs(ref - ours) <= 2.0 ** -7 * np.abs(ours) + 1e-2), st


# --------------------------------------------------------------------------- elementwise
def test_gelu_and_softcap_match_torch():
    x = torch.linspace(-12, 12, 20001, dtype=torch.float64)
    np.testing.assert_allclose(O.gelu_tanh(x.numpy()), F.gelu(x, approximate="tanh").numpy(),
                               rtol=1e-12, atol=1e-14)
    np.testing.assert_allclose(O.softcap(x.numpy() * 10, 30.0), (30 * torch.tanh(x * 10 / 30)).numpy(),
                               rtol=1e-12)


def test_elementwise_golden_roundtrip():
    g = load("elementwise")
    x, w = f64(g["x_bf16"]), f64(g["w_bf16"])
    r = 1.0 / np.sqrt((x * x).mean(-1, keepdims=True) + 1e-6)
    np.testing.assert_allclose(O.bf16_round(x * r * w), f64(g["rms_bf16"]), rtol=2.0 ** -7, atol=1e-6)
    np.testing.assert_allclose(O.bf16_round(x * r * (1 + w)), f64(g["rms_unit_bf16"]), rtol=2.0 ** -7,
                               atol=1e-6)
    # the reference's CPU softcap runs in bf16 tensor ops (pybind.cpp:134): x/cap and
    # tanh are each rounded to bf16 before the final product, so allow two bf16 ulps
    np.testing.assert_allclose(O.bf16_round(O.softcap(f64(g["logits_bf16"]), 30.0)), f64(g["capped_bf16"]),
                               rtol=2.0 ** -6, atol=1e-6)


def test_gated_mlp_act_matches_torch_statements():
    """activations.py:26-28 on bf16 tensors: F.gelu(approximate='tanh') of the
    bf16 gate output, times the bf16 up output, each rounded to bf16."""
    B1, S1 = synth.linear_weights(256, 96, 64, seed=41)
    B2, S2 = synth.linear_weights(256, 96, 64, seed=42)
    a = synth.activations(3, 256, seed=43)
    ours = O.gated_mlp_act(t64(a), (B1.numpy(), t64(S1)), (B2.numpy(), t64(S2)), 64)
    g = torch.from_numpy(O.bf16_round(O.w4a16_linear(t64(a), B1.numpy(), t64(S1), 64))).to(torch.bfloat16)
    u = torch.from_numpy(O.bf16_round(O.w4a16_linear(t64(a), B2.numpy(), t64(S2), 64))).to(torch.bfloat16)
    theirs = t64(F.gelu(g, approximate="tanh") * u)
    ulp = np.ldexp(1.0, np.frexp(np.maximum(np.abs(theirs), 2.0 ** -126))[1] - 8)
    # torch evaluates gelu in fp32, where tanh of a large negative argument is
    # exactly -1 and gelu(-5.6) is 0; the float64 oracle keeps ~1e-9 there
    assert np.all(np.abs(ours - theirs) <= ulp + 1e-7)
    assert np.mean(ours == theirs) > 0.97


# --------------------------------------------------------------------------- router front-end
def _ulp_bf16(v):
    """Spacing of bf16 values at |v| (normal range)."""
    _, e = np.frexp(np.maximum(np.abs(v), 2.0 ** -126))
    return np.ldexp(1.0, e - 8)


def test_router_golden_steps():
    """Each step of the oracle's router front-end against the fixture made by the
    reference's CPU rmsnorm (no weight) and the module's torch statements."""
    g = load("router_m3_h512_e16")
    x, rs, gate = f64(g["x_bf16"]), f64(g["router_scale_bf16"]), f64(g["gate_bf16"])
    eps = float(g["eps"])
    n = O.rmsnorm_noscale_bf16(x, eps)
    ref_n = f64(g["norm_bf16"])
    assert np.mean(n == ref_n) > 0.995
    assert np.all(np.abs(n - ref_n) <= _ulp_bf16(ref_n))
    # scale and product: exact given the reference's norm
    xr = O.bf16_round(ref_n * O.router_scale_bf16(rs, x.shape[1]))
    np.testing.assert_array_equal(xr, f64(g["x_normed_bf16"]))
    logits, xr_full = O.router_logits(x, rs, gate, eps)
    ref_l = f64(g["logits_bf16"])
    assert np.all(np.abs(logits - ref_l) <= _ulp_bf16(ref_l)), np.abs(logits - ref_l).max()
    assert np.mean(logits == ref_l) > 0.9


def test_router_steps_match_torch_statements():
    """gemma.py:75-76 as torch evaluates it on bf16 CPU tensors, at Gemma's shape."""
    R = ref_module()
    x = synth.activations(9, 2816, seed=31) * torch.linspace(0.01, 30, 9).unsqueeze(1).to(torch.bfloat16)
    W = synth.router_weights(128, 2816, seed=31)
    y = torch.empty_like(x)
    R.rmsnorm(x, torch.empty(0), y, 1e-6, False)
    n = O.rmsnorm_noscale_bf16(t64(x), 1e-6)
    assert np.all(np.abs(n - t64(y)) <= _ulp_bf16(t64(y)))
    assert np.mean(n == t64(y)) > 0.995
    s_torch = W["router_scale"] * (2816 ** -0.5)
    np.testing.assert_array_equal(O.router_scale_bf16(t64(W["router_scale"]), 2816), t64(s_torch))
    xr_torch = y * s_torch
    np.testing.assert_array_equal(O.bf16_round(t64(y) * t64(s_torch)), t64(xr_torch))
    lin = F.linear(xr_torch, W["gate"])
    ours = O.bf16_round(t64(xr_torch) @ t64(W["gate"]).T)
    assert np.all(np.abs(ours - t64(lin)) <= _ulp_bf16(t64(lin)))


def test_router_closed_forms():
    h, e = 256, 64
    # constant rows: norm = a / sqrt(a^2 + eps) -> bf16 1.0 for |a| >> sqrt(eps);
    # identity gate rows pick x_normed[e] = bf16(H^-0.5)
    x = np.full((2, h), 2.0)
    x[1] = -0.5
    gate = np.zeros((e, h))
    gate[np.arange(e), np.arange(e)] = 1.0
    logits, xr = O.router_logits(x, None, gate)
    c = float(torch.tensor(h ** -0.5, dtype=torch.float32).to(torch.bfloat16))
    np.testing.assert_array_equal(logits[0], np.full(e, c))
    np.testing.assert_array_equal(logits[1], np.full(e, -c))
    # all-zero row stays zero (eps keeps rsqrt finite)
    z, _ = O.router_logits(np.zeros((1, h)), None, gate)
    assert np.all(z == 0.0)
    # exact symmetries: negating router_scale negates the logits; a power-of-two
    # gate scale scales them exactly
    rng = np.random.default_rng(3)
    xs = O.bf16_round(rng.standard_normal((4, h)))
    rs = O.bf16_round(1 + 0.2 * rng.standard_normal(h))
    g = O.bf16_round(rng.standard_normal((e, h)))
    a, _ = O.router_logits(xs, rs, g)
    b, _ = O.router_logits(xs, -rs, g)
    d, _ = O.router_logits(xs, rs, 4.0 * g)
    np.testing.assert_array_equal(a, -b)
    np.testing.assert_array_equal(4.0 * a, d)
    # brute force on a tiny case: scalar loops with the same roundings
    xt, rt, gt = xs[:2, :16], rs[:16], g[:3, :16]
    ref = np.zeros((2, 3))
    for m in range(2):
        ms = sum(v * v for v in xt[m]) / 16
        r = np.float32(1.0 / np.sqrt(ms + np.float64(np.float32(1e-6))))
        for k in range(3):
            acc = 0.0
            for j in range(16):
                nv = O.bf16_round(np.float64(np.float32(xt[m, j]) * r))
                sv = O.bf16_round(np.float64(np.float32(rt[j]) * np.float32(16 ** -0.5)))
                acc += O.bf16_round(nv * sv) * gt[k, j]
            ref[m, k] = O.bf16_round(acc)
    np.testing.assert_array_equal(O.router_logits(xt, rt, gt)[0], ref)


# --------------------------------------------------------------------------- routing
@pytest.mark.parametrize("m,e,k", [(1, 128, 8), (7, 128, 8), (33, 64, 4), (5, 8, 2)])
def test_route_matches_torch_topk_softmax(m, e, k):
    logits = synth.router_logits(m, e, seed=m * e)
    idx, p, w = O.route_topk_softmax(t64(logits), k)
    tv, ti = torch.topk(logits.double(), k, dim=-1)
    np.testing.assert_array_equal(idx, ti.numpy())
    np.testing.assert_allclose(p, torch.softmax(tv, -1).numpy(), rtol=1e-12)
    np.testing.assert_allclose(p.sum(-1), 1.0, rtol=1e-12)            # expert_scale = 1
    assert np.all(np.diff(np.take_along_axis(t64(logits), idx.astype(np.int64), 1), axis=1) <= 0)
    np.testing.assert_array_equal(w, O.bf16_round(p))


def test_route_tie_rule_nan_and_expert_scale():
    logits = np.zeros((2, 16))
    logits[0, [3, 9, 12]] = 1.0
    logits[1, 5] = np.nan
    idx, p, _ = O.route_topk_softmax(logits, 4, expert_scale=np.arange(16) + 1.0)
    np.testing.assert_array_equal(idx[0], [3, 9, 12, 0])   # ties: lower index first
    assert idx[1, 0] == 5                                  # NaN ranks highest
    base = np.exp([1, 1, 1, 0]) / np.exp([1, 1, 1, 0]).sum()
    np.testing.assert_allclose(p[0], base * (idx[0] + 1.0), rtol=1e-12)


# --------------------------------------------------------------------------- alignment
def _reference_scan(idx_flat, E):
    """Literal restatement of the reference kernel's per-block scan
    (marlin.cu:298-331), uncapped: block u finds the u-th first occurrence."""
    S = len(idx_flat)
    out_u, out_slots = [], []
    u = 0
    while True:
        seen, target = 0, -1
        for s in range(S):
            e = idx_flat[s]
            if e < 0 or e >= E:
                continue
            if e not in idx_flat[:s]:
                if seen == u:
                    target = e
                    break
                seen += 1
        if target < 0:
            break
        out_u.append(target)
        out_slots.append([s for s in range(S) if idx_flat[s] == target])
        u += 1
    return out_u, out_slots


ALIGN_KATS = [
    ([[3, 1, 4, 15, 9, 2, 6, 5]], 16, [3, 1, 4, 15, 9, 2, 6, 5], [[0], [1], [2], [3], [4], [5], [6], [7]]),
    ([[1, 2], [2, 3], [3, 1]], 8, [1, 2, 3], [[0, 5], [1, 2], [3, 4]]),
    ([[4, 4, 4, 1]], 8, [4, 1], [[0, 1, 2], [3]]),
    ([[-1, 3, 99, 3], [8, 0, -5, 2]], 8, [3, 0, 2], [[1, 3], [5], [7]]),
    ([[6, 6], [6, 6], [6, 6]], 8, [6], [[0, 1, 2, 3, 4, 5]]),
    ([[-1, 8], [9, -2]], 8, [], []),
]


@pytest.mark.parametrize("ids,E,uniq,slots", ALIGN_KATS)
def test_align_known_answers(ids, E, uniq, slots):
    al = O.token_union_align(np.array(ids), E)
    assert al.unique_experts.tolist() == uniq
    got = [al.slots[al.offsets[u]:al.offsets[u + 1]].tolist() for u in range(al.num_unique)]
    assert got == slots
    for u, sl in enumerate(slots):
        assert all(al.slot_to_unique[s] == u for s in sl)
    assert np.all(al.slot_to_unique[[s for s in range(len(al.slot_to_unique))
                                     if all(s not in sl for sl in slots)]] == -1)


def test_align_matches_reference_scan_random():
    rng = np.random.default_rng(4)
    for _ in range(200):
        m, k, E = rng.integers(1, 10), rng.integers(1, 9), int(rng.integers(1, 20))
        ids = rng.integers(-2, E + 2, size=(m, k))
        al = O.token_union_align(ids, E)
        ru, rs = _reference_scan(ids.reshape(-1).tolist(), E)
        assert al.unique_experts.tolist() == ru
        assert [al.slots[al.offsets[u]:al.offsets[u + 1]].tolist() for u in range(al.num_unique)] == rs
        assert al.num_unique <= min(m * k, E)
        assert al.offsets[-1] == sum(1 for e in ids.reshape(-1) if 0 <= e < E)


# --------------------------------------------------------------------------- fused MoE
def _golden_moe(name):
    g = load(name)
    gs = int(g["group_size"])
    out, al = O.fused_batched_moe(f64(g["x_bf16"]), g["gate_up_packed"], f64(g["gate_up_scales_bf16"]),
                                  g["down_packed"], f64(g["down_scales_bf16"]), g["idx"],
                                  f64(g["w_bf16"]), np.zeros_like(f64(g["x_bf16"])), gs)
    return f64(g["out_bf16"]), out


@pytest.mark.parametrize("name", ["moe_m5_small_top2_gs64", "moe_m1_small_top2_gs64", "moe_m3_dups_gs64"])
def test_moe_matches_reference_golden(name):
    ref, ours = _golden_moe(name)
    # the reference fallback rounds gate/up, the activation, each expert output
    # and every accumulation to bf16; the oracle rounds only the activation
    st = O.error_stats(ref, ours)
    assert st["rel_l2"] < 1.5e-2, st
    assert st["max_abs_over_rms"] < 0.1, st


def test_moe_brute_force_tiny():
    rng = np.random.default_rng(5)
    E, H, I, gs, m, k = 3, 16, 8, 8, 2, 2
    gu = rng.integers(-2**31, 2**31, size=(E, H // 8, 2 * I)).astype(np.int32)
    gus = rng.random((E, H // gs, 2 * I)) * 0.1
    dp = rng.integers(-2**31, 2**31, size=(E, I // 8, H)).astype(np.int32)
    dss = rng.random((E, I // gs, H)) * 0.1
    x = rng.standard_normal((m, H))
    idx = np.array([[2, 0], [0, 0]])
    w = np.array([[0.75, 0.25], [0.5, 0.5]])
    out, _ = O.fused_batched_moe(x, gu, gus, dp, dss, idx, w, np.zeros((m, H)), gs, act_round=False)
    brute = np.zeros((m, H))
    for t in range(m):
        for j in range(k):
            e = idx[t, j]
            g_u = np.zeros(2 * I)
            for c in range(2 * I):
                for kk in range(H):
                    q = (int(gu[e, kk // 8, c]) & 0xFFFFFFFF) >> (4 * (kk % 8)) & 0xF
                    g_u[c] += x[t, kk] * (q - 8) * gus[e, kk // gs, c]
            a = 0.5 * g_u[:I] * (1 + np.tanh(np.sqrt(2 / np.pi) * (g_u[:I] + 0.044715 * g_u[:I] ** 3))) * g_u[I:]
            y = np.zeros(H)
            for h in range(H):
                for ii in range(I):
                    q = (int(dp[e, ii // 8, h]) & 0xFFFFFFFF) >> (4 * (ii % 8)) & 0xF
                    y[h] += a[ii] * (q - 8) * dss[e, ii // gs, h]
            brute[t] += O.bf16_round(w[t, j]) * y
    np.testing.assert_allclose(out, brute, rtol=1e-10, atol=1e-10)


def test_moe_invariants():
    W = synth.moe_weights(8, 64, 32, 16, seed=9)
    Wn = {k: (v.numpy() if v.dtype == torch.int32 else t64(v)) for k, v in W.items()}
    x = t64(synth.activations(9, 64, seed=9))
    logits = t64(synth.router_logits(9, 8, seed=9))
    idx, _, w = O.route_topk_softmax(logits, 3)
    args = (Wn["gate_up_packed"], Wn["gate_up_scales"], Wn["down_packed"], Wn["down_scales"])
    full, _ = O.fused_batched_moe(x, *args, idx, w, np.zeros_like(x), 16)
    # chunked (gemma.py:99-112) == unchunked
    np.testing.assert_allclose(O.chunked_batched_moe(x, *args, idx, w, np.zeros_like(x), 16), full,
                               rtol=1e-12, atol=1e-12)
    # accumulate semantics: out_in is added
    acc, _ = O.fused_batched_moe(x, *args, idx, w, np.ones_like(x), 16)
    np.testing.assert_allclose(acc, full + 1.0, rtol=1e-12, atol=1e-12)
    # linear in the routing weights (w exactly representable in bf16)
    w2 = np.full_like(w, 0.5)
    half, _ = O.fused_batched_moe(x, *args, idx, w2, np.zeros_like(x), 16)
    one, _ = O.fused_batched_moe(x, *args, idx, 2 * w2, np.zeros_like(x), 16)
    np.testing.assert_allclose(one, 2 * half, rtol=1e-12, atol=1e-12)
    # zero scales -> zero output (the reference's own zero-initialised test state)
    z, _ = O.fused_batched_moe(x, np.zeros_like(args[0]), np.zeros_like(args[1]), *args[2:], idx, w,
                               np.zeros_like(x), 16)
    assert np.all(z == 0.0)


# --------------------------------------------------------------------------- reference fallback
def test_oracle_against_reference_fallback_live():
    R = ref_module()
    W = synth.moe_weights(8, 256, 128, 64, seed=21)
    x = synth.activations(4, 256, seed=21)
    logits = synth.router_logits(4, 8, seed=21)
    top, idx = torch.topk(logits, 2, dim=-1)
    w = torch.softmax(top, -1).to(torch.bfloat16)
    out = torch.zeros(4, 256, dtype=torch.bfloat16)
    R.fused_batched_moe(x, W["gate_up_packed"], W["gate_up_scales"], W["down_packed"], W["down_scales"],
                        idx.to(torch.int32), w, out, 64)
    ours, _ = O.fused_batched_moe(t64(x), W["gate_up_packed"].numpy(), t64(W["gate_up_scales"]),
                                  W["down_packed"].numpy(), t64(W["down_scales"]), idx.numpy(), t64(w),
                                  np.zeros((4, 256)), 64)
    st = O.error_stats(t64(out), ours)
    assert st["rel_l2"] < 1.5e-2, st
    A = synth.activations(2, 2816, seed=22)
    B, S = synth.linear_weights(2816, 64, 128, seed=22)
    C = torch.empty(2, 64, dtype=torch.bfloat16)
    R.marlin_w4a16(A, B, S, C, 128)
    st = O.error_stats(t64(C), O.w4a16_linear(t64(A), B.numpy(), t64(S), 128))
    assert st["rel_l2"] < 4e-3, st


# --------------------------------------------------------------------------- fp16 / fp32
def test_round_to_matches_torch_casts():
    rng = np.random.default_rng(3)
    vals = np.concatenate([
        rng.standard_normal(100_000) * 10.0 ** rng.integers(-9, 6, 100_000),
        # exact ties between two fp16 values, normal and subnormal
        (np.arange(-3000, 3000) + 0.5).astype(np.float64) * 2.0 ** -10,
        (np.arange(-300, 300) + 0.5).astype(np.float64) * 2.0 ** -24,
        np.array([0.0, -0.0, 65504.0, 65520.0, -65520.0, 1e-9]),
    ]).astype(np.float32).astype(np.float64)
    theirs16 = torch.from_numpy(vals.astype(np.float32)).to(torch.float16).float().numpy().astype(np.float64)
    np.testing.assert_array_equal(O.round_to(vals, "fp16"), theirs16)
    np.testing.assert_array_equal(O.round_to(vals, "fp32"), vals)
    np.testing.assert_array_equal(O.round_to(vals, "bf16"), O.bf16_round(vals))
    with pytest.raises(ValueError):
        O.round_to(vals, "fp8")


@pytest.mark.parametrize("tag", ["fp16", "fp32"])
def test_linear_matches_reference_golden_other_dtypes(tag):
    g = load(f"linear_m3_k512_n128_gs128_{tag}")
    gs = int(g["group_size"])
    y = O.round_to(O.w4a16_linear(g["A"].astype(np.float64), g["B_packed"], g["scales"].astype(np.float64), gs),
                   tag)
    ref = g["C"].astype(np.float64)
    if tag == "fp32":   # float32 sums in the reference, float64 here
        np.testing.assert_allclose(y, ref, rtol=1e-5, atol=1e-5 * np.abs(ref).max())
    else:               # within one fp16 ulp
        ulp = np.ldexp(1.0, np.frexp(np.maximum(np.abs(ref), 2.0 ** -14))[1] - 11)
        assert np.all(np.abs(y - ref) <= ulp)


@pytest.mark.parametrize("tag", ["fp16", "fp32"])
def test_moe_matches_reference_golden_other_dtypes(tag):
    g = load(f"moe_m3_dups_gs64_{tag}")
    gs = int(g["group_size"])
    x = g["x"].astype(np.float64)
    out, _ = O.fused_batched_moe(x, g["gate_up_packed"], g["gate_up_scales"].astype(np.float64), g["down_packed"],
                                 g["down_scales"].astype(np.float64), g["idx"], g["w"].astype(np.float64),
                                 np.zeros_like(x), gs, dtype=tag)
    ref = g["out"].astype(np.float64)
    st = O.error_stats(O.round_to(out, tag), ref)
    # the reference fallback also rounds gate/up, each expert output and each
    # accumulation to the dtype; in fp32 only the sum order differs
    if tag == "fp32":
        assert st["rel_l2"] < 1e-5, st
    else:
        assert st["rel_l2"] < 3e-3, st
        assert st["max_abs_over_rms"] < 2e-2, st
