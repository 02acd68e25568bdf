"""GPU parity of the Token-Union MoE path against the CPU oracle.

Routing ids, the unique-expert list and the slot map must be bit-exact; bf16
outputs must pass the tolerance gate in tests/helpers.py.
"""
import numpy as np
import pytest
import torch

from gemmainfer_amd import ops, synth
from gemmainfer_amd import _lib as L
from oracle import moe_oracle as O
from tests.helpers import assert_bf16_close, assert_logits_close, np64, record_parity

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _dev(d):
    return {k: v.to(DEV) for k, v in d.items()}


def _oracle_moe(x, W, idx, w, out_in, gs):
    return O.fused_batched_moe(np64(x), W["gate_up_packed"].numpy(), np64(W["gate_up_scales"]),
                               W["down_packed"].numpy(), np64(W["down_scales"]), idx.cpu().numpy(),
                               np64(w), np64(out_in), gs)


@pytest.fixture(scope="module")
def small():
    W = synth.moe_weights(E=8, H=256, I=128, group_size=64, seed=11)
    return W, _dev(W)


@pytest.fixture(scope="module")
def gemma128():
    # Gemma-4-26B-A4B expert shapes, group 128: down has 6 groups, the last ragged.
    W = synth.moe_weights(E=128, H=2816, I=704, group_size=128, seed=1)
    return W, _dev(W)


# ---------------------------------------------------------------- routing
@pytest.mark.parametrize("m", [1, 7, 64, 200])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_route_topk_softmax(m, dtype):
    logits = synth.router_logits(m, 128, seed=m).to(dtype)
    idx, w = ops.route_topk_softmax(logits.to(DEV), 8)
    ref_idx, _, ref_w = O.route_topk_softmax(np64(logits), 8)
    np.testing.assert_array_equal(idx.cpu().numpy(), ref_idx)
    # weights: fp32 softmax then one bf16 rounding; allow one bf16 ulp
    np.testing.assert_allclose(np64(w), ref_w, rtol=2.0 ** -7, atol=0)
    if dtype == torch.float32:
        _, ti = torch.topk(logits, 8, dim=-1)  # (values, indices)
        np.testing.assert_array_equal(idx.cpu().numpy(), ti.numpy())


def test_route_ties_and_expert_scale():
    logits = torch.zeros(3, 128)
    logits[0, [5, 9, 77]] = 1.0            # ties among the top values
    logits[1, 100] = float("nan")          # NaN ranks highest
    es = torch.linspace(0.5, 1.5, 128)
    idx, w = ops.route_topk_softmax(logits.to(DEV), 8, expert_scale=es.to(DEV))
    ref_idx, _, ref_w = O.route_topk_softmax(np64(logits), 8, expert_scale=es.numpy())
    np.testing.assert_array_equal(idx.cpu().numpy(), ref_idx)
    finite = np.isfinite(ref_w)
    np.testing.assert_allclose(np64(w)[finite], ref_w[finite], rtol=2.0 ** -7)


# ---------------------------------------------------------------- alignment
ALIGN_CASES = [
    ("m1_distinct", [[3, 1, 4, 15, 9, 2, 6, 5]], 16),
    ("dup_across_tokens", [[1, 2], [2, 3], [3, 1]], 8),
    ("dup_within_token", [[4, 4, 4, 1]], 8),
    ("invalid_ids", [[-1, 3, 99, 3], [8, 0, -5, 2]], 8),
    ("all_same", [[6, 6], [6, 6], [6, 6]], 8),
    ("all_invalid", [[-1, 8], [9, -2]], 8),
]


@pytest.mark.parametrize("name,ids,E", ALIGN_CASES, ids=[c[0] for c in ALIGN_CASES])
@pytest.mark.parametrize("idt", [torch.int32, torch.int64])
def test_align_known_answers(name, ids, E, idt):
    idx = torch.tensor(ids, dtype=idt)
    got = ops.moe_align(idx.to(DEV), E)
    ref = O.token_union_align(idx.numpy(), E)
    u = int(got["num_unique"].item())
    assert u == ref.num_unique
    np.testing.assert_array_equal(got["unique_experts"][:u].cpu().numpy(), ref.unique_experts)
    np.testing.assert_array_equal(got["slot_to_unique"].cpu().numpy(), ref.slot_to_unique)
    np.testing.assert_array_equal(got["offsets"][:u + 1].cpu().numpy(), ref.offsets)
    n = int(ref.offsets[-1])
    np.testing.assert_array_equal(got["slots"][:n].cpu().numpy(), ref.slots)


@pytest.mark.parametrize("m,noise", [(1, 0.0), (7, 0.5), (8, 0.5), (32, 0.0)])
def test_align_random_routing(m, noise):
    logits = synth.router_logits(m, 128, seed=100 + m, verify_noise=noise)
    idx, _, _ = O.route_topk_softmax(np64(logits), 8)
    got = ops.moe_align(torch.from_numpy(idx).to(DEV), 128)
    ref = O.token_union_align(idx, 128)
    u = int(got["num_unique"].item())
    assert u == ref.num_unique
    np.testing.assert_array_equal(got["unique_experts"][:u].cpu().numpy(), ref.unique_experts)
    np.testing.assert_array_equal(got["slot_to_unique"].cpu().numpy(), ref.slot_to_unique)
    np.testing.assert_array_equal(got["slots"][:int(ref.offsets[-1])].cpu().numpy(), ref.slots)


# ---------------------------------------------------------------- fused MoE
@pytest.mark.parametrize("m", [1, 2, 5, 8, 9, 33, 300])
def test_fused_small_shapes(small, m):
    W, Wd = small
    x = synth.activations(m, 256, seed=m)
    logits = synth.router_logits(m, 8, seed=m)
    idx, _, w = O.route_topk_softmax(np64(logits), 2)
    idx_t = torch.from_numpy(idx)
    w_t = torch.from_numpy(w).to(torch.bfloat16)
    out_in = (torch.randn(m, 256) * 0.1).to(torch.bfloat16)   # out is accumulated into
    out = out_in.to(DEV).clone()
    ops.fused_batched_moe(x.to(DEV), Wd["gate_up_packed"], Wd["gate_up_scales"], Wd["down_packed"],
                          Wd["down_scales"], idx_t.to(DEV), w_t.to(DEV), out, 64)
    ref, _ = _oracle_moe(x, W, idx_t, w_t, out_in, 64)
    assert_bf16_close(out, ref, f"small m={m}")


@pytest.mark.parametrize("gs", [8, 16, 24, 32, 96])
@pytest.mark.parametrize("m", [1, 3, 9])
def test_fused_group_sizes(gs, m):
    """Group sizes that are not multiples of 32 take the VALU kernel, the others
    the matrix-core kernel; 24 and 96 leave a ragged last group (ceil groups)."""
    W = synth.moe_weights(E=8, H=256, I=128, group_size=gs, seed=gs + m)
    Wd = _dev(W)
    x = synth.activations(m, 256, seed=m + 40)
    logits = synth.router_logits(m, 8, seed=m + 40)
    idx, _, w = O.route_topk_softmax(np64(logits), 2)
    idx_t = torch.from_numpy(idx)
    w_t = torch.from_numpy(w).to(torch.bfloat16)
    out = torch.zeros(m, 256, dtype=torch.bfloat16, device=DEV)
    ops.fused_batched_moe(x.to(DEV), Wd["gate_up_packed"], Wd["gate_up_scales"], Wd["down_packed"],
                          Wd["down_scales"], idx_t.to(DEV), w_t.to(DEV), out, gs)
    ref, _ = _oracle_moe(x, W, idx_t, w_t, torch.zeros(m, 256), gs)
    assert_bf16_close(out, ref, f"gs={gs} m={m}")


def test_fused_duplicates_invalid_and_dtypes(small):
    """Duplicate ids within a token are separate slots (pybind.cpp:219-244, no
    MAX_MATCH cap); ids outside [0, E) are skipped (marlin.cu:304,473);
    int64 ids and fp32 weights are accepted and cast like marlin.cu:631-636."""
    W, Wd = small
    x = synth.activations(3, 256, seed=5)
    idx = torch.tensor([[1, 1, 1, 1], [7, -1, 8, 7], [2, 3, 2, 3]], dtype=torch.int64)
    w = torch.tensor([[0.3, 0.2, 0.1, 0.4], [0.5, 9.0, 9.0, 0.25], [0.1, 0.2, 0.3, 0.4]])
    out = torch.zeros(3, 256, dtype=torch.bfloat16, device=DEV)
    ops.fused_batched_moe(x.to(DEV), Wd["gate_up_packed"], Wd["gate_up_scales"], Wd["down_packed"],
                          Wd["down_scales"], idx.to(DEV), w.to(DEV), out, 64)
    ref, _ = _oracle_moe(x, W, idx, w, torch.zeros(3, 256), 64)
    assert_bf16_close(out, ref, "duplicates/invalid")


@pytest.mark.parametrize("m,noise", [(1, 0.0), (7, 0.5), (8, 0.5)])
def test_fused_gemma_shapes_gs128(gemma128, m, noise):
    W, Wd = gemma128
    x = synth.activations(m, 2816, seed=m)
    logits = synth.router_logits(m, 128, seed=m, verify_noise=noise)
    idx, _, w = O.route_topk_softmax(np64(logits), 8)
    idx_t = torch.from_numpy(idx)
    w_t = torch.from_numpy(w).to(torch.bfloat16)
    out = torch.zeros(m, 2816, dtype=torch.bfloat16, device=DEV)
    ops.fused_batched_moe(x.to(DEV), Wd["gate_up_packed"], Wd["gate_up_scales"], Wd["down_packed"],
                          Wd["down_scales"], idx_t.to(DEV), w_t.to(DEV), out, 128)
    ref, al = _oracle_moe(x, W, idx_t, w_t, torch.zeros(m, 2816), 128)
    stats = assert_bf16_close(out, ref, f"gemma m={m}")
    print(f"m={m} U={al.num_unique} {stats}")
    if (m, noise) in ((1, 0.0), (7, 0.5)):
        record_parity("cfg1_M1" if m == 1 else "cfg2_M7", stats, unique_experts=al.num_unique)


@pytest.mark.parametrize("m", [64, 512])
def test_prefill_grouped_gemm_gemma(gemma128, m):
    """From 64 rows the sorted-by-expert grouped GEMM replaces the 8-row slices
    (gemma.py:99-112): BASELINE config 3 at m=512, i.i.d. router logits."""
    W, Wd = gemma128
    x = synth.activations(m, 2816, seed=500 + m)
    logits = synth.router_logits(m, 128, seed=500 + m)
    idx, _, w = O.route_topk_softmax(np64(logits), 8)
    idx_t = torch.from_numpy(idx)
    w_t = torch.from_numpy(w).to(torch.bfloat16)
    out_in = (torch.randn(m, 2816) * 0.1).to(torch.bfloat16)   # accumulated into
    out = out_in.to(DEV).clone()
    ops.fused_batched_moe(x.to(DEV), Wd["gate_up_packed"], Wd["gate_up_scales"], Wd["down_packed"],
                          Wd["down_scales"], idx_t.to(DEV), w_t.to(DEV), out, 128)
    ref, al = _oracle_moe(x, W, idx_t, w_t, out_in, 128)
    stats = assert_bf16_close(out, ref, f"prefill m={m}")
    print(f"m={m} U={al.num_unique} {stats}")
    if m == 512:
        record_parity("cfg3_M512", stats, unique_experts=al.num_unique)


def test_prefill_duplicates_invalid_skewed(small):
    """Prefill path with duplicate ids inside a token, ids outside [0, E), int64
    ids, fp32 weights and a skewed routing that puts > 32 pairs on one expert
    (several 32-row passes of one expert's weights)."""
    W, Wd = small
    m = 96
    g = torch.Generator().manual_seed(9)
    idx = torch.randint(0, 8, (m, 4), generator=g, dtype=torch.int64)
    idx[::3, 0] = 5                       # expert 5 gets > 64 pairs
    idx[1::7, 1] = idx[1::7, 2]           # duplicates within a token
    idx[2::11, 3] = -1                    # skipped slots
    idx[4::13, 2] = 8                     # id == E: skipped
    w = torch.rand(m, 4, generator=g)
    x = synth.activations(m, 256, seed=12)
    out = torch.zeros(m, 256, dtype=torch.bfloat16, device=DEV)
    ops.fused_batched_moe(x.to(DEV), Wd["gate_up_packed"], Wd["gate_up_scales"], Wd["down_packed"],
                          Wd["down_scales"], idx.to(DEV), w.to(DEV), out, 64)
    ref, _ = _oracle_moe(x, W, idx, w, torch.zeros(m, 256), 64)
    assert_bf16_close(out, ref, "prefill duplicates/invalid")


@pytest.mark.parametrize("m,top_k,idx_dtype", [(1024, 8, torch.int32), (1025, 8, torch.int64),
                                               (1100, 4, torch.int32), (64, 1, torch.int64),
                                               (96, 16, torch.int32)])
def test_prefill_many_pairs_and_heavy_expert(small, m, top_k, idx_dtype):
    """The front launch's align sorts up to 8192 (token, slot) pairs from
    registers (1024 x 8 is the largest such call, 64 x 1 the smallest prefill
    call) and more in a loop (1025 x 8); top_k 16 takes the combine's general
    form.  Eight experts take ~500-1000 pairs
    each, i.e. 11-22 passes of 48 pairs per workgroup, and one expert takes
    most of them; ids outside [0, E) are skipped, duplicate ids within a
    token each count, and the output is the same on a second call."""
    W, Wd = small
    g = torch.Generator().manual_seed(m + top_k)
    idx = torch.randint(0, 8, (m, top_k), generator=g, dtype=torch.int64)
    idx[::2, 0] = 3                        # expert 3: > 512 pairs
    if top_k > 1:
        idx[1::5, 1] = idx[1::5, 0]        # duplicates within a token
        idx[3::17, 1] = 8                  # id == E: skipped
    idx[7::23, 0] = -1                     # skipped slots
    w = torch.rand(m, top_k, generator=g).to(torch.bfloat16)
    x = synth.activations(m, 256, seed=m)
    out_in = (torch.randn(m, 256, generator=g) * 0.1).to(torch.bfloat16)
    print(f"prefill modes m={m} top_k={top_k} {idx_dtype}", flush=True)
    out = out_in.to(DEV).clone()
    ops.fused_batched_moe(x.to(DEV), Wd["gate_up_packed"], Wd["gate_up_scales"], Wd["down_packed"],
                          Wd["down_scales"], idx.to(idx_dtype).to(DEV), w.to(DEV), out, 64)
    ref, _ = _oracle_moe(x, W, idx, w, out_in, 64)
    assert_bf16_close(out, ref, f"prefill modes m={m} top_k={top_k}")
    out2 = out_in.to(DEV).clone()
    ops.fused_batched_moe(x.to(DEV), Wd["gate_up_packed"], Wd["gate_up_scales"], Wd["down_packed"],
                          Wd["down_scales"], idx.to(idx_dtype).to(DEV), w.to(DEV), out2, 64)
    assert torch.equal(out, out2)


@pytest.mark.parametrize("H,I,gs", [(320, 96, 64), (320, 96, 128), (256, 96, 128), (320, 128, 128),
                                     (2816, 704, 256)])
def test_prefill_partial_last_scale_group(H, I, gs):
    """K ends inside a scale group that is not the last of its 8-k-block chunk
    (I = 96: 3 k blocks; H = 320: 10): the partial group's sums must reach the
    output, as in the oracle, which counts ceil(K / gs) groups."""
    m, e, top_k = 64, 8, 4
    W = synth.moe_weights(E=e, H=H, I=I, group_size=gs, seed=40 + I + gs)
    Wd = _dev(W)
    g = torch.Generator().manual_seed(41)
    idx = torch.stack([torch.randperm(e, generator=g)[:top_k] for _ in range(m)]).to(torch.int32)
    w = torch.softmax(torch.randn(m, top_k, generator=g), dim=-1).to(torch.bfloat16)   # sums to 1, gemma.py:78
    x = synth.activations(m, H, seed=42)
    print(f"prefill partial group H={H} I={I} gs={gs}", flush=True)
    out = torch.zeros(m, H, dtype=torch.bfloat16, device=DEV)
    ops.fused_batched_moe(x.to(DEV), Wd["gate_up_packed"], Wd["gate_up_scales"], Wd["down_packed"],
                          Wd["down_scales"], idx.to(DEV), w.to(DEV), out, gs)
    ref, _ = _oracle_moe(x, W, idx, w, torch.zeros(m, H), gs)
    assert_bf16_close(out, ref, f"prefill partial group H={H} I={I} gs={gs}")


@pytest.mark.parametrize("I", [7168, 7200])
def test_prefill_scale_table_at_lds_limit(I):
    """Group size 32 puts I / 32 scale groups of a down workgroup's 64 column
    quads in LDS beside the staged tiles: at I = 7168 that workgroup uses the
    whole 160 KB of a CU, at I = 7200 it would not fit and the call takes the
    general path instead of failing its launch."""
    m, top_k, gs, H = 64, 2, 32, 256
    W = synth.moe_weights(E=4, H=H, I=I, group_size=gs, seed=31)
    Wd = _dev(W)
    g = torch.Generator().manual_seed(32)
    idx = torch.randint(0, 4, (m, top_k), generator=g, dtype=torch.int32)
    w = torch.rand(m, top_k, generator=g).to(torch.bfloat16)
    x = synth.activations(m, H, seed=33)
    out = torch.zeros(m, H, dtype=torch.bfloat16, device=DEV)
    ops.fused_batched_moe(x.to(DEV), Wd["gate_up_packed"], Wd["gate_up_scales"], Wd["down_packed"],
                          Wd["down_scales"], idx.to(DEV), w.to(DEV), out, gs)
    ref, _ = _oracle_moe(x, W, idx, w, torch.zeros(m, H), gs)
    assert_bf16_close(out, ref, f"prefill I={I} gs32")


@pytest.mark.parametrize("m", [100, 512])
def test_prefill_layer_matches_oracle_and_is_deterministic(gemma128, m):
    """Layer mode through the prefill path: routing bit-exact, output within
    tolerance, and bitwise-identical across calls.  The routed ids reach the
    align from 7 (m = 100) or 32 (m = 512) routing workgroups of the same
    launch."""
    W, Wd = gemma128
    x = synth.activations(m, 2816, seed=77 + m)
    logits = synth.router_logits(m, 128, seed=77 + m)
    outs = []
    for _ in range(2):
        out, idx, w = ops.moe_layer(x.to(DEV), logits.to(DEV), Wd["gate_up_packed"],
                                    Wd["gate_up_scales"], Wd["down_packed"], Wd["down_scales"], 8, 128)
        outs.append(out.clone())
    ref_out, ref_idx, ref_w, _ = O.moe_layer_from_logits(
        np64(x), np64(logits), W["gate_up_packed"].numpy(), np64(W["gate_up_scales"]),
        W["down_packed"].numpy(), np64(W["down_scales"]), 8, 128)
    np.testing.assert_array_equal(idx.cpu().numpy(), ref_idx)
    np.testing.assert_allclose(np64(w), ref_w, rtol=2.0 ** -7)
    assert_bf16_close(outs[0], ref_out, "prefill layer")
    assert torch.equal(outs[0], outs[1])


def test_layer_from_logits_gemma(gemma128):
    """Layer mode; 12 and 16 rows take several launches of up to 8 rows each."""
    W, Wd = gemma128
    for m, noise in ((1, 0.0), (7, 0.5), (12, 0.5), (16, 0.0)):
        x = synth.activations(m, 2816, seed=10 + m)
        logits = synth.router_logits(m, 128, seed=10 + m, verify_noise=noise)
        out, idx, w = ops.moe_layer(x.to(DEV), logits.to(DEV), Wd["gate_up_packed"],
                                    Wd["gate_up_scales"], Wd["down_packed"], Wd["down_scales"],
                                    8, 128)
        ref_out, ref_idx, ref_w, al = O.moe_layer_from_logits(
            np64(x), np64(logits), W["gate_up_packed"].numpy(), np64(W["gate_up_scales"]),
            W["down_packed"].numpy(), np64(W["down_scales"]), 8, 128)
        np.testing.assert_array_equal(idx.cpu().numpy(), ref_idx)
        np.testing.assert_allclose(np64(w), ref_w, rtol=2.0 ** -7)
        assert_bf16_close(out, ref_out, f"layer m={m}")


# ---------------------------------------------------------------- router front-end
ROUTER_SHAPES = [(1, 2816, 128), (7, 2816, 128), (8, 2816, 128), (13, 2816, 128),
                 (100, 2816, 128), (3, 256, 8), (5, 1024, 1000), (2, 4096, 64), (9, 520, 36),
                 (40, 1024, 72), (17, 4096, 130)]


@pytest.mark.parametrize("m,h,e", ROUTER_SHAPES)
def test_router_logits_match_oracle(m, h, e):
    """gemma.py:75-76 in one launch against the oracle: every logit within one
    bf16 ulp, nearly all bit-identical; with and without router_scale."""
    x = synth.activations(m, h, seed=m + h) * torch.linspace(0.05, 8, m).unsqueeze(1).to(torch.bfloat16)
    W = synth.router_weights(e, h, seed=e)
    for rs in (W["router_scale"], None):
        print(f"router m={m} h={h} e={e} scale={rs is not None}", flush=True)
        got = ops.moe_router_logits(x.to(DEV), None if rs is None else rs.to(DEV), W["gate"].to(DEV))
        ref, xr = O.router_logits(np64(x), None if rs is None else np64(rs), np64(W["gate"]), 1e-6)
        assert_logits_close(got, ref, f"router m={m} h={h} e={e}",
                            abs_terms=np.abs(xr) @ np.abs(np64(W["gate"])).T, k=h)


def test_router_matches_reference_golden():
    g = np.load(GOLDEN / "router_m3_h512_e16.npz")
    x = _bits_to_bf16(g["x_bf16"]).to(DEV)
    rs = _bits_to_bf16(g["router_scale_bf16"]).to(DEV)
    gate = _bits_to_bf16(g["gate_bf16"]).to(DEV)
    got = ops.moe_router_logits(x, rs, gate, float(g["eps"]))
    ref = O.bf16_bits_to_f64(g["logits_bf16"])
    assert_logits_close(got, ref, "router golden", min_exact=0.9)


@pytest.mark.parametrize("m", [1, 7, 100])
def test_layer_from_hidden_gemma(gemma128, m):
    """The MoE block from the hidden state: logits as the oracle's router
    front-end; routing bit-exact and output within tolerance against the
    oracle run on those logits; bitwise equal to moe_layer on the same logits."""
    W, Wd = gemma128
    R = synth.router_weights(128, 2816, seed=m)
    x = synth.activations(m, 2816, seed=40 + m).to(DEV)
    es = R["expert_scale"].to(DEV)
    print(f"layer_from_hidden m={m}", flush=True)
    out, idx, w, logits = ops.moe_layer_from_hidden(
        x, R["router_scale"].to(DEV), R["gate"].to(DEV), Wd["gate_up_packed"], Wd["gate_up_scales"],
        Wd["down_packed"], Wd["down_scales"], 8, 128, expert_scale=es)
    ref_logits, xr = O.router_logits(np64(x), np64(R["router_scale"]), np64(R["gate"]), 1e-6)
    assert_logits_close(logits, ref_logits, f"layer_from_hidden logits m={m}",
                        abs_terms=np.abs(xr) @ np.abs(np64(R["gate"])).T, k=2816)
    ref_out, ref_idx, ref_w, _ = O.moe_layer_from_logits(
        np64(x), np64(logits), W["gate_up_packed"].numpy(), np64(W["gate_up_scales"]),
        W["down_packed"].numpy(), np64(W["down_scales"]), 8, 128, expert_scale=np64(R["expert_scale"]))
    np.testing.assert_array_equal(idx.cpu().numpy(), ref_idx)
    np.testing.assert_allclose(np64(w), ref_w, rtol=2.0 ** -7)
    assert_bf16_close(out, ref_out, f"layer_from_hidden m={m}")
    out2, idx2, w2 = ops.moe_layer(x, logits, Wd["gate_up_packed"], Wd["gate_up_scales"],
                                   Wd["down_packed"], Wd["down_scales"], 8, 128, expert_scale=es)
    assert torch.equal(out, out2) and torch.equal(idx, idx2) and torch.equal(w, w2)


def test_deterministic_bitwise(gemma128):
    W, Wd = gemma128
    x = synth.activations(7, 2816, seed=3).to(DEV)
    logits = synth.router_logits(7, 128, seed=3, verify_noise=0.5).to(DEV)
    outs = []
    for _ in range(3):
        out, _, _ = ops.moe_layer(x, logits, Wd["gate_up_packed"], Wd["gate_up_scales"],
                                  Wd["down_packed"], Wd["down_scales"], 8, 128)
        outs.append(out.clone())
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[0], outs[2])


def test_zero_scales_give_zero(small):
    """The reference's own test state (zero-initialised buffers, gemma.py:43-58)."""
    _, Wd = small
    x = synth.activations(5, 256, seed=1).to(DEV)
    idx = torch.randint(0, 8, (5, 2), dtype=torch.int32).to(DEV)
    w = torch.full((5, 2), 0.5, dtype=torch.bfloat16, device=DEV)
    out = torch.zeros(5, 256, dtype=torch.bfloat16, device=DEV)
    ops.fused_batched_moe(x, Wd["gate_up_packed"], torch.zeros_like(Wd["gate_up_scales"]),
                          Wd["down_packed"], Wd["down_scales"], idx, w, out, 64)
    assert torch.count_nonzero(out).item() == 0


def test_device_status_clean_and_timeout_path(small):
    W, Wd = small
    assert ops.workspace_status() == 0
    # A spin limit of 1 poll forces the bounded-wait error path from the host:
    # the kernel must still finish and report the flag.
    x = synth.activations(4, 256, seed=2).to(DEV)
    idx = torch.tensor([[0, 1], [2, 3], [4, 5], [6, 7]], dtype=torch.int32, device=DEV)
    w = torch.full((4, 2), 0.5, dtype=torch.bfloat16, device=DEV)
    out = torch.zeros(4, 256, dtype=torch.bfloat16, device=DEV)
    ops.fused_batched_moe(x, Wd["gate_up_packed"], Wd["gate_up_scales"], Wd["down_packed"],
                          Wd["down_scales"], idx, w, out, 64, spin_limit=1)
    torch.cuda.synchronize()
    st = ops.workspace_status()
    assert st in (0, L.DEVICE_SPIN_TIMEOUT)
    assert ops.workspace_status() == 0  # read clears it
    # the workspace is usable again afterwards
    out2 = torch.zeros(4, 256, dtype=torch.bfloat16, device=DEV)
    ops.fused_batched_moe(x, Wd["gate_up_packed"], Wd["gate_up_scales"], Wd["down_packed"],
                          Wd["down_scales"], idx, w, out2, 64)
    ref, _ = _oracle_moe(x.cpu(), W, idx.cpu(), w.cpu(), torch.zeros(4, 256), 64)
    assert_bf16_close(out2, ref, "after timeout path")
    assert ops.workspace_status() == 0


# ---------------------------------------------------------------- golden vectors
GOLDEN = __import__("pathlib").Path(__file__).resolve().parent / "golden"


def _bits_to_bf16(a):
    return torch.from_numpy(a.view(np.int16).copy()).view(torch.bfloat16)


@pytest.mark.parametrize("name", ["moe_m5_small_top2_gs64", "moe_m1_small_top2_gs64", "moe_m3_dups_gs64"])
def test_fused_matches_reference_golden(name):
    """Inputs/outputs produced by the reference's own CPU fallback (pybind.cpp:198-245)."""
    g = dict(np.load(GOLDEN / f"{name}.npz"))
    x = _bits_to_bf16(g["x_bf16"])
    gus, ds, w = (_bits_to_bf16(g[k]) for k in ("gate_up_scales_bf16", "down_scales_bf16", "w_bf16"))
    gu, dp, idx = (torch.from_numpy(g[k]) for k in ("gate_up_packed", "down_packed", "idx"))
    gs = int(g["group_size"])
    out = torch.zeros_like(x).to(DEV)
    ops.fused_batched_moe(x.to(DEV), gu.to(DEV), gus.to(DEV), dp.to(DEV), ds.to(DEV), idx.to(DEV),
                          w.to(DEV), out, gs)
    ref_golden = O.bf16_bits_to_f64(g["out_bf16"])
    # the reference fallback rounds several intermediates to bf16 (see tests/test_oracle.py)
    st = O.error_stats(np64(out), ref_golden)
    assert st["rel_l2"] < 1.5e-2 and st["max_abs_over_rms"] < 0.1, st
    # and the strict gate against the float64 oracle on the same inputs
    oracle, _ = O.fused_batched_moe(np64(x), g["gate_up_packed"], np64(gus), g["down_packed"], np64(ds),
                                    g["idx"], np64(w), np.zeros(x.shape), gs)
    assert_bf16_close(out, oracle, name)
