"""GPU parity of checkpoint ingest (gemmainfer/utils/weights.py:100-159) and of
the dense W4A16 callers at Gemma-4-26B-A4B shapes with the checkpoint's group
size 64 (attention.py:115-122, activations.py:26-28 -> marlin_w4a16).

Ingest must be bit-exact against torch's own transposition (the reference's
``t.t()`` + copy); linears against the oracle within the tolerance gate."""
from __future__ import annotations

import numpy as np
import pytest
import torch
from safetensors.torch import save_file

from gemmainfer_amd import checkpoint as C
from gemmainfer_amd import ops, synth
from oracle import moe_oracle as O
from tests.helpers import assert_bf16_close, assert_logits_close, np64

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.mark.parametrize("n,k", [(1, 8), (63, 512), (704, 2816), (2112, 2816), (2816, 2112), (130, 72)])
@pytest.mark.parametrize("sdt", [torch.bfloat16, torch.float16, torch.float32])
def test_ingest_matches_torch_transpose(n, k, sdt):
    print(f"ingest n={n} k={k} {sdt}", flush=True)
    g = torch.Generator().manual_seed(n * 7 + k)
    wp = torch.randint(-2 ** 31, 2 ** 31 - 1, (n, k // 8), generator=g, dtype=torch.int64).to(torch.int32)
    groups = max(1, k // 64)
    ws = (torch.randn(n, groups, generator=g) * 0.02).to(sdt)
    p, s = C.ingest_linear(wp.to(DEV), ws.to(DEV))
    assert torch.equal(p.cpu(), wp.t().contiguous())
    assert torch.equal(s.cpu(), ws.t().to(torch.bfloat16).contiguous())


def test_ingest_into_gate_up_halves():
    e, h, i = 3, 256, 96
    gu = torch.full((e, h // 8, 2 * i), 7, dtype=torch.int32, device=DEV)
    gus = torch.zeros((e, h // 64, 2 * i), dtype=torch.bfloat16, device=DEV)
    ref_p = torch.empty((e, h // 8, 2 * i), dtype=torch.int32)
    ref_s = torch.empty((e, h // 64, 2 * i), dtype=torch.bfloat16)
    for x in range(e):
        for proj, lo in ((0, 0), (1, i)):
            g = torch.Generator().manual_seed(10 * x + proj)
            wp = torch.randint(0, 2 ** 31 - 1, (i, h // 8), generator=g, dtype=torch.int64).to(torch.int32)
            ws = torch.randn(i, h // 64, generator=g).to(torch.bfloat16)
            C.ingest_linear(wp.to(DEV), ws.to(DEV), gu[x, :, lo:lo + i], gus[x, :, lo:lo + i])
            ref_p[x, :, lo:lo + i] = wp.t()        # weights.py:152-159
            ref_s[x, :, lo:lo + i] = ws.t()
    assert torch.equal(gu.cpu(), ref_p) and torch.equal(gus.cpu(), ref_s)


def _to_ckpt(packed, scales):
    """Kernel layout -> compressed-tensors layout (what a checkpoint holds)."""
    return packed.t().contiguous(), scales.t().contiguous()


def test_synthetic_checkpoint_layer(tmp_path):
    """A compressed-tensors checkpoint with the multimodal key prefix, two layers
    and a vision tensor: layer 0 is ingested, its tensors come back bit-exact,
    and the dense linears and the MoE block run on them match the oracle fed
    straight from the checkpoint tensors."""
    h, i_moe, e, gs, top_k = 256, 128, 8, 64, 2
    dense_shapes = {"self_attn.q_proj": (256, 512), "self_attn.k_proj": (256, 128),
                    "self_attn.v_proj": (256, 128), "self_attn.o_proj": (512, 256),
                    "mlp.gate_proj": (256, 384), "mlp.up_proj": (256, 384), "mlp.down_proj": (384, 256)}
    pre = "model.language_model.layers."
    tensors, originals = {}, {}
    for layer in (0, 1):
        for j, (name, (k, n)) in enumerate(dense_shapes.items()):
            p, s = synth.linear_weights(k, n, gs, seed=100 * layer + j)
            wp, ws = _to_ckpt(p, s)
            tensors[f"{pre}{layer}.{name}.weight_packed"] = wp
            tensors[f"{pre}{layer}.{name}.weight_scale"] = ws
            if layer == 0:
                originals[C.DENSE_LINEARS[name]] = (p, s, wp, ws)
        W = synth.moe_weights(E=e, H=h, I=i_moe, group_size=gs, seed=7 + layer)
        for x in range(e):
            gp, gsc = _to_ckpt(W["gate_up_packed"][x, :, :i_moe], W["gate_up_scales"][x, :, :i_moe])
            up, usc = _to_ckpt(W["gate_up_packed"][x, :, i_moe:], W["gate_up_scales"][x, :, i_moe:])
            dp, dsc = _to_ckpt(W["down_packed"][x], W["down_scales"][x])
            for proj, (a, b) in (("gate_proj", (gp, gsc)), ("up_proj", (up, usc)), ("down_proj", (dp, dsc))):
                tensors[f"{pre}{layer}.experts.{x}.{proj}.weight_packed"] = a
                tensors[f"{pre}{layer}.experts.{x}.{proj}.weight_scale"] = b
        R = synth.router_weights(e, h, seed=layer)
        tensors[f"{pre}{layer}.router.proj.weight"] = R["gate"]
        tensors[f"{pre}{layer}.router.scale"] = R["router_scale"]
        tensors[f"{pre}{layer}.router.per_expert_scale"] = R["expert_scale"]
        tensors[f"{pre}{layer}.input_layernorm.weight"] = torch.ones(h, dtype=torch.bfloat16)
        if layer == 0:
            W0, R0 = W, R
    tensors["model.vision_tower.layers.0.mlp.up_proj.weight_packed"] = torch.zeros(4, 4, dtype=torch.int32)
    keys = sorted(tensors)
    save_file({k: tensors[k] for k in keys[: len(keys) // 2]}, str(tmp_path / "model-00001.safetensors"))
    save_file({k: tensors[k] for k in keys[len(keys) // 2:]}, str(tmp_path / "model-00002.safetensors"))

    got = C.load_layer(C.safetensors_files(tmp_path), 0, DEV)
    assert set(got["dense"]) == set(C.DENSE_LINEARS.values())
    x = synth.activations(3, 512, seed=5)
    for name, (p, s, wp, ws) in originals.items():
        gp, gsc = got["dense"][name]
        assert torch.equal(gp.cpu(), p) and torch.equal(gsc.cpu(), s), name
        k = p.shape[0] * 8
        y = ops.w4a16_linear(x[:, :k].contiguous().to(DEV), gp, gsc, gs)
        op, osc = O.from_compressed(wp.numpy(), np64(ws))
        assert_bf16_close(y, O.w4a16_linear(np64(x[:, :k]), op, osc, gs), f"ckpt {name}")
    m = got["moe"]
    for key in ("gate_up_packed", "gate_up_scales", "down_packed", "down_scales"):
        assert torch.equal(m[key].cpu(), W0[key]), key
    assert torch.equal(m["gate"].cpu(), R0["gate"]) and torch.equal(m["expert_scale"].cpu(), R0["expert_scale"])
    xm = synth.activations(5, h, seed=6).to(DEV)
    out, idx, w, logits = ops.moe_layer_from_hidden(
        xm, m["router_scale"], m["gate"], m["gate_up_packed"], m["gate_up_scales"], m["down_packed"],
        m["down_scales"], top_k, gs, expert_scale=m["expert_scale"])
    ref_logits, _ = O.router_logits(np64(xm), np64(R0["router_scale"]), np64(R0["gate"]))
    assert_logits_close(logits, ref_logits, "ckpt router")
    ref_out, ref_idx, _, _ = O.moe_layer_from_logits(
        np64(xm), np64(logits), W0["gate_up_packed"].numpy(), np64(W0["gate_up_scales"]),
        W0["down_packed"].numpy(), np64(W0["down_scales"]), top_k, gs,
        expert_scale=np64(R0["expert_scale"]))
    np.testing.assert_array_equal(idx.cpu().numpy(), ref_idx)
    assert_bf16_close(out, ref_out, "ckpt moe block")


# Gemma-4-26B-A4B dense W4A16 linears (K, N): sliding-window attention (16 heads
# x 256, 8 kv heads), global attention (16 x 512, 2 kv heads), shared MLP 2112.
DENSE_GEMMA = {
    "q": (2816, 4096), "kv": (2816, 2048), "o": (4096, 2816),
    "q_global": (2816, 8192), "kv_global": (2816, 1024), "o_global": (8192, 2816),
    "mlp_gate_up": (2816, 2112), "mlp_down": (2112, 2816),
}


@pytest.mark.parametrize("name", list(DENSE_GEMMA))
@pytest.mark.parametrize("m", [1, 7, 64])
def test_dense_callers_gemma_gs64(name, m):
    k, n = DENSE_GEMMA[name]
    print(f"dense {name} m={m} k={k} n={n}", flush=True)
    B, S = synth.linear_weights(k, n, 64, seed=k + n)
    A = synth.activations(m, k, seed=m)
    C_ = ops.w4a16_linear(A.to(DEV), B.to(DEV), S.to(DEV), 64)
    cols = torch.randperm(n, generator=torch.Generator().manual_seed(m))[:384].sort().values
    ref = O.w4a16_linear(np64(A), B[:, cols].numpy(), np64(S[:, cols]), 64)
    assert_bf16_close(C_[:, cols.to(DEV)], ref, f"dense {name} m={m}")


@pytest.mark.parametrize("m", [1, 2, 7, 64])
def test_linear_multi_qkv(m):
    """q, k, v of one input in one call: bit-identical to three separate linears
    at 1-2 rows (same kernel, same sums), within tolerance of the oracle on
    sampled columns at every M (3+ rows split K over the whole grid, so the
    partial sums differ from separate calls)."""
    print(f"qkv m={m}", flush=True)
    shapes = [(2816, 4096), (2816, 2048), (2816, 2048)]
    W = [synth.linear_weights(k, n, 64, seed=50 + i) for i, (k, n) in enumerate(shapes)]
    Wd = [(B.to(DEV), S.to(DEV)) for B, S in W]
    A = synth.activations(m, 2816, seed=60 + m).to(DEV)
    outs = ops.w4a16_linear_multi(A, Wd, 64)
    for i, ((B, S), (Bd, Sd)) in enumerate(zip(W, Wd)):
        if m <= 2:
            sep = ops.w4a16_linear(A, Bd, Sd, 64)
            assert torch.equal(outs[i], sep), f"projection {i}"
        cols = torch.arange(0, B.shape[1], 17)
        ref = O.w4a16_linear(np64(A), B[:, cols].numpy(), np64(S[:, cols]), 64)
        assert_bf16_close(outs[i][:, cols.to(DEV)], ref, f"qkv[{i}] m={m}")


@pytest.mark.parametrize("m", [1, 2, 7, 64])
def test_gated_mlp_act(m):
    """Shared-MLP gate/up with the gelu*up epilogue (one launch at 1-2 rows)
    against the oracle of activations.py:26-28."""
    print(f"gated mlp m={m}", flush=True)
    k, n = 2816, 2112
    G = synth.linear_weights(k, n, 64, seed=70)
    U = synth.linear_weights(k, n, 64, seed=71)
    A = synth.activations(m, k, seed=72 + m)
    out = ops.gated_mlp_act(A.to(DEV), (G[0].to(DEV), G[1].to(DEV)), (U[0].to(DEV), U[1].to(DEV)), 64)
    cols = torch.arange(0, n, 11)
    ref = O.gated_mlp_act(np64(A), (G[0][:, cols].numpy(), np64(G[1][:, cols])),
                          (U[0][:, cols].numpy(), np64(U[1][:, cols])), 64)
    assert_bf16_close(out[:, cols.to(DEV)], ref, f"gated mlp m={m}")


@pytest.mark.parametrize("m,k,gs,floor", [(5, 2880, 128, True), (12, 4096, 128, False), (3, 8192, 64, False)])
def test_matrix_core_narrow_group_sizes(m, k, gs, floor):
    """The 3-16 row matrix-core path at group size 128 (floor-size scales: rows
    past the last whole group dropped) and at a long K with group size 64."""
    n = 2048
    print(f"mfma narrow m={m} k={k} gs={gs} floor={floor}", flush=True)
    g = torch.Generator().manual_seed(m + k)
    B = torch.randint(-(2 ** 31), 2 ** 31 - 1, (k // 8, n), generator=g, dtype=torch.int64).to(torch.int32)
    groups = k // gs if floor else -(-k // gs)
    S = (torch.randn(groups, n, generator=g).abs() * 0.02).to(torch.bfloat16)
    A = synth.activations(m, k, seed=m)
    C = ops.w4a16_linear(A.to(DEV), B.to(DEV), S.to(DEV), gs)
    cols = torch.arange(0, n, 5)
    ref = O.w4a16_linear(np64(A), B[:, cols].numpy(), np64(S[:, cols]), gs)
    assert_bf16_close(C[:, cols.to(DEV)], ref, f"mfma narrow m={m} k={k} gs={gs}")
