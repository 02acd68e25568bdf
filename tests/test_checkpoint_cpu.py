"""Host logic of checkpoint ingest (gemmainfer/utils/weights.py:55-159) and the
oracle's reading of the compressed-tensors layout; no GPU needed."""
from __future__ import annotations

import numpy as np
import torch
from safetensors.torch import save_file

from gemmainfer_amd import checkpoint as C
from gemmainfer_amd import synth
from oracle import moe_oracle as O


def test_clean_and_split_keys():
    assert C.clean_key("model.language_model.layers.3.mlp.up_proj.weight_packed") == \
        "model.layers.3.mlp.up_proj.weight_packed"
    assert C.clean_key("language_model.layers.0.router.scale") == "model.layers.0.router.scale"
    assert C.clean_key("model.layers.1.x") == "model.layers.1.x"
    assert C.split_layer_key("model.language_model.layers.12.experts.5.down_proj.weight_scale") == \
        (12, "experts.5.down_proj.weight_scale")
    assert C.split_layer_key("model.embed_tokens.weight") is None
    assert C.split_layer_key("model.vision_tower.layers.0.mlp.up_proj.weight_packed") is None
    assert C.split_layer_key("model.layers.x.mlp") is None


def test_classify_suffix():
    assert C.classify_suffix("self_attn.q_proj.weight_packed") == ("dense", "q_proj", "weight_packed")
    assert C.classify_suffix("mlp.down_proj.weight_scale") == ("dense", "mlp_down_proj", "weight_scale")
    assert C.classify_suffix("experts.17.gate_proj.weight_packed") == ("expert", 17, "gate_proj", "weight_packed")
    assert C.classify_suffix("router.proj.weight") == ("router", "gate")
    assert C.classify_suffix("router.per_expert_scale") == ("router", "expert_scale")
    for unused in ("input_layernorm.weight", "self_attn.q_norm.weight", "layer_scalar",
                   "experts.3.gate_proj.weight_shape", "experts.x.up_proj.weight_packed"):
        assert C.classify_suffix(unused) is None


def test_scan_layer_indexes_one_layer_without_reading(tmp_path):
    t = {
        "model.language_model.layers.0.self_attn.q_proj.weight_packed": torch.zeros(64, 4, dtype=torch.int32),
        "model.language_model.layers.0.self_attn.q_proj.weight_scale": torch.zeros(64, 1, dtype=torch.bfloat16),
        "model.language_model.layers.0.experts.2.up_proj.weight_scale": torch.zeros(16, 1, dtype=torch.float16),
        "model.language_model.layers.0.input_layernorm.weight": torch.zeros(32),
        "model.language_model.layers.1.self_attn.q_proj.weight_packed": torch.zeros(8, 4, dtype=torch.int32),
        "model.vision_tower.layers.0.self_attn.q_proj.weight_packed": torch.zeros(8, 4, dtype=torch.int32),
    }
    save_file(dict(list(t.items())[:3]), str(tmp_path / "a.safetensors"))
    save_file(dict(list(t.items())[3:]), str(tmp_path / "b.safetensors"))
    idx = C.scan_layer(C.safetensors_files(tmp_path), 0)
    assert set(idx) == {("dense", "q_proj", "weight_packed"), ("dense", "q_proj", "weight_scale"),
                        ("expert", 2, "up_proj", "weight_scale")}
    assert idx[("dense", "q_proj", "weight_packed")][2] == (64, 4)
    assert idx[("expert", 2, "up_proj", "weight_scale")][3] == "F16"


def test_oracle_reads_compressed_layout_brute_force():
    """Nibble i of word [n][j] is the code of k = 8j + i (value code - 8) times
    weight_scale[n][k // gs]: a scalar loop over the checkpoint layout."""
    n, k, gs = 5, 48, 16
    packed, scales = synth.linear_weights(k, n, gs, seed=4)       # kernel layout [K/8, N], [G, N]
    wp = packed.t().contiguous().numpy()                           # checkpoint layout [N, K/8]
    ws = scales.t().contiguous().float().numpy().astype(np.float64)
    ref = np.zeros((k, n))
    for nn in range(n):
        for kk in range(k):
            code = (int(wp[nn, kk // 8]) >> (4 * (kk % 8))) & 0xF
            ref[kk, nn] = (code - 8) * ws[nn, kk // gs]
    p2, s2 = O.from_compressed(wp, ws)
    np.testing.assert_array_equal(O.dequant(p2, s2, gs), ref)
    np.testing.assert_array_equal(p2, packed.numpy())
