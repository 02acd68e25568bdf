"""Checkpoint ingest for the W4A16 path: compressed-tensors safetensors -> the
layout the kernels read.

Restates the parts of gemmainfer/utils/weights.py:55-159 that feed this path:
key cleaning (``model.language_model.`` / ``language_model.`` -> ``model.``,
weights.py:66-70), one decoder layer's tensors by suffix (weights.py:81-159),
and the transposition of every W4A16 linear: compressed-tensors stores
``weight_packed`` int32 [N, K/8] and ``weight_scale`` [N, K/gs]; the kernels
read packed [K/8, N] and bf16 scales [K/gs, N] (weights.py:100-147 ``t.t()``),
with an expert's gate_proj and up_proj in columns [0, I) and [I, 2I) of
gate_up (weights.py:148-159).

The transposition runs on the device through ``gi_w4a16_ingest`` (one tiled
launch per tensor); tensors are read with ``safetensors.safe_open`` (no
pickle).  Reading is host work; nothing here computes on the CPU.
"""
from __future__ import annotations

from pathlib import Path
from typing import Dict, Iterable, List, Optional, Tuple

import torch
from safetensors import safe_open

from . import _lib as L
from .ops import _DTYPE_CODE, _on_device, _ptr, _require, _stream

# suffix (after "model.layers.<i>.") of each dense W4A16 linear -> name used here
DENSE_LINEARS = {
    "self_attn.q_proj": "q_proj",
    "self_attn.k_proj": "k_proj",
    "self_attn.v_proj": "v_proj",
    "self_attn.o_proj": "o_proj",
    "mlp.gate_proj": "mlp_gate_proj",
    "mlp.up_proj": "mlp_up_proj",
    "mlp.down_proj": "mlp_down_proj",
}
# router tensors, copied as they are (weights.py:116-121)
ROUTER_TENSORS = {
    "router.proj.weight": "gate",
    "router.scale": "router_scale",
    "router.per_expert_scale": "expert_scale",
}


def clean_key(key: str) -> str:
    """weights.py:66-70: the multimodal checkpoint's language-model prefix."""
    if key.startswith("model.language_model."):
        return "model." + key[len("model.language_model."):]
    if key.startswith("language_model."):
        return "model." + key[len("language_model."):]
    return key


def split_layer_key(key: str) -> Optional[Tuple[int, str]]:
    """``model.layers.<i>.<suffix>`` -> (i, suffix) (weights.py:81-85), else None.
    Vision tensors are skipped (weights.py:63)."""
    if "vision" in key:
        return None
    parts = clean_key(key).split(".")
    if len(parts) >= 4 and parts[1] == "layers" and parts[2].isdigit():
        return int(parts[2]), ".".join(parts[3:])
    return None


def classify_suffix(suffix: str):
    """What one layer tensor is, for this path:
      ("dense", name, "weight_packed"|"weight_scale")
      ("expert", idx, "gate_proj"|"up_proj"|"down_proj", "weight_packed"|"weight_scale")
      ("router", name)
    or None for tensors this path does not use (norms, attention norms, ...)."""
    for pre, name in DENSE_LINEARS.items():
        for kind in ("weight_packed", "weight_scale"):
            if suffix == f"{pre}.{kind}":
                return ("dense", name, kind)
    if suffix in ROUTER_TENSORS:
        return ("router", ROUTER_TENSORS[suffix])
    if suffix.startswith("experts."):
        p = suffix.split(".")
        if len(p) == 4 and p[1].isdigit() and p[2] in ("gate_proj", "up_proj", "down_proj") \
                and p[3] in ("weight_packed", "weight_scale"):
            return ("expert", int(p[1]), p[2], p[3])
    return None


def scan_layer(paths: Iterable, layer: int) -> Dict[tuple, Tuple[str, str, tuple, str]]:
    """Index one layer's tensors across safetensors files without reading them:
    classify_suffix(...) -> (file, key, shape, dtype string)."""
    out = {}
    for path in sorted(str(p) for p in paths):
        with safe_open(path, framework="pt", device="cpu") as f:
            for key in f.keys():
                lk = split_layer_key(key)
                if lk is None or lk[0] != layer:
                    continue
                c = classify_suffix(lk[1])
                if c is None:
                    continue
                sl = f.get_slice(key)
                out[c] = (path, key, tuple(sl.get_shape()), sl.get_dtype())
    return out


def ingest_linear(weight_packed: torch.Tensor, weight_scale: torch.Tensor,
                  packed_out: Optional[torch.Tensor] = None,
                  scales_out: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """compressed-tensors [N, K/8] words + [N, G] scales (device tensors) ->
    (packed [K/8, N] int32, scales [G, N] bf16).  ``packed_out`` /
    ``scales_out`` may be column slices of wider row-major buffers (the
    gate/up halves of an expert); otherwise they are allocated."""
    dev = _on_device(weight_packed, weight_scale)
    _require(weight_packed.dim() == 2 and weight_packed.dtype == torch.int32,
             "weight_packed must be int32 [N, K/8]")
    _require(weight_scale.dim() == 2 and weight_scale.shape[0] == weight_packed.shape[0],
             "weight_scale must be [N, groups]")
    _require(weight_scale.dtype in (torch.bfloat16, torch.float16, torch.float32),
             "weight_scale must be bf16, fp16 or fp32", TypeError)
    n, kp = weight_packed.shape
    g = weight_scale.shape[1]
    if packed_out is None:
        packed_out = torch.empty((kp, n), dtype=torch.int32, device=dev)
    if scales_out is None:
        scales_out = torch.empty((g, n), dtype=torch.bfloat16, device=dev)
    _on_device(weight_packed, packed_out, scales_out)
    _require(tuple(packed_out.shape) == (kp, n) and packed_out.dtype == torch.int32 and
             packed_out.stride(1) == 1, f"packed_out must be int32 [{kp}, {n}] with unit column stride")
    _require(tuple(scales_out.shape) == (g, n) and scales_out.dtype == torch.bfloat16 and
             scales_out.stride(1) == 1, f"scales_out must be bf16 [{g}, {n}] with unit column stride")
    ld = packed_out.stride(0)
    _require(g <= 1 or scales_out.stride(0) == ld,
             "packed_out and scales_out must share one row stride")
    _require(ld >= n, "row stride of the outputs must be >= N")
    wp = weight_packed.contiguous()
    ws = weight_scale.contiguous()
    L.check(L.load().gi_w4a16_ingest(_ptr(wp), _ptr(ws), _DTYPE_CODE[ws.dtype], n, kp * 8, g,
                                     _ptr(packed_out), _ptr(scales_out), ld, _stream(dev)),
            "w4a16_ingest")
    return packed_out, scales_out


def ingest_batched(weight_packed: torch.Tensor, weight_scale: torch.Tensor, packed_out: torch.Tensor,
                   scales_out: torch.Tensor) -> None:
    """``B`` linears of one shape in one launch: weight_packed [B, N, K/8] and
    weight_scale [B, N, G] (device tensors, checkpoint layout) into
    packed_out [B, K/8, N] and scales_out [B, G, N] (unit column stride; views
    such as the gate or up half of gate_up are fine)."""
    dev = _on_device(weight_packed, weight_scale, packed_out, scales_out)
    _require(weight_packed.dim() == 3 and weight_packed.dtype == torch.int32, "weight_packed must be int32 [B, N, K/8]")
    _require(weight_scale.dim() == 3 and weight_scale.shape[:2] == weight_packed.shape[:2],
             "weight_scale must be [B, N, groups]")
    _require(weight_scale.dtype in (torch.bfloat16, torch.float16, torch.float32),
             "weight_scale must be bf16, fp16 or fp32", TypeError)
    b, n, kp = weight_packed.shape
    g = weight_scale.shape[2]
    _require(tuple(packed_out.shape) == (b, kp, n) and packed_out.dtype == torch.int32 and packed_out.stride(2) == 1,
             f"packed_out must be int32 [{b}, {kp}, {n}] with unit column stride")
    _require(tuple(scales_out.shape) == (b, g, n) and scales_out.dtype == torch.bfloat16 and scales_out.stride(2) == 1,
             f"scales_out must be bf16 [{b}, {g}, {n}] with unit column stride")
    ld = packed_out.stride(1)
    _require(g <= 1 or scales_out.stride(1) == ld, "packed_out and scales_out must share one row stride")
    wp = weight_packed.contiguous()
    ws = weight_scale.contiguous()
    L.check(L.load().gi_w4a16_ingest_batched(
        _ptr(wp), _ptr(ws), _DTYPE_CODE[ws.dtype], b, n, kp * 8, g, n * kp, n * g, _ptr(packed_out),
        _ptr(scales_out), ld, packed_out.stride(0), scales_out.stride(0), _stream(dev)), "w4a16_ingest_batched")


def load_layer(paths: Iterable, layer: int, device, dtype=torch.bfloat16) -> dict:
    """One decoder layer's W4A16 tensors on ``device``:

      {"dense": {name: (packed [K/8, N], scales [G, N])},
       "moe": {"gate_up_packed" [E, H/8, 2I], "gate_up_scales" [E, G, 2I],
               "down_packed" [E, I/8, H], "down_scales" [E, G, H],
               "gate" [E, H], "router_scale" [H], "expert_scale" [E]}}

    Missing pieces are simply absent (a dense-MLP layer has no "moe")."""
    paths = [str(p) for p in paths]
    idx = scan_layer(paths, layer)
    handles = {p: safe_open(p, framework="pt", device="cpu") for p in {v[0] for v in idx.values()}}

    def read_cpu(c):
        path, key, _, _ = idx[c]
        return handles[path].get_tensor(key)

    def read(c):
        return read_cpu(c).to(device)

    out = {"dense": {}, "moe": {}}
    for name in DENSE_LINEARS.values():
        kp_, ks_ = ("dense", name, "weight_packed"), ("dense", name, "weight_scale")
        if kp_ in idx and ks_ in idx:
            out["dense"][name] = ingest_linear(read(kp_), read(ks_))
    experts = sorted({c[1] for c in idx if c[0] == "expert"})
    if experts:
        e_count = experts[-1] + 1
        g_shape = idx[("expert", experts[0], "gate_proj", "weight_packed")][2]
        d_shape = idx[("expert", experts[0], "down_proj", "weight_packed")][2]
        gs_shape = idx[("expert", experts[0], "gate_proj", "weight_scale")][2]
        ds_shape = idx[("expert", experts[0], "down_proj", "weight_scale")][2]
        i_size, hp = g_shape
        h_size, ip = d_shape
        _require(hp * 8 == h_size and ip * 8 == i_size,
                 f"expert shapes disagree: gate_proj {g_shape}, down_proj {d_shape}")
        moe = out["moe"]
        moe["gate_up_packed"] = torch.zeros((e_count, hp, 2 * i_size), dtype=torch.int32, device=device)
        moe["gate_up_scales"] = torch.zeros((e_count, gs_shape[1], 2 * i_size), dtype=torch.bfloat16,
                                            device=device)
        moe["down_packed"] = torch.zeros((e_count, ip, h_size), dtype=torch.int32, device=device)
        moe["down_scales"] = torch.zeros((e_count, ds_shape[1], h_size), dtype=torch.bfloat16,
                                         device=device)
        if experts == list(range(e_count)):
            # every expert present: one batched transpose per tensor kind
            for proj, lo, dp, ds in (("gate_proj", 0, "gate_up_packed", "gate_up_scales"),
                                     ("up_proj", i_size, "gate_up_packed", "gate_up_scales"),
                                     ("down_proj", 0, "down_packed", "down_scales")):
                wp = torch.stack([read_cpu(("expert", e, proj, "weight_packed")) for e in experts]).to(device)
                ws = torch.stack([read_cpu(("expert", e, proj, "weight_scale")) for e in experts]).to(device)
                n = wp.shape[1]
                ingest_batched(wp, ws, moe[dp][:, :, lo:lo + n], moe[ds][:, :, lo:lo + n])
        else:
            for e in experts:
                for proj, lo in (("gate_proj", 0), ("up_proj", i_size)):
                    ingest_linear(read(("expert", e, proj, "weight_packed")),
                                  read(("expert", e, proj, "weight_scale")),
                                  moe["gate_up_packed"][e, :, lo:lo + i_size],
                                  moe["gate_up_scales"][e, :, lo:lo + i_size])
                ingest_linear(read(("expert", e, "down_proj", "weight_packed")),
                              read(("expert", e, "down_proj", "weight_scale")),
                              moe["down_packed"][e], moe["down_scales"][e])
    for name in ROUTER_TENSORS.values():
        if ("router", name) in idx:
            out["moe"][name] = read(("router", name)).to(dtype).contiguous()
    if not out["moe"]:
        del out["moe"]
    return out


def safetensors_files(model_dir) -> List[str]:
    """The ``*.safetensors`` files of a checkpoint directory (weights.py:55-59)."""
    return sorted(str(p) for p in Path(model_dir).glob("*.safetensors"))
