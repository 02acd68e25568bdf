"""Synthetic inputs of the shapes and distributions the benchmark configurations name.

Weights: packed int4 words drawn uniformly over all 2^32 bit patterns (eight
i.i.d. codes 0..15 per word, zero point 8) and bf16 group scales
|N(0,1)| * 0.02.  Activations ~ N(0,1) in bf16.  Router logits N(0,1) fp32,
optionally a shared base plus per-token noise (speculative verify).  A fixed
seed gives the same tensors on every machine (torch's CPU generator); device
copies are made with ``.to(device)``.  ``device_moe_weights`` fills large
sets directly on the GPU with torch's device generator (for the benchmark,
where values only need the right distribution).
"""
from __future__ import annotations

import math

import torch

SCALE_STD = 0.02


def _gen(seed: int) -> torch.Generator:
    g = torch.Generator()
    g.manual_seed(int(seed))
    return g


def packed_words(shape, gen: torch.Generator) -> torch.Tensor:
    return torch.randint(-(2 ** 31), 2 ** 31, shape, generator=gen, dtype=torch.int64).to(torch.int32)


def group_scales(shape, gen: torch.Generator, std: float = SCALE_STD) -> torch.Tensor:
    return (torch.randn(shape, generator=gen).abs() * std).to(torch.bfloat16)


def moe_weights(E: int, H: int, I: int, group_size: int, seed: int = 0,
                scale_std: float = SCALE_STD) -> dict:
    """CPU tensors in the reference layout (weights.py:153-159): gate_up
    [E, H/8, 2I], down [E, I/8, H]; ceil(K/gs) scale groups per projection."""
    g = _gen(seed)
    return {
        "gate_up_packed": packed_words((E, H // 8, 2 * I), g),
        "gate_up_scales": group_scales((E, math.ceil(H / group_size), 2 * I), g, scale_std),
        "down_packed": packed_words((E, I // 8, H), g),
        "down_scales": group_scales((E, math.ceil(I / group_size), H), g, scale_std),
    }


def device_moe_weights(E: int, H: int, I: int, group_size: int, device, seed: int = 0,
                       scale_std: float = SCALE_STD) -> dict:
    """Same distributions, generated on the device (fast for 0.4 GB sets)."""
    g = torch.Generator(device=device)
    g.manual_seed(int(seed))

    def words(shape):
        return torch.randint(-(2 ** 31), 2 ** 31, shape, generator=g, dtype=torch.int64,
                             device=device).to(torch.int32)

    def scales(shape):
        return (torch.randn(shape, generator=g, device=device).abs() * scale_std).to(torch.bfloat16)

    return {
        "gate_up_packed": words((E, H // 8, 2 * I)),
        "gate_up_scales": scales((E, math.ceil(H / group_size), 2 * I)),
        "down_packed": words((E, I // 8, H)),
        "down_scales": scales((E, math.ceil(I / group_size), H)),
    }


def linear_weights(K: int, N: int, group_size: int, seed: int = 0, scale_std: float = SCALE_STD):
    g = _gen(seed)
    return packed_words((K // 8, N), g), group_scales((math.ceil(K / group_size), N), g, scale_std)


def activations(M: int, H: int, seed: int = 0) -> torch.Tensor:
    return torch.randn((M, H), generator=_gen(seed + 1000)).to(torch.bfloat16)


def router_weights(E: int, H: int, seed: int = 0, gate_std: float = 2.0) -> dict:
    """Router parameters of one MoE block (gemma.py:31-34) in bf16: router_scale
    [H] around 1, the gate nn.Linear weight [E, H] and expert_scale [E] around 1.
    gate_std 2 gives logits of roughly unit spread for N(0, 1) hidden states."""
    g = _gen(seed + 3000)
    return {
        "router_scale": (1.0 + 0.25 * torch.randn(H, generator=g)).to(torch.bfloat16),
        "gate": (gate_std * torch.randn((E, H), generator=g)).to(torch.bfloat16),
        "expert_scale": (1.0 + 0.1 * torch.randn(E, generator=g)).to(torch.bfloat16),
    }


def router_logits(M: int, E: int, seed: int = 0, verify_noise: float = 0.0) -> torch.Tensor:
    """i.i.d. N(0,1) logits, or (verify_noise > 0) a shared base N(0,1) row plus
    per-token N(0, verify_noise) noise, so that draft tokens overlap."""
    g = _gen(seed + 2000)
    if verify_noise > 0:
        base = torch.randn((1, E), generator=g)
        return base + torch.randn((M, E), generator=g) * verify_noise
    return torch.randn((M, E), generator=g)
