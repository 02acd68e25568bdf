"""Shared test helpers: tolerance gate, tensor conversion and the parity record."""
from __future__ import annotations

import numpy as np
import torch

from oracle import moe_oracle as O

# Tolerance gate for bf16 outputs against the float64 oracle.
#   * rel-L2 <= 1e-2: the bound of BASELINE.json's north_star, literally.
#   * elementwise |got - ref| <= 2e-2 + 2^-7 |ref|: the north-star max-abs 2e-2
#     made scale-aware.  A literal max-abs of 2e-2 is below the bf16 spacing of
#     outputs this large (|out| reaches 50-85, spacing 0.25-0.5); 2^-7 |ref| is
#     two half-ulps of bf16.
REL_L2 = 1e-2
ATOL = 2e-2
RTOL = 2.0 ** -7


def np64(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy().astype(np.float64)


def assert_bf16_close(got: torch.Tensor, ref64: np.ndarray, what: str = "") -> dict:
    g = np64(got)
    stats = O.error_stats(g, ref64)
    bound = ATOL + RTOL * np.abs(ref64)
    bad = np.abs(g - ref64) > bound
    assert np.isfinite(g).all(), f"{what}: non-finite outputs"
    assert stats["rel_l2"] <= REL_L2, f"{what}: rel-L2 {stats['rel_l2']:.3e} > {REL_L2} ({stats})"
    assert not bad.any(), (
        f"{what}: {int(bad.sum())} elements outside {ATOL} + 2^-7|ref|; worst "
        f"{float(np.max(np.abs(g - ref64) - bound)):.3e} over bound ({stats})")
    return stats


def assert_close_rms(got: torch.Tensor, ref64: np.ndarray, what: str = "",
                     max_over_rms: float = 3e-2) -> dict:
    """The gate for inputs far outside a checkpoint's value range (the
    reference's sanitizer inputs: std-1 scales, packed words from
    randint(-1e5, 1e5)), whose outputs (RMS ~1e7) are sums of terms ~1e5 that
    cancel.  There the fp32 sums and a bf16 rounding flip of one activation
    (its float64 value within fp32 error of a rounding midpoint) move an output
    by amounts that scale with the terms, not with the output, so the
    elementwise 2e-2 + 2^-7|ref| bound does not apply.  Instead: rel-L2 <= 1e-2
    (literally) and max |got - ref| <= max_over_rms * RMS(ref)
    (the max-abs bound in units of the output's own size)."""
    g = np64(got)
    stats = O.error_stats(g, ref64)
    assert np.isfinite(g).all(), f"{what}: non-finite outputs"
    assert stats["rel_l2"] <= REL_L2, f"{what}: rel-L2 {stats['rel_l2']:.3e} > {REL_L2} ({stats})"
    assert stats["max_abs_over_rms"] <= max_over_rms, f"{what}: max-abs/RMS too large ({stats})"
    return stats


def bf16_ulp(v) -> np.ndarray:
    """Spacing of bf16 values at |v| (normal range; 2^-133 floor)."""
    _, e = np.frexp(np.maximum(np.abs(np.asarray(v, dtype=np.float64)), 2.0 ** -126))
    return np.ldexp(1.0, e - 8)


def assert_logits_close(got: torch.Tensor, ref64: np.ndarray, what: str = "",
                        min_exact: float = 0.97, abs_terms=None, k: int = 0) -> None:
    """Router logits: every element within one bf16 ulp of the oracle (the fp32
    sum order may move a value across a rounding boundary), and nearly all of
    them bit-identical.  With ``abs_terms`` (sum over k of |x_normed * gate|)
    and the length k of the sums, the classical bound on an fp32 sum in any
    order, k * 2^-24 * abs_terms, is added: a logit near zero whose terms
    cancel has a bf16 ulp smaller than that error."""
    g = np64(got)
    assert g.shape == ref64.shape, (what, g.shape, ref64.shape)
    diff = np.abs(g - ref64)
    bound = bf16_ulp(ref64)
    if abs_terms is not None:
        bound = bound + k * 2.0 ** -24 * np.asarray(abs_terms, dtype=np.float64)
    bad = diff > bound
    assert not bad.any(), f"{what}: {int(bad.sum())} logits more than one bf16 ulp off; max diff {diff.max():.3e}"
    exact = float(np.mean(g == ref64))
    assert exact >= min_exact, f"{what}: only {exact:.4f} of logits bit-identical"


def assert_dtype_close(got: torch.Tensor, ref64: np.ndarray, dtype: str, what: str = "") -> dict:
    """The tolerance gate for outputs in the activation dtype of a call.

    bf16: assert_bf16_close.  fp16: rel-L2 <= 1e-2 and every element within
    2e-2 + 2^-10 |ref| (the north-star max-abs plus one fp16 ulp; fp16 keeps 3
    more mantissa bits than bf16).  fp32 (nothing is rounded but the float32
    sums): rel-L2 <= 2e-5 and max |got - ref| <= 1e-4 * RMS(ref)."""
    if dtype == "bf16":
        return assert_bf16_close(got, ref64, what)
    g = np64(got)
    stats = O.error_stats(g, ref64)
    assert np.isfinite(g).all(), f"{what}: non-finite outputs"
    if dtype == "fp16":
        assert stats["rel_l2"] <= REL_L2, f"{what}: rel-L2 {stats['rel_l2']:.3e} ({stats})"
        bound = ATOL + 2.0 ** -10 * np.abs(ref64)
        bad = np.abs(g - ref64) > bound
        assert not bad.any(), f"{what}: {int(bad.sum())} elements outside 2e-2 + 2^-10|ref| ({stats})"
    elif dtype == "fp32":
        assert stats["rel_l2"] <= 2e-5, f"{what}: rel-L2 {stats['rel_l2']:.3e} ({stats})"
        assert stats["max_abs_over_rms"] <= 1e-4, f"{what}: max-abs/RMS too large ({stats})"
    else:
        raise ValueError(dtype)
    return stats


# Error statistics of the BASELINE configs' parity tests, by config name;
# tests/conftest.py writes them to the JSON file named by GI_PARITY_STATS
# at the end of the session (when that variable is set).
PARITY_RECORD: dict = {}


def record_parity(config: str, stats: dict, **extra) -> None:
    PARITY_RECORD[config] = {**{k: float(v) for k, v in stats.items()}, **extra}
