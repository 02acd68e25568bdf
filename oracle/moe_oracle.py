"""numpy restatement of GemmaInfer's Token-Union W4A16 MoE path (TEST INFRASTRUCTURE).

Arithmetic is float64; values are rounded to bf16 exactly where the reference
rounds them (the bf16 activation store of the gate_up kernel, the cast of the
routing weights to the activation dtype, the bf16 output).  Every function
cites the reference file:line it restates (paths relative to the reference
repository root).

Pinning (what checks this restatement, see tests/test_oracle.py):

  bf16_round            exhaustive-ish: torch's own float32->bfloat16 cast on
                        ~10^6 values incl. ties, subnormals, inf/nan.
  round_to              torch's own float32->float16 cast (fp16) and the
                        float32 cast (fp32) on the same values; bf16 = bf16_round.
  unpack_int4/dequant   exhaustive over 16 nibble values x 8 positions x scale
                        sign; packer round trip (pack_int4); reference C++
                        fallback ``cpu_marlin_w4a16`` from oracle/_ref.
  w4a16_linear          brute-force scalar loop on tiny shapes; integer special
                        case (scale=1, q=8+v -> exact integer matmul);
                        reference C++ fallback from oracle/_ref at gs=64 and
                        gs=128 (K % gs == 0).
  gelu_tanh / softcap   torch.nn.functional.gelu(approximate='tanh') and
                        torch.tanh (the library routines the reference calls).
  route_topk_softmax    torch.topk + torch.softmax (the reference's own calls,
                        gemma.py:77-80) on tie-free fp32 logits; invariants
                        (weights sum to 1 with expert_scale=1, sortedness).
  token_union_align     hand-written known-answer cases (duplicates across and
                        within tokens, invalid ids, U=1, U=S, M=1/7/8/9) and a
                        brute-force restatement of the reference's O(S^2) scan.
  router_logits         norm step against the reference C++ fallback
                        ``cpu_gemma_rmsnorm`` (no weight) from oracle/_ref; the
                        scale and product steps against torch's own bf16
                        elementwise ops (the statements of gemma.py:75); the
                        gate against torch.nn.functional.linear in bf16;
                        closed forms (constant rows, identity gate).
  gated_mlp_act         the torch statements (F.gelu approximate='tanh' and the
                        product on bf16 tensors) on the same bf16 linear outputs.
  from_compressed       scalar brute force over the compressed-tensors layout
                        (nibble i of word [n][j] is k = 8j + i); round trip
                        through the transposed writer.
  fused_batched_moe     reference C++ fallback ``cpu_fused_batched_moe`` from
                        oracle/_ref (gs=64, all groups full); brute force on tiny
                        shapes; all-zero scales -> zero output; linearity in the
                        routing weights; chunked == unchunked.

No function is "parity unpinned"; the bf16 *atomic* accumulation order of the
reference CUDA kernel (marlin.cu:583) is non-deterministic and is not restated:
this oracle combines in float64 and rounds once.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np

# Zero point of the symmetric int4 code: w = (q - 8) * scale
# (quant.py:38 packs round(w/s)+8; marlin.cu:76 / quant.py:71 subtract 8).
ZERO_POINT = 8
GELU_C = math.sqrt(2.0 / math.pi)  # 0.7978845608..., marlin.cu:9
GELU_A = 0.044715                  # marlin.cu:9

_BF16_MIN_NORMAL = 2.0 ** -126
_BF16_SUBNORMAL_STEP = 2.0 ** -133
_BF16_MAX = float(np.float32(3.3895313892515355e38))


# --------------------------------------------------------------------------
# bf16 helpers
# --------------------------------------------------------------------------
def bf16_round(a) -> np.ndarray:
    """Round float64 values to the nearest bf16 (ties to even), returned as float64.

    Rounds the exact float64 value once (no detour through float32), which is
    what a correctly rounded fp32->bf16 cast does for float32 inputs.
    """
    x = np.asarray(a, dtype=np.float64)
    out = np.empty_like(x)
    finite = np.isfinite(x)
    out[~finite] = x[~finite]
    xf = x[finite]
    ax = np.abs(xf)
    res = np.empty_like(xf)
    small = ax < _BF16_MIN_NORMAL
    res[small] = np.rint(xf[small] / _BF16_SUBNORMAL_STEP) * _BF16_SUBNORMAL_STEP
    big = ~small
    m, e = np.frexp(xf[big])  # xf = m * 2**e, 0.5 <= |m| < 1
    res[big] = np.ldexp(np.rint(m * 256.0), e - 8)
    over = np.abs(res) > _BF16_MAX
    res[over] = np.copysign(np.inf, res[over])
    out[finite] = res
    return out


def round_to(a, dtype: str = "bf16") -> np.ndarray:
    """Round float64 values to the activation dtype of a call: "bf16"
    (bf16_round), "fp16" (nearest IEEE half, ties to even: numpy's correctly
    rounded float64 -> float16 cast) or "fp32" (float64 -> float32 cast);
    returned as float64.  The reference dispatches these three dtypes
    (marlin.cu:694-700, :764-842) and rounds to the one of x at the same
    points for each."""
    x = np.asarray(a, dtype=np.float64)
    if dtype == "bf16":
        return bf16_round(x)
    if dtype == "fp16":
        return x.astype(np.float16).astype(np.float64)
    if dtype == "fp32":
        return x.astype(np.float32).astype(np.float64)
    raise ValueError(f"dtype {dtype!r}")


def bf16_bits_to_f64(bits) -> np.ndarray:
    """Interpret uint16 bf16 bit patterns as float64 values."""
    b = np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16
    return b.view(np.float32).astype(np.float64)


def f64_to_bf16_bits(a) -> np.ndarray:
    """bf16 bit patterns (uint16) of bf16_round(a)."""
    r = bf16_round(a).astype(np.float32)
    return (r.view(np.uint32) >> 16).astype(np.uint16)


# --------------------------------------------------------------------------
# int4 packing (quant.py:12-46) and dequantisation (quant.py:67-74, marlin.cu:69-91)
# --------------------------------------------------------------------------
def unpack_int4(packed) -> np.ndarray:
    """[Kp, N] int32 words -> [8*Kp, N] codes 0..15.

    Nibble i (bits 4i..4i+3) of word [pk, n] is the code of row k = 8*pk + i
    (packer quant.py:41-43; readers quant.py:70-71, marlin.cu:75, pybind.cpp:76).
    """
    p = np.asarray(packed).astype(np.int64) & 0xFFFFFFFF
    kp, n = p.shape
    shifts = (4 * np.arange(8, dtype=np.int64))[None, :, None]
    q = (p[:, None, :] >> shifts) & 0xF
    return q.reshape(kp * 8, n).astype(np.int64)


def pack_int4(q) -> np.ndarray:
    """[K, N] codes 0..15 -> [K/8, N] int32 words (inverse of unpack_int4; quant.py:41-44)."""
    q = np.asarray(q, dtype=np.int64)
    k, n = q.shape
    assert k % 8 == 0
    q = q.reshape(k // 8, 8, n)
    words = np.zeros((k // 8, n), dtype=np.int64)
    for i in range(8):
        words |= (q[:, i, :] & 0xF) << (4 * i)
    return words.astype(np.uint32).view(np.int32)


def quantize_w4(weight, group_size) -> tuple[np.ndarray, np.ndarray]:
    """Symmetric group-wise int4 quantiser restating quant.py:12-46.

    weight [N, K] (float) -> (packed int32 [K/8, N], scales float64 [K/gs, N]
    already rounded to bf16).  scale = max|w| / 7 over each group of ``gs`` k
    (clamped at 1e-5, quant.py:33-34), code = clamp(round_half_even(w/s) + 8, 0, 15)
    (quant.py:38; torch.round rounds half to even, as np.rint does).
    """
    w = np.asarray(weight, dtype=np.float64)
    n, k = w.shape
    assert k % group_size == 0 and k % 8 == 0
    wt = w.T.reshape(k // group_size, group_size, n)
    s = bf16_round(np.maximum(np.abs(wt).max(axis=1), 1e-5) / 7.0)
    q = np.clip(np.rint(wt / s[:, None, :]) + ZERO_POINT, 0, 15).reshape(k, n)
    return pack_int4(q), s


def from_compressed(weight_packed, weight_scale):
    """compressed-tensors W4A16 linear (``weight_packed`` int32 [N, K/8],
    ``weight_scale`` [N, groups]) -> (packed [K/8, N], scales [groups, N]) as
    this oracle and the kernels take them: the ``t.t()`` of
    weights.py:100-159."""
    return (np.ascontiguousarray(np.asarray(weight_packed).T),
            np.ascontiguousarray(np.asarray(weight_scale, dtype=np.float64).T))


def dequant(packed, scales, group_size) -> np.ndarray:
    """[Kp, N] words + [G, N] scales -> float64 weights [K, N], K = 8*Kp.

    w[k, n] = (q[k, n] - 8) * scales[k // gs, n].  Rows k >= G*gs (a scales
    tensor with fewer groups than ceil(K/gs)) contribute zero: this is how the
    reference CUDA kernel behaves, since it loops only over the groups it
    counts (marlin.cu:357,371 gate_up; :526,538 down).
    """
    q = unpack_int4(packed).astype(np.float64) - ZERO_POINT
    s = np.asarray(scales, dtype=np.float64)
    k = q.shape[0]
    g = np.arange(k) // group_size
    valid = g < s.shape[0]
    w = np.zeros_like(q)
    w[valid] = q[valid] * s[g[valid]]
    return w


def w4a16_linear(a, packed, scales, group_size) -> np.ndarray:
    """Exact (float64) C = A @ dequant(B); the W4A16 linear of marlin.cu:704-856
    and pybind.cpp:46-85 before the output cast."""
    a = np.asarray(a, dtype=np.float64)
    return a @ dequant(packed, scales, group_size)


def w4a16_linear_bf16(a, packed, scales, group_size, softcap_cap=None) -> np.ndarray:
    """bf16 output of the W4A16 linear, optionally followed by the final logit
    softcap cap*tanh(y/cap) (gemma.py:356-357 -> softcapping.cu:16-17)."""
    y = w4a16_linear(a, packed, scales, group_size)
    if softcap_cap is not None:
        y = softcap(y, softcap_cap)
    return bf16_round(y)


# --------------------------------------------------------------------------
# elementwise functions
# --------------------------------------------------------------------------
def gelu_tanh(x) -> np.ndarray:
    """0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3)))  (marlin.cu:7-11;
    F.gelu(approximate='tanh') at gemma.py:137, pybind.cpp:237)."""
    x = np.asarray(x, dtype=np.float64)
    return 0.5 * x * (1.0 + np.tanh(GELU_C * (x + GELU_A * x * x * x)))


def gated_mlp_act(a, gate, up, group_size) -> np.ndarray:
    """GemmaMLP's first half on bf16 tensors (activations.py:26-28):
    bf16(bf16(gelu_tanh(bf16(a @ Wg))) * bf16(a @ Wu)); gate/up = (packed, scales)."""
    g = bf16_round(w4a16_linear(a, *gate, group_size))
    u = bf16_round(w4a16_linear(a, *up, group_size))
    return bf16_round(bf16_round(gelu_tanh(g)) * u)


def softcap(y, cap) -> np.ndarray:
    """cap * tanh(y / cap)  (softcapping.cu:16-17, pybind.cpp:134)."""
    y = np.asarray(y, dtype=np.float64)
    return cap * np.tanh(y / cap)


# --------------------------------------------------------------------------
# router front-end (gemma.py:75-76)
# --------------------------------------------------------------------------
def rmsnorm_noscale_bf16(x, eps):
    """GemmaRMSNorm(with_scale=False) on bf16 rows (norm.py:28-40 ->
    rmsnorm.cu:16-73 on the GPU, pybind.cpp:87-103 on the CPU): fp32 products
    x * rsqrt(mean(x^2) + eps), rounded to bf16.  The mean is taken in float64
    and rsqrt rounded to fp32 once; the product is formed in fp32 as the
    reference does, then rounded to bf16."""
    xf = np.asarray(x, dtype=np.float64)
    ms = np.mean(xf * xf, axis=-1, keepdims=True)
    r = (1.0 / np.sqrt(ms + np.float64(np.float32(eps)))).astype(np.float32)
    return bf16_round((xf.astype(np.float32) * r).astype(np.float64))


def router_scale_bf16(router_scale, hidden):
    """``router_scale * (hidden_size ** -0.5)`` (gemma.py:75): a bf16 parameter
    times a Python float, computed in fp32 with the scalar cast to fp32, bf16
    result.  router_scale None = the parameter's initial ones (gemma.py:32)."""
    c = np.float32(hidden ** -0.5)
    rs = (np.ones(hidden, dtype=np.float32) if router_scale is None
          else np.asarray(router_scale, dtype=np.float64).astype(np.float32))
    return bf16_round((rs * c).astype(np.float64))


def router_logits(x, router_scale, gate_w, eps=1e-6):
    """Router front-end of GemmaBatchedMoE.forward (gemma.py:75-76):

        x_normed = bf16(norm(x) * bf16(router_scale * H^-0.5))   (bf16 * bf16)
        logits   = bf16(x_normed @ gate_w.T)                      (nn.Linear, no bias)

    The dot products are exact (float64) and rounded once; the reference's
    fp32 accumulation differs from them by far less than one bf16 ulp except
    next to a rounding boundary.  Returns (logits float64 [M, E],
    x_normed float64 [M, H])."""
    xf = np.asarray(x, dtype=np.float64)
    n = rmsnorm_noscale_bf16(xf, eps)
    s = router_scale_bf16(router_scale, xf.shape[-1])
    xr = bf16_round(n * s)
    g = np.asarray(gate_w, dtype=np.float64)
    return bf16_round(xr @ g.T), xr


# --------------------------------------------------------------------------
# routing (gemma.py:77-80)
# --------------------------------------------------------------------------
def route_topk_softmax(logits, top_k, expert_scale=None):
    """Top-k over experts, softmax over the k selected logits, times expert_scale.

    Restates gemma.py:77-80: ``torch.topk(router_logits, k)`` (descending),
    ``F.softmax(top, dtype=float32)``, ``* expert_scale[idx]``, ``.type_as(x)``.
    Order: value descending, ties broken by the lower expert index; NaN ranks
    above every number (torch.topk's convention).

    Returns (idx int32 [M, k], weights float64 [M, k] before the dtype cast,
    weights rounded to bf16 as float64 [M, k]).
    """
    l = np.asarray(logits, dtype=np.float64)
    m, e = l.shape
    assert 1 <= top_k <= e
    idx = np.empty((m, top_k), dtype=np.int32)
    for t in range(m):
        row = l[t]
        nan = np.isnan(row)
        key_val = np.where(nan, 0.0, row)
        order = np.lexsort((np.arange(e), -key_val, ~nan))
        idx[t] = order[:top_k]
    top = np.take_along_axis(l, idx.astype(np.int64), axis=1)
    mx = top.max(axis=1, keepdims=True)
    ex = np.exp(top - mx)
    p = ex / ex.sum(axis=1, keepdims=True)
    if expert_scale is not None:
        p = p * np.asarray(expert_scale, dtype=np.float64)[idx]
    return idx, p, bf16_round(p)


# --------------------------------------------------------------------------
# Token-Union deduplication (marlin.cu:285-335 gate_up, :453-505 down)
# --------------------------------------------------------------------------
@dataclass
class Alignment:
    unique_experts: np.ndarray   # int32 [U], first-occurrence slot order
    slot_to_unique: np.ndarray   # int32 [S], -1 for an invalid expert id
    offsets: np.ndarray          # int32 [U+1], CSR over unique experts
    slots: np.ndarray            # int32 [offsets[U]], slots of each expert, ascending

    @property
    def num_unique(self) -> int:
        return int(self.unique_experts.shape[0])


def token_union_align(idx, num_experts) -> Alignment:
    """The reference kernel's implicit dedup, materialised.

    Block u of marlin.cu:285-335 scans the flattened slots s = 0..S-1, skips
    ids outside [0, E) (:304), and picks the u-th id whose first occurrence is
    at s (:305-318).  It then gathers every slot holding that id in ascending
    s (:323-330).  The reference caps that gather at MAX_MATCH (:325) and at
    MAX_SLOTS=128 slots (:300); this restatement is uncapped -- the reference's
    own CPU path (pybind.cpp:219-244) processes every slot.
    """
    flat = np.asarray(idx).reshape(-1).astype(np.int64)
    s_total = flat.shape[0]
    pos: dict[int, int] = {}
    unique: list[int] = []
    s2u = np.full(s_total, -1, dtype=np.int32)
    for s in range(s_total):
        e = int(flat[s])
        if e < 0 or e >= num_experts:
            continue
        if e not in pos:
            pos[e] = len(unique)
            unique.append(e)
        s2u[s] = pos[e]
    n_u = len(unique)
    counts = np.bincount(s2u[s2u >= 0], minlength=n_u) if n_u else np.zeros(0, np.int64)
    offsets = np.zeros(n_u + 1, dtype=np.int32)
    offsets[1:] = np.cumsum(counts)
    slots = np.nonzero(s2u >= 0)[0]
    slots = slots[np.argsort(s2u[slots], kind="stable")].astype(np.int32)
    return Alignment(np.asarray(unique, dtype=np.int32), s2u, offsets, slots)


# --------------------------------------------------------------------------
# fused MoE (marlin.cu:262-702; pybind.cpp:198-245; gemma.py:82-113)
# --------------------------------------------------------------------------
def expert_forward(x_rows, gu_packed_e, gu_scales_e, d_packed_e, d_scales_e,
                   group_size, act_round=True, dtype="bf16"):
    """One expert on a block of rows: gate_up -> gelu_tanh(gate)*up -> down.

    gate/up are float64 sums of x*(q-8)*s (marlin.cu:371-416); the activation
    is rounded to the activation dtype (bf16 by default) as the reference
    stores it (``static_cast<scalar_t>``, marlin.cu:421-423) when
    ``act_round``; down is a float64 sum over I (marlin.cu:538-576).
    Returns (act [n, I], y [n, H]) float64.
    """
    wgu = dequant(gu_packed_e, gu_scales_e, group_size)
    n_inter = wgu.shape[1] // 2
    gu = np.asarray(x_rows, dtype=np.float64) @ wgu
    act = gelu_tanh(gu[:, :n_inter]) * gu[:, n_inter:]
    if act_round:
        act = round_to(act, dtype)
    y = act @ dequant(d_packed_e, d_scales_e, group_size)
    return act, y


def fused_batched_moe(x, gu_packed, gu_scales, d_packed, d_scales, idx, w,
                      out_in, group_size, act_round=True, dtype="bf16"):
    """out = out_in + sum over slots of T(w[slot]) * expert(x[token])[slot],
    T the activation dtype ("bf16" default, "fp16", "fp32").

    Semantics of ``gemmainfer_csrc.fused_batched_moe`` (pybind.cpp:247-271 ->
    marlin.cu:612-702): top_k = numel(idx)/M (:628-629); routing weights are
    cast to the activation dtype (:634-636); slots whose id is outside [0, E)
    contribute nothing (:304,473); the result is *added* to ``out``
    (:583, caller zeroes it at gemma.py:82).  The combine here is float64 in
    slot order; the caller rounds once (the reference adds bf16-rounded terms
    with atomics in an unspecified order, :583).

    Returns (out float64 [M, H] before rounding, Alignment).
    """
    x = np.asarray(x, dtype=np.float64)
    m = x.shape[0]
    flat_idx = np.asarray(idx).reshape(-1)
    s_total = flat_idx.shape[0]
    assert s_total % m == 0
    top_k = s_total // m
    w_used = round_to(np.asarray(w, dtype=np.float64).reshape(-1), dtype)
    num_experts = np.asarray(gu_packed).shape[0]
    al = token_union_align(flat_idx, num_experts)
    contrib = np.zeros((s_total, x.shape[1]), dtype=np.float64)
    for u in range(al.num_unique):
        e = int(al.unique_experts[u])
        sl = al.slots[al.offsets[u]:al.offsets[u + 1]]
        toks = sl // top_k
        _, y = expert_forward(x[toks], gu_packed[e], gu_scales[e], d_packed[e],
                              d_scales[e], group_size, act_round, dtype)
        contrib[sl] = y * w_used[sl][:, None]
    out = np.asarray(out_in, dtype=np.float64).copy()
    for t in range(m):
        for k in range(top_k):
            out[t] += contrib[t * top_k + k]
    return out, al


def chunked_batched_moe(x, gu_packed, gu_scales, d_packed, d_scales, idx, w,
                        out_in, group_size, chunk=8, act_round=True):
    """gemma.py:99-112: the M>8 path issues one fused call per 8-row slice."""
    x = np.asarray(x, dtype=np.float64)
    idx = np.asarray(idx)
    w = np.asarray(w, dtype=np.float64)
    out = np.asarray(out_in, dtype=np.float64).copy()
    for start in range(0, x.shape[0], chunk):
        end = min(start + chunk, x.shape[0])
        out[start:end], _ = fused_batched_moe(
            x[start:end], gu_packed, gu_scales, d_packed, d_scales,
            idx[start:end], w[start:end], out[start:end], group_size, act_round)
    return out


def moe_layer_from_logits(x, logits, gu_packed, gu_scales, d_packed, d_scales,
                          top_k, group_size, expert_scale=None, act_round=True):
    """Router (gemma.py:77-80) followed by the fused MoE into a zeroed output
    (gemma.py:82-98).  Returns (out float64, idx, w_bf16, Alignment)."""
    idx, _, w_bf16 = route_topk_softmax(logits, top_k, expert_scale)
    x = np.asarray(x, dtype=np.float64)
    out, al = fused_batched_moe(x, gu_packed, gu_scales, d_packed, d_scales,
                                idx, w_bf16, np.zeros_like(x), group_size, act_round)
    return out, idx, w_bf16, al


# --------------------------------------------------------------------------
# comparison helpers used by the tests
# --------------------------------------------------------------------------
def error_stats(got, ref) -> dict:
    """max-abs, relative L2 and max-abs/RMS of ``got`` against float64 ``ref``."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    diff = got - ref
    rms = float(np.sqrt(np.mean(ref * ref))) if ref.size else 0.0
    l2 = float(np.linalg.norm(ref.ravel()))
    return {
        "max_abs": float(np.max(np.abs(diff))) if diff.size else 0.0,
        "rel_l2": float(np.linalg.norm(diff.ravel()) / l2) if l2 > 0 else float(np.linalg.norm(diff.ravel())),
        "max_abs_over_rms": (float(np.max(np.abs(diff))) / rms) if rms > 0 else 0.0,
        "ref_rms": rms,
        "ref_max": float(np.max(np.abs(ref))) if ref.size else 0.0,
    }
