"""The two exact operand forms the fp16 MoE paths rest on, checked over every
input they can see (CPU, numpy; the kernels' own arithmetic is checked against
the oracle by the GPU tests).

* One-token kernel (moe_decode1.hip, F16): an fp16 value v splits into
  hi = v's float32 bits with the low 16 cleared (a bf16 value) and
  lo = bf16(v - hi); hi + lo == v exactly, for every finite fp16 value,
  subnormals included, so the two bf16 operand rows carry v without loss.
* 8-row kernel (moe_decode.hip, F16): the half whose high byte is 0x58 and
  low byte is 0x80 | q << 3 is 144 + q (the bytes of the bf16 16 + q operand
  under another high byte), and one fp16 add of -152 gives q - 8 exactly,
  for every code q; products of an fp16 value and q - 8 are exact in fp32.
"""
import numpy as np
import pytest


def _all_finite_fp16() -> np.ndarray:
    v = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16).view(np.float16)
    return v[np.isfinite(v)]


def _bf16_truncate(f32: np.ndarray) -> np.ndarray:
    return (f32.view(np.uint32) & np.uint32(0xFFFF0000)).view(np.float32)


def _bf16_round(f32: np.ndarray) -> np.ndarray:
    """Round to nearest even bf16 (the hardware's float -> bf16 conversion)."""
    b = f32.view(np.uint32).astype(np.uint64)
    r = ((b + 0x7FFF + ((b >> 16) & 1)) & 0xFFFF0000).astype(np.uint32)
    return r.view(np.float32)


def test_fp16_splits_exactly_into_bf16_hi_and_lo():
    v = _all_finite_fp16()
    f = v.astype(np.float32)
    hi = _bf16_truncate(f)
    lo = _bf16_round((f - hi).astype(np.float32))
    # f - hi is exact in float32 and already a bf16 value: the rounding keeps it
    assert np.array_equal((f - hi).astype(np.float32), lo)
    assert np.array_equal((hi.astype(np.float64) + lo.astype(np.float64)), f.astype(np.float64))
    # lo has at most 3 significant bits (fp16 keeps 11, hi takes the leading 8)
    nz = lo != 0
    mant = (lo[nz].view(np.uint32) >> 16) & 0x7F
    assert np.all((mant & 0x0F) == 0)
    # the split is not the identity: lo is in use for most values
    assert nz.mean() > 0.8


@pytest.mark.parametrize("q", range(16))
def test_int4_code_as_exact_fp16_q_minus_8(q):
    half_bits = np.array([(0x58 << 8) | (0x80 | (q << 3))], dtype=np.uint16)
    h = half_bits.view(np.float16)[0]
    assert float(h) == 144.0 + q
    d = np.float16(h) + np.float16(-152.0)       # one fp16 add (v_pk_add_f16 per pair)
    assert d.dtype == np.float16 and float(d) == q - 8
    # the bf16 operand of the same bytes (high byte 0x41) is 16 + q
    bf = np.array([((0x41 << 8) | (0x80 | (q << 3))) << 16], dtype=np.uint32).view(np.float32)[0]
    assert float(bf) == 16.0 + q


def test_fp16_times_code_is_exact_in_float32():
    v = _all_finite_fp16().astype(np.float64)
    for c in range(-8, 8):
        p64 = v * c
        p32 = (v.astype(np.float32) * np.float32(c)).astype(np.float64)
        assert np.array_equal(p64, p32)
