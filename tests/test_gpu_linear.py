"""GPU parity of the W4A16 linear (marlin_w4a16) and the lm_head softcap epilogue."""
import numpy as np
import pytest
import torch

import gemmainfer_csrc
from gemmainfer_amd import ops, synth
from oracle import moe_oracle as O
from tests.helpers import assert_bf16_close, np64, record_parity

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.mark.parametrize("m,k,n,gs", [
    (1, 2816, 2816, 128),    # BASELINE config 0 shape
    (5, 2816, 2112, 64),     # reference sanitizer test shape (M=5)
    (16, 2816, 2112, 64),    # M > 8 (reference's coalesced path)
    (8, 256, 1000, 64),      # test-small lm_head (vocab 1000)
    (3, 704, 2816, 128),     # ragged K groups (ceil), like the MoE down projection
    (2, 64, 4, 8),           # tiny
])
def test_w4a16_linear(m, k, n, gs):
    B, S = synth.linear_weights(k, n, gs, seed=m + n)
    A = synth.activations(m, k, seed=k)
    C = torch.empty(m, n, dtype=torch.bfloat16, device=DEV)
    gemmainfer_csrc.marlin_w4a16(A.to(DEV), B.to(DEV), S.to(DEV), C, gs)
    ref = O.w4a16_linear(np64(A), B.numpy(), np64(S), gs)
    stats = assert_bf16_close(C, ref, f"w4a16 m={m} k={k} n={n} gs={gs}")
    if (m, k, n, gs) == (1, 2816, 2816, 128):
        record_parity("cfg0_linear", stats)


@pytest.mark.parametrize("m,k,n,gs", [
    (1, 2816, 1028, 96),   # N not a multiple of the 16-column tile; 12 packed rows per group
    (2, 8000, 1024, 8000), # one group over all of K (1000 packed rows, the largest step count)
    (1, 520, 2048, 40),    # 65 packed rows: most of the second step past K; 5 rows per group
    (2, 256, 1036, 8),     # one packed row per group
])
def test_w4a16_narrow_path_odd_shapes(m, k, n, gs):
    """One and two rows at N >= 1024 take the 16-column narrow kernel: rows past
    K, columns past N and group sizes that are not a power of two."""
    B, S = synth.linear_weights(k, n, gs, seed=m + 3 * n)
    A = synth.activations(m, k, seed=k + 1)
    C = torch.empty(m, n, dtype=torch.bfloat16, device=DEV)
    gemmainfer_csrc.marlin_w4a16(A.to(DEV), B.to(DEV), S.to(DEV), C, gs)
    ref = O.w4a16_linear(np64(A), B.numpy(), np64(S), gs)
    assert_bf16_close(C, ref, f"narrow m={m} k={k} n={n} gs={gs}")


def test_w4a16_reference_floor_groups_drop_tail():
    """A scales tensor with K//gs groups drops rows past the last group, like
    the reference kernel (marlin.cu:128)."""
    k, n, gs = 704, 256, 128
    B, S = synth.linear_weights(k, n, gs, seed=3)
    S = S[: k // gs].contiguous()
    A = synth.activations(2, k, seed=4)
    C = torch.empty(2, n, dtype=torch.bfloat16, device=DEV)
    ops.marlin_w4a16(A.to(DEV), B.to(DEV), S.to(DEV), C, gs)
    ref = O.w4a16_linear(np64(A), B.numpy(), np64(S), gs)
    assert_bf16_close(C, ref, "floor groups")


def test_lm_head_softcap_column_subset():
    """BASELINE config 4 shape (M=6, K=2816, N=262144, gs=128): every output is
    computed on the GPU; the float64 oracle checks 2048 random columns."""
    m, k, n, gs = 6, 2816, 262144, 128
    g = torch.Generator(device=DEV)
    g.manual_seed(4)
    B = torch.randint(-(2 ** 31), 2 ** 31, (k // 8, n), generator=g, device=DEV,
                      dtype=torch.int64).to(torch.int32)
    S = (torch.randn((k // gs, n), generator=g, device=DEV).abs() * 0.02).to(torch.bfloat16)
    A = synth.activations(m, k, seed=6).to(DEV)
    C = ops.w4a16_linear(A, B, S, gs, softcap=30.0)
    cols = torch.randperm(n, generator=torch.Generator().manual_seed(0))[:2048].sort().values
    Bs, Ss = B[:, cols.to(DEV)].cpu(), S[:, cols.to(DEV)].cpu()
    ref = O.softcap(O.w4a16_linear(np64(A), Bs.numpy(), np64(Ss), gs), 30.0)
    stats = assert_bf16_close(C[:, cols.to(DEV)], ref, "lm_head subset")
    record_parity("cfg4_lm_head", stats, columns_checked=len(cols))
    # size-independent property: softcap bounds every logit by the cap
    assert float(C.float().abs().max()) <= 30.0


@pytest.mark.parametrize("m,gs,floor_groups,cap,n", [
    (3, 128, False, None, 65536),   # the wide-N matrix-core path
    (6, 64, False, 30.0, 65536),    # two k blocks per group, softcap
    (16, 128, False, None, 65536),  # a full 16-row operand
    (7, 128, True, None, 65536),    # floor-size scales: rows past the last group dropped
    (1, 128, False, 30.0, 65536),   # one row (zero operand rows) on the wide-N matrix-core path
    (1, 128, False, 30.0, 16384),   # one row: the 16-column narrow path with the softcap epilogue
    (2, 64, True, None, 16384),     # two rows, floor-size scales on the narrow path
])
def test_w4a16_matrix_core_path(m, gs, floor_groups, cap, n):
    """N >= 65536 runs the wide matrix-core kernel (any M <= 16); 1-2 rows at
    narrower N the 16-column narrow kernel: checked against the float64 oracle
    on 1024 random columns."""
    k = 2816 if not floor_groups else 2880
    g = torch.Generator(device=DEV)
    g.manual_seed(m * 7 + gs)
    B = torch.randint(-(2 ** 31), 2 ** 31, (k // 8, n), generator=g, device=DEV,
                      dtype=torch.int64).to(torch.int32)
    n_groups = k // gs if floor_groups else -(-k // gs)
    S = (torch.randn((n_groups, n), generator=g, device=DEV).abs() * 0.02).to(torch.bfloat16)
    A = synth.activations(m, k, seed=m).to(DEV)
    C = ops.w4a16_linear(A, B, S, gs, softcap=cap) if cap else ops.w4a16_linear(A, B, S, gs)
    cols = torch.randperm(n, generator=torch.Generator().manual_seed(m))[:1024].sort().values
    Bs, Ss = B[:, cols.to(DEV)].cpu(), S[:, cols.to(DEV)].cpu()
    ref = O.w4a16_linear(np64(A), Bs.numpy(), np64(Ss), gs)
    if cap:
        ref = O.softcap(ref, cap)
    assert_bf16_close(C[:, cols.to(DEV)], ref, f"matrix-core m={m} gs={gs} floor={floor_groups}")


def test_companions_match_cpu_semantics():
    x = torch.randn(3, 2816).to(torch.bfloat16)
    w = torch.randn(2816).to(torch.bfloat16)
    for unit in (False, True):
        out = torch.empty(3, 2816, dtype=torch.bfloat16, device=DEV)
        gemmainfer_csrc.rmsnorm(x.to(DEV), w.to(DEV), out, 1e-6, unit)
        ref_out = torch.empty_like(x)
        gemmainfer_csrc.rmsnorm(x, w, ref_out, 1e-6, unit)
        torch.testing.assert_close(out.cpu().float(), ref_out.float(), rtol=1e-2, atol=1e-2)
    logits = (torch.randn(1, 262144) * 40).to(torch.bfloat16)
    g = logits.to(DEV)
    gemmainfer_csrc.softcapping(g, 30.0)
    c = logits.clone()
    gemmainfer_csrc.softcapping(c, 30.0)
    torch.testing.assert_close(g.cpu().float(), c.float(), rtol=1e-2, atol=1e-2)
    q = torch.randn(2, 4, 5, 64).to(torch.bfloat16)
    k = torch.randn(2, 2, 5, 64).to(torch.bfloat16)
    pos = torch.arange(5).unsqueeze(0).expand(2, -1).contiguous()
    inv = 1.0 / (10000 ** (torch.arange(0, 64, 2).float() / 64))
    fr = torch.outer(torch.arange(16).float(), inv)
    emb = torch.cat((fr, fr), -1)
    cos, sin = emb.cos().to(torch.bfloat16), emb.sin().to(torch.bfloat16)
    qd, kd = q.to(DEV), k.to(DEV)
    gemmainfer_csrc.fused_rope_inplace(qd, kd, cos.to(DEV), sin.to(DEV), pos.to(DEV))
    qc, kc = q.clone(), k.clone()
    gemmainfer_csrc.fused_rope_inplace(qc, kc, cos, sin, pos)
    torch.testing.assert_close(qd.cpu().float(), qc.float(), rtol=2e-2, atol=2e-2)
    torch.testing.assert_close(kd.cpu().float(), kc.float(), rtol=2e-2, atol=2e-2)


@pytest.mark.parametrize("name", ["linear_m1_k256_n96_gs64", "linear_m5_k512_n128_gs128",
                                  "linear_m3_k2816_n64_gs128"])
def test_w4a16_matches_reference_golden(name):
    """Inputs/outputs produced by the reference's own CPU fallback (pybind.cpp:46-85)."""
    from pathlib import Path
    g = dict(np.load(Path(__file__).resolve().parent / "golden" / f"{name}.npz"))
    bf = lambda a: torch.from_numpy(a.view(np.int16).copy()).view(torch.bfloat16)  # noqa: E731
    A, S = bf(g["A_bf16"]), bf(g["scales_bf16"])
    B = torch.from_numpy(g["B_packed"])
    gs = int(g["group_size"])
    C = torch.empty(A.shape[0], B.shape[1], dtype=torch.bfloat16, device=DEV)
    gemmainfer_csrc.marlin_w4a16(A.to(DEV), B.to(DEV), S.to(DEV), C, gs)
    ref = O.bf16_bits_to_f64(g["C_bf16"])
    st = O.error_stats(np64(C), ref)
    assert st["rel_l2"] < 4e-3, st
    assert np.all(np.abs(np64(C) - ref) <= 2.0 ** -6 * np.abs(ref) + 1e-2), st
