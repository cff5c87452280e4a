"""The benchmark configurations at their full sizes on gfx950, checked on sampled rows and heads against float64
(and exact integer) arithmetic: the bf16 8192^3 GEMM, fp8 e4m3 8192^3 and the small-M shapes, W8A8 int8 with
N=14336 K=4096, and causal bf16 flash attention B=4 H=32 S=4096 D=128. Every output element of a sampled row is
checked; the sampled rows include the first and last tile rows and the last row of the output."""

import math

import numpy as np
import pytest

from krn_amd import Blocks, T
from oracle.numerics import bf16_values, bf16_words, e4m3_decode, e4m3_encode
from tests.helpers import assert_agrees
from tests.kernels import tile_programs as programs

pytestmark = pytest.mark.gpu


def sample_rows(m: int, rng: np.random.Generator, count: int = 24) -> np.ndarray:
    picks = {0, 1, min(255, m - 1), m - 1} | set(rng.integers(0, m, count).tolist())
    return np.array(sorted(p for p in picks if p < m))


def test_bf16_gemm_8192_cubed(device):
    n = 8192
    rng = np.random.default_rng(0)
    aw = bf16_words(rng.standard_normal((n, n), dtype=np.float32))
    bw = bf16_words(rng.standard_normal((n, n), dtype=np.float32))
    c = device.empty(T.bf16, n, n)
    programs.gemm_nt[programs.Tiling(bm=256, bn=256, bk=64)](device.to_device(aw, T.bf16), device.to_device(bw, T.bf16), c)
    got = c.to_host()
    rows = sample_rows(n, rng)
    a, b = bf16_values(aw[rows]), bf16_values(bw)
    assert_agrees(bf16_values(got[rows]), a, b.T, n, "bf16")
    # the configuration's own criterion: relative error 1e-2 against an fp32-accumulated reference
    reference = a.astype(np.float64) @ b.T.astype(np.float64)
    rel = np.linalg.norm(bf16_values(got[rows]) - reference) / np.linalg.norm(reference)
    assert rel < 1e-2, rel
    assert rel < 5e-3, rel  # the stated figure: the bf16 output rounding (about 1.1e-3 RMS) dominates


@pytest.mark.parametrize("m", [8192, 128, 16, 1])
def test_fp8_gemm_full_size(device, m):
    n = k = 8192
    rng = np.random.default_rng(81 + m)
    x, w = rng.standard_normal((m, k), dtype=np.float32), rng.standard_normal((n, k), dtype=np.float32)
    sx, sw = np.float32(np.abs(x).max() / 448), np.float32(np.abs(w).max() / 448)
    a, b = e4m3_encode(x / sx), e4m3_encode(w / sw)
    c = device.empty(T.bf16, m, n)
    programs.gemm_fp8[programs.Tiling(bm=256, bn=256, bk=128)](
        device.to_device(a, T.f8e4m3fn), device.to_device(b, T.f8e4m3fn), c, sx, sw)
    rows = sample_rows(m, rng)
    got = bf16_values(c.to_host()[rows]).astype(np.float64)
    da, db = e4m3_decode(a[rows]).astype(np.float64), e4m3_decode(b).astype(np.float64)
    scale = np.float64(np.float32(sx * sw))
    reference = (da @ db.T) * scale
    bound = 8 * 2.0**-24 * (k + 8) * (np.abs(da) @ np.abs(db).T) * scale + np.abs(reference) * 2.0**-8 * 1.01
    assert np.all(np.abs(got - reference) <= bound + 1e-30)
    # the stated relative error of this configuration against the decoded-operand product: the bf16 output rounding
    rel = np.linalg.norm(got - reference) / np.linalg.norm(reference)
    assert rel < 5e-3, rel


@pytest.mark.parametrize("m", [4096, 16])
def test_int8_gemm_full_size_is_bit_exact(device, m):
    n, k = 14336, 4096
    rng = np.random.default_rng(5 + m)
    a = rng.integers(-127, 128, (m, k), dtype=np.int8)
    w = rng.integers(-127, 128, (n, k), dtype=np.int8)
    sa = (rng.uniform(0.5, 1.5, (m, 1)) / 127).astype(np.float32)
    sw = (rng.uniform(0.5, 1.5, (1, n)) / 127).astype(np.float32)
    da, dw = device.to_device(a), device.to_device(w)
    acc = device.empty(T.i32, m, n)
    programs.gemm_i8_i32[programs.Tiling(bm=256, bn=256, bk=64)](da, dw, acc)
    out = device.empty(T.bf16, m, n)
    programs.gemm_w8a8[programs.Tiling(bm=256, bn=256, bk=64)](da, dw, device.to_device(sa), device.to_device(sw), out)
    rows = sample_rows(m, rng)
    # |sum| <= 4096 * 127^2 < 2^53: float64 BLAS is exact here
    exact = (a[rows].astype(np.float64) @ w.astype(np.float64).T).astype(np.int64)
    np.testing.assert_array_equal(acc.to_host()[rows], exact)
    dequant = (exact.astype(np.float32) * sa[rows]).astype(np.float32) * sw
    np.testing.assert_array_equal(out.to_host()[rows], bf16_words(dequant.astype(np.float32)))


def test_causal_bf16_flash_attention_b4_h32_s4096_d128(device):
    bh, s, d = 4 * 32, 4096, 128
    rng = np.random.default_rng(3)
    words = [bf16_words(rng.standard_normal((bh, s, d), dtype=np.float32)) for _ in range(3)]
    o = device.empty(T.bf16, bh, s, d)
    tiling = programs.Attention(bq=128, bk=64, d=d, causal=True)
    programs.flash_attention_bf16(tiling, *(device.to_device(w, T.bf16) for w in words), o,
                                  math.log2(math.e) / math.sqrt(d), launch=Blocks(s // 128, bh))
    got = o.to_host()
    # 16 heads spread over the batch and head range, first and last included
    heads = sorted({0, bh - 1} | set(np.linspace(1, bh - 2, 14).astype(int).tolist()))
    assert len(heads) == 16
    causal = np.tril(np.ones((s, s), bool))
    for head in heads:
        q, k, v = (bf16_values(w[head]).astype(np.float64) for w in words)
        scores = np.where(causal, q @ k.T / math.sqrt(d), -np.inf)
        p = np.exp(scores - scores.max(axis=-1, keepdims=True))
        want = (p / p.sum(axis=-1, keepdims=True)) @ v
        out = bf16_values(got[head]).astype(np.float64)
        np.testing.assert_allclose(out, want, atol=2e-2, err_msg=f"head {head}")
        # the stated relative error of this configuration: p and o each round once to bf16 (8 significant bits)
        rel = np.linalg.norm(out - want) / np.linalg.norm(want)
        assert rel < 1e-2, f"head {head}: relative error {rel}"


def test_f16_nn_matmul_example_8192_cubed(device):
    """krn's own GEMM example (reference examples/04_libraries/01_gemm_tiles.py:34-40: `b[ks, cols]`, b stored
    K x N) at the headline size: the NN product on the MFMA GEMM, sampled rows against float64."""
    n = 8192
    rng = np.random.default_rng(9)
    a = rng.uniform(-1, 1, (n, n)).astype(np.float16)
    b = rng.uniform(-1, 1, (n, n)).astype(np.float16)
    c = device.empty(T.f16, n, n)
    programs.matmul[programs.Tiling(bm=256, bn=256, bk=64)](device.to_device(a), device.to_device(b), c)
    rows = sample_rows(n, rng)
    got = c.to_host()[rows]
    assert_agrees(got.astype(np.float32), a[rows].astype(np.float32), b.astype(np.float32), n, "f16")
    reference = a[rows].astype(np.float64) @ b.astype(np.float64)
    rel = np.linalg.norm(got.astype(np.float64) - reference) / np.linalg.norm(reference)
    assert rel < 2e-3, rel
