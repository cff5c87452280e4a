"""Products of tile programs that no hand-written kernel serves run on the matrix cores through the generic
lowering (reference src/krn/compiler/emit.py:924-955 `matrix_stage`, compiler/hip.py:70-97 `AMDMFMA.product`): a
partial-K GEMM, an int8 one (bit-exact), a GEMM on a grid larger than its output, and flash attention with head
dimension 32. `explain()` names the route and each product's instruction."""

import math

import numpy as np
import pytest

from krn_amd import Blocks, T
from krn_amd.compiler.capture import capture
from oracle import cbackend, emulate
from oracle.numerics import bf16_values, bf16_words
from tests.conftest import KERNELS
from tests.helpers import assert_agrees
from tests.kernels import tile_programs as programs

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("m,n,k,kk", [(64, 64, 96, 96), (100, 130, 200, 96), (128, 192, 256, 160)])
def test_partial_k_bf16_gemm_runs_on_mfma(device, m, n, k, kk):
    rng = np.random.default_rng(m + n + k)
    aw = bf16_words(rng.standard_normal((m, k)).astype(np.float32))
    bw = bf16_words(rng.standard_normal((n, k)).astype(np.float32))
    a, b = device.to_device(aw, T.bf16), device.to_device(bw, T.bf16)
    c = device.empty(T.f32, m, n)
    tiling = programs.PartialK(bm=64, bn=64, bk=32, kk=kk)
    launcher = programs.gemm_partial_k[tiling]
    explained = launcher.explain(a, b, c)
    assert explained["plan"] == "GenericPlan" and explained["products"] == ["mfma 16x16x32 bf16"]
    launcher(a, b, c)
    got = c.to_host()
    used = min(kk, k)
    assert_agrees(got, bf16_values(aw[:, :used]), bf16_values(bw[:, :used]).T, used, "f32")
    # the oracle C backend runs the same program (k-ordered fused multiply-adds): equal within the product bound
    want = np.zeros((m, n), np.float32)
    cbackend.run(capture(KERNELS, "gemm_partial_k", consts={"t": tiling.__dict__}), None, [aw, bw, want])
    bound = 16 * 2.0**-24 * (used + 8) * (np.abs(bf16_values(aw[:, :used])).astype(np.float64)
                                          @ np.abs(bf16_values(bw[:, :used])).T)
    assert np.all(np.abs(got.astype(np.float64) - want) <= bound)


def test_partial_k_int8_gemm_on_mfma_is_bit_exact(device):
    m, n, k, kk = 96, 160, 256, 192
    rng = np.random.default_rng(8)
    a = rng.integers(-127, 128, (m, k), dtype=np.int8)
    b = rng.integers(-127, 128, (n, k), dtype=np.int8)
    c = device.empty(T.i32, m, n)
    launcher = programs.gemm_i8_partial_k[programs.PartialK(bm=64, bn=64, bk=64, kk=kk)]
    assert launcher.explain(device.to_device(a), device.to_device(b), c)["products"] == ["mfma 16x16x32 i8"]
    launcher(device.to_device(a), device.to_device(b), c)
    np.testing.assert_array_equal(c.to_host(), a[:, :kk].astype(np.int64) @ b[:, :kk].astype(np.int64).T)


def test_nn_gemm_on_a_larger_grid_keeps_its_meaning_on_mfma(device):
    """krn's GEMM example launched on one block row and column more than the output needs: the extra blocks read
    and store nothing, so it is not the whole-product kernel's launch; the generic lowering runs it on MFMA."""
    m, n, k = 96, 80, 64
    rng = np.random.default_rng(4)
    a = rng.uniform(-1, 1, (m, k)).astype(np.float16)
    b = rng.uniform(-1, 1, (k, n)).astype(np.float16)
    c = device.empty(T.f16, m, n)
    launcher = device.launcher(programs.matmul, Blocks(-(-n // 32) + 1, -(-m // 32) + 1))
    tiling = programs.Tiling(bm=32, bn=32, bk=16)
    explained = launcher.explain(tiling, device.to_device(a), device.to_device(b), c)
    assert explained["plan"] == "GenericPlan" and explained["products"] == ["mfma 16x16x16 f16"]
    launcher(tiling, device.to_device(a), device.to_device(b), c)
    assert_agrees(c.to_host().astype(np.float32), a.astype(np.float32), b.astype(np.float32), k, "f16")


@pytest.mark.parametrize("causal", [True, False])
def test_flash_attention_head_dimension_32_runs_on_mfma(device, causal):
    rng = np.random.default_rng(32)
    heads, seq, d = 3, 150, 32
    words = [bf16_words(rng.standard_normal((heads, seq, d)).astype(np.float32)) for _ in range(3)]
    consts = {"bq": 64, "bk": 64, "d": d, "causal": causal}
    scale = math.log2(math.e) / math.sqrt(d)
    launch = Blocks(-(-seq // 64), heads)
    o = device.empty(T.bf16, heads, seq, d)
    launcher = device.launcher(programs.flash_attention_bf16, launch)
    tensors = [device.to_device(w, T.bf16) for w in words]
    explained = launcher.explain(programs.Attention(**consts), *tensors, o, scale)
    assert explained["plan"] == "GenericPlan" and explained["products"] == ["mfma 16x16x32 bf16"] * 2
    assert any("flash-attention" in reason for reason in explained["why"])
    launcher(programs.Attention(**consts), *tensors, o, scale)
    got = bf16_values(o.to_host()).astype(np.float64)
    want = np.zeros((heads, seq, d), np.uint16)
    emulate.run(capture(KERNELS, "flash_attention_bf16", consts={"t": consts}), launch, [*words, want, scale])
    np.testing.assert_allclose(got, bf16_values(want), atol=2e-2)
    q, kk, v = (bf16_values(w).astype(np.float64) for w in words)
    scores = np.einsum("hqd,hkd->hqk", q, kk) / math.sqrt(d)
    if causal:
        scores = np.where(np.tril(np.ones((seq, seq), bool)), scores, -np.inf)
    p = np.exp(scores - scores.max(axis=-1, keepdims=True))
    reference = np.einsum("hqk,hkd->hqd", p / p.sum(axis=-1, keepdims=True), v)
    np.testing.assert_allclose(got, reference, atol=2e-2)


def test_fp8_gemm_on_a_larger_grid_runs_on_the_fp8_mfma(device):
    """An fp8 e4m3 GEMM with per-tensor scales, launched on one block column more than its output: not the
    whole-product kernel's launch, so the generic lowering runs its product on 16x16x32 fp8 MFMAs (OCP e4m3 on
    gfx950, the format krn's tensors hold). Checked against the decoded operands in float64."""
    from krn_amd import Blocks
    from oracle.numerics import e4m3_decode, e4m3_encode

    m, n, k = 128, 192, 256
    rng = np.random.default_rng(33)
    x, w = rng.standard_normal((m, k)).astype(np.float32), rng.standard_normal((n, k)).astype(np.float32)
    sa, sb = np.float32(np.abs(x).max() / 448), np.float32(np.abs(w).max() / 448)
    a, b = e4m3_encode(x / sa), e4m3_encode(w / sb)
    c = device.empty(T.bf16, m, n)
    tiling = programs.Tiling(bm=64, bn=64, bk=64)
    launcher = device.launcher(programs.gemm_fp8, Blocks(n // 64 + 1, m // 64))
    args = (tiling, device.to_device(a, T.f8e4m3fn), device.to_device(b, T.f8e4m3fn), c, sa, sb)
    explained = launcher.explain(*args)
    assert explained["plan"] == "GenericPlan" and explained["products"] == ["mfma 16x16x32 fp8"]
    launcher(*args)
    got = bf16_values(c.to_host()).astype(np.float64)
    da, db = e4m3_decode(a).astype(np.float64), e4m3_decode(b).astype(np.float64)
    scale = np.float64(np.float32(sa * sb))
    reference = (da @ db.T) * scale
    bound = (8 * 2.0**-24 * (k + 8) * (np.abs(da) @ np.abs(db).T)) * scale + np.abs(reference) * 2.0**-8 * 1.01
    assert np.all(np.abs(got - reference) <= bound + 1e-30)
