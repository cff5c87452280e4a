"""The flash-attention tile program on gfx950 against a float64 softmax and the oracle emulator."""

import math

import numpy as np
import pytest

from krn_amd import T, Blocks
from oracle import emulate
from oracle.numerics import bf16_values, bf16_words
from tests.conftest import KERNELS
from tests.kernels import tile_programs as programs

pytestmark = pytest.mark.gpu


def numpy_attention(q, k, v, causal):
    """softmax(Q K^T / sqrt(d)) V in float64 (reference tests/frontend/test_tile_ops.py:120-128)."""
    q, k, v = (x.astype(np.float64) for x in (q, k, v))
    s = q @ k.transpose(0, 2, 1) / math.sqrt(q.shape[-1])
    if causal:
        s = np.where(np.tril(np.ones(s.shape[-2:], bool)), s, -np.inf)
    p = np.exp(s - s.max(axis=-1, keepdims=True))
    return (p / p.sum(axis=-1, keepdims=True)) @ v


CASES = [(1, 37, 128, True), (2, 200, 128, False), (2, 200, 64, True), (3, 129, 128, True), (1, 256, 64, False),
         (2, 1, 128, True), (4, 512, 128, True)]


@pytest.mark.parametrize("heads,seq,d,causal", CASES)
def test_f16_flash_attention_matches_float64(device, heads, seq, d, causal):
    rng = np.random.default_rng(0)
    q, k, v = (rng.standard_normal((heads, seq, d)).astype(np.float16) for _ in range(3))
    o = device.empty(T.f16, heads, seq, d)
    tiling = programs.Attention(bq=16, bk=16, d=d, causal=causal)
    programs.flash_attention(tiling, *(device.to_device(x) for x in (q, k, v)), o,
                             math.log2(math.e) / math.sqrt(d), launch=Blocks(-(-seq // 16), heads))
    np.testing.assert_allclose(o.to_host().astype(np.float64), numpy_attention(q, k, v, causal), atol=3e-3)


@pytest.mark.parametrize("heads,seq,d,causal", CASES)
def test_bf16_flash_attention_matches_float64(device, heads, seq, d, causal):
    """bf16 keeps 8 significant bits: p and the output each round once, so the tolerance is 2e-2 absolute on
    N(0, 1) inputs (outputs are averages of v rows, |o| < 4)."""
    rng = np.random.default_rng(1)
    words = [bf16_words(rng.standard_normal((heads, seq, d)).astype(np.float32)) for _ in range(3)]
    values = [bf16_values(w) for w in words]
    o = device.empty(T.bf16, heads, seq, d)
    tiling = programs.Attention(bq=64, bk=64, d=d, causal=causal)
    programs.flash_attention_bf16(tiling, *(device.to_device(w, T.bf16) for w in words), o,
                                  math.log2(math.e) / math.sqrt(d), launch=Blocks(-(-seq // 64), heads))
    np.testing.assert_allclose(bf16_values(o.to_host()).astype(np.float64), numpy_attention(*values, causal),
                               atol=2e-2)


@pytest.mark.parametrize("causal", [False, True])
def test_f16_flash_attention_matches_the_oracle_emulator(device, causal):
    from krn_amd.compiler.capture import capture

    rng = np.random.default_rng(2)
    heads, seq, d = 2, 77, 64
    q, k, v = (rng.standard_normal((heads, seq, d)).astype(np.float16) for _ in range(3))
    scale = math.log2(math.e) / math.sqrt(d)
    consts = {"bq": 16, "bk": 16, "d": d, "causal": causal}
    launch = Blocks(-(-seq // 16), heads)
    o = device.empty(T.f16, heads, seq, d)
    programs.flash_attention(programs.Attention(**consts), *(device.to_device(x) for x in (q, k, v)), o, scale,
                             launch=launch)
    want = np.zeros((heads, seq, d), np.float16)
    emulate.run(capture(KERNELS, "flash_attention", consts={"t": consts}), launch, [q, k, v, want, scale])
    np.testing.assert_allclose(o.to_host().astype(np.float32), want.astype(np.float32), atol=2e-3)


def program_attention(q, k, v, scale, causal):
    """The flash-attention program's result in float64: p = exp2(scale * q.k - max) (the scale carries log2 e), the
    causal mask keeps key positions <= query positions, o = p v / sum p (tile_programs.flash_attention_bf16)."""
    q, k, v = (x.astype(np.float64) for x in (q, k, v))
    s = (q @ k.transpose(0, 2, 1)) * scale
    if causal:
        sq, sk = s.shape[-2:]
        s = np.where(np.arange(sk)[None, :] <= np.arange(sq)[:, None], s, -np.inf)
    p = np.exp2(s - s.max(axis=-1, keepdims=True))
    return (p / p.sum(axis=-1, keepdims=True)) @ v


def run_bf16_attention(device, words, causal, scale, d):
    heads, sq = words[0].shape[:2]
    o = device.empty(T.bf16, heads, sq, d)
    tiling = programs.Attention(bq=64, bk=64, d=d, causal=causal)
    programs.flash_attention_bf16(tiling, *(device.to_device(w, T.bf16) for w in words), o, scale,
                                  launch=Blocks(-(-sq // 64), heads))
    return bf16_values(o.to_host()).astype(np.float64)


@pytest.mark.parametrize("sq,sk,causal", [(200, 520, False), (200, 520, True), (300, 70, True), (300, 70, False),
                                          (64, 1, False), (1, 300, True), (1, 300, False)])
def test_bf16_flash_attention_with_different_query_and_key_lengths(device, sq, sk, causal):
    """Queries and keys of different lengths: the program runs over k's own length, and the causal mask compares
    absolute positions, so a query row at or past the last key sees every key."""
    heads, d = 2, 128
    rng = np.random.default_rng(sq * 1000 + sk)
    words = [bf16_words(rng.standard_normal((heads, n, d)).astype(np.float32)) for n in (sq, sk, sk)]
    scale = math.log2(math.e) / math.sqrt(d)
    got = run_bf16_attention(device, words, causal, scale, d)
    np.testing.assert_allclose(got, program_attention(*(bf16_values(w) for w in words), scale, causal), atol=2e-2)


@pytest.mark.parametrize("causal", [False, True])
def test_bf16_flash_attention_when_the_running_maximum_keeps_rising(device, causal):
    """Scores that climb by about 9 (in log2 units) every 64 keys: the kernel refreshes its exponent base only when
    a row maximum beats it by more than 8, so here it rescales the output and the row sum on nearly every tile, and
    the earlier tiles still weigh about 2^-9 each: a missed or doubled rescale shows at once."""
    heads, seq, d = 2, 512, 128
    rng = np.random.default_rng(9)
    q = np.ones((heads, seq, d), np.float32)
    level = 0.55 * (np.arange(seq) // 64)
    k = level[None, :, None] + 0.05 * rng.standard_normal((heads, seq, d))
    v = rng.standard_normal((heads, seq, d))
    words = [bf16_words(x.astype(np.float32)) for x in (q, k, v)]
    scale = math.log2(math.e) / math.sqrt(d)
    want = program_attention(*(bf16_values(w) for w in words), scale, causal)
    np.testing.assert_allclose(run_bf16_attention(device, words, causal, scale, d), want, atol=2e-2)


@pytest.mark.parametrize("factor", [-1.0, 0.0])
@pytest.mark.parametrize("causal", [False, True])
def test_bf16_flash_attention_with_a_scale_that_is_not_positive(device, factor, causal):
    """A negative scale reverses the order of the scores, so the row maximum cannot be taken on the raw scores; a
    zero scale makes every valid key weigh the same. The kernel scales every score first on that path."""
    heads, seq, d = 2, 200, 64
    rng = np.random.default_rng(11)
    words = [bf16_words(rng.standard_normal((heads, seq, d)).astype(np.float32)) for _ in range(3)]
    scale = factor * math.log2(math.e) / math.sqrt(d)
    want = program_attention(*(bf16_values(w) for w in words), scale, causal)
    np.testing.assert_allclose(run_bf16_attention(device, words, causal, scale, d), want, atol=2e-2)


@pytest.mark.parametrize("causal,d,heads,seq,rows,step", [(True, 128, 3, 300, 256, 32), (False, 64, 2, 200, 64, 32)])
def test_a_rewritten_attention_program_runs_on_the_attention_kernel(device, causal, d, heads, seq, rows, step):
    """krn's flash attention written another way (names, tiling, temporaries, operand order, the mask as
    `q_pos >= k_pos`): planned as the attention kernel and equal to a float64 softmax."""
    from tests.kernels import attention_variants as variants

    rng = np.random.default_rng(7)
    words = [bf16_words(rng.standard_normal((heads, seq, d)).astype(np.float32)) for _ in range(3)]
    values = [bf16_values(w) for w in words]
    o = device.empty(T.bf16, heads, seq, d)
    shape = variants.Shape(rows_per_block=rows, keys_per_step=step, head_dim=d, masked=causal)
    args = (shape, *(device.to_device(w, T.bf16) for w in words), o, math.log2(math.e) / math.sqrt(d))
    launcher = device.launcher(variants.reordered, Blocks(-(-seq // rows), heads))
    assert launcher.explain(*args)["plan"] == "AttentionPlan"
    launcher(*args)
    np.testing.assert_allclose(bf16_values(o.to_host()).astype(np.float64), numpy_attention(*values, causal),
                               atol=2e-2)


def test_a_4d_natural_exp_attention_program_runs_on_the_attention_kernel(device):
    """(batch, heads, seq, d) tensors indexed by blocks z and y, and `exp` with the plain 1/sqrt(d) scale: the
    kernel runs it as exp2 with the scale times log2(e)."""
    from tests.kernels import attention_variants as variants

    batch, heads, seq, d = 2, 3, 260, 128
    rng = np.random.default_rng(8)
    words = [bf16_words(rng.standard_normal((batch, heads, seq, d)).astype(np.float32)) for _ in range(3)]
    values = [bf16_values(w).reshape(batch * heads, seq, d) for w in words]
    o = device.empty(T.bf16, batch, heads, seq, d)
    args = (variants.Natural(), *(device.to_device(w, T.bf16) for w in words), o, 1 / math.sqrt(d))
    launcher = device.launcher(variants.natural_exp_4d, Blocks(-(-seq // 128), heads, batch))
    assert launcher.explain(*args)["plan"] == "AttentionPlan"
    launcher(*args)
    got = bf16_values(o.to_host()).astype(np.float64).reshape(batch * heads, seq, d)
    np.testing.assert_allclose(got, numpy_attention(*values, True), atol=2e-2)


def test_a_4d_attention_program_the_kernel_does_not_serve_runs_generically(device):
    """Head dimension 32 is outside the attention kernel: the same 4-D program lowers to generated HIP (two
    16x16x32 bf16 MFMA products, blocks over x, y and z) and still equals the float64 softmax."""
    from tests.kernels import attention_variants as variants

    batch, heads, seq, d = 2, 2, 130, 32
    rng = np.random.default_rng(9)
    words = [bf16_words(rng.standard_normal((batch, heads, seq, d)).astype(np.float32)) for _ in range(3)]
    values = [bf16_values(w).reshape(batch * heads, seq, d) for w in words]
    o = device.empty(T.bf16, batch, heads, seq, d)
    cfg = variants.Natural(bq=64, bk=64, d=d, causal=True)
    args = (cfg, *(device.to_device(w, T.bf16) for w in words), o, 1 / math.sqrt(d))
    launcher = device.launcher(variants.natural_exp_4d, Blocks(-(-seq // 64), heads, batch))
    explained = launcher.explain(*args)
    assert explained["plan"] == "GenericPlan" and explained["products"] == ["mfma 16x16x32 bf16"] * 2
    launcher(*args)
    got = bf16_values(o.to_host()).astype(np.float64).reshape(batch * heads, seq, d)
    np.testing.assert_allclose(got, numpy_attention(*values, True), atol=2e-2)
