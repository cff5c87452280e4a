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
