"""Flash attention on the paired grid with a ragged last query tile, through the C ABI.

At 1024 query tiles or more the kernel gives each workgroup two query tiles of one head, the late one first; the
second tile's first barrier waits only for the loads issued before the first tile's output stores, which counts on
every wave issuing all D / 16 of its stores, including waves whose rows all lie past the sequence end (those stores
fall outside the buffer resource over the head's rows and are dropped). Here sq = sk = 4136: 17 query tiles of 256
per head (the middle one runs alone), and the last tile holds 40 rows, so six of its eight waves have none. Sampled
heads are checked against a float64 softmax (bf16 operands: atol 2e-2, as for the other bf16 attention tests), and
the rows past the end must stay untouched."""

import math

import numpy as np
import pytest

from krn_amd import T
from krn_amd.dtypes import BF16
from krn_amd.runtime import library
from oracle.numerics import bf16_values, bf16_words

pytestmark = pytest.mark.gpu

HEADS, SEQ = 64, 4136
CHECKED = [0, 37, 63]


def float64_attention(q, k, v, causal):
    s = q @ k.T / math.sqrt(q.shape[-1])
    if causal:
        s = np.where(np.tril(np.ones(s.shape, bool)), s, -np.inf)
    p = np.exp(s - s.max(axis=-1, keepdims=True))
    return (p / p.sum(axis=-1, keepdims=True)) @ v


@pytest.mark.parametrize("d,causal", [(128, True), (128, False), (64, True)])
def test_paired_grid_with_a_ragged_last_query_tile(device, d, causal):
    rng = np.random.default_rng(700 + d + causal)
    words = [bf16_words(rng.standard_normal((HEADS, SEQ, d)).astype(np.float32)) for _ in range(3)]
    q, k, v = (device.to_device(w, T.bf16) for w in words)
    # one extra head's worth of sentinel rows after O: nothing may be written past the last head
    o = device.to_device(np.full((HEADS + 1, SEQ, d), 0x7FC1, np.uint16), T.bf16)
    library.attention_fwd(BF16, q.pointer, k.pointer, v.pointer, o.pointer, HEADS, SEQ, SEQ, d,
                          math.log2(math.e) / math.sqrt(d), causal, device.default_stream.handle)
    got = o.to_host()
    assert np.all(got[HEADS] == 0x7FC1)
    for h in CHECKED:
        want = float64_attention(*(bf16_values(w[h]).astype(np.float64) for w in words), causal)
        np.testing.assert_allclose(bf16_values(got[h]).astype(np.float64), want, atol=2e-2)
