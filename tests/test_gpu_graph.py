"""`Device.graph` on gfx950: the launches of one function captured into a hipGraph and replayed with one call
(reference runtime/api.py:222-242 `Graph`, runtime/cuda_backend.py:486-551 `CUDAGraph`). Every replay is checked
against the eager result of the same launches, with eager work and synchronizations between the replays; a replay
sees new tensor contents; new arguments raise TargetError; scratch that a recorded launch allocated (the NN
product's transposed operand) outlives the recording."""

import gc
import math

import numpy as np
import pytest

from krn_amd import Blocks, T
from krn_amd.compiler.capture import TargetError
from oracle.numerics import bf16_values
from tests.helpers import bf16_normal
from tests.kernels import tile_programs as programs

pytestmark = pytest.mark.gpu

SENTINEL = 0x7FC0  # a bf16 NaN: an output the replay did not write stays visible


def pipeline(device, rng):
    """Three launches of different kinds: the bf16 NT product (MFMA kernel), causal flash attention, and a row
    softmax (generic lowering), with their inputs and outputs."""
    (aw, _), (bw, _) = bf16_normal(rng, (256, 192)), bf16_normal(rng, (320, 192))
    a, b = device.to_device(aw, T.bf16), device.to_device(bw, T.bf16)
    c = device.empty(T.bf16, 256, 320)
    heads, seq, d = 2, 192, 128
    qkv = [device.to_device(bf16_normal(rng, (heads, seq, d))[0], T.bf16) for _ in range(3)]
    o = device.empty(T.bf16, heads, seq, d)
    x = device.to_device(rng.standard_normal((8, 16)).astype(np.float32))
    y = device.empty(T.f32, 8, 16)

    def step():
        programs.gemm_nt[programs.Tiling(bm=64, bn=64, bk=32)](a, b, c)
        programs.flash_attention_bf16(programs.Attention(bq=64, bk=64, d=d, causal=True), *qkv, o,
                                      math.log2(math.e) / math.sqrt(d), launch=Blocks(-(-seq // 64), heads))
        programs.row_softmax(programs.Shape(), x, y, launch=Blocks(1))

    return step, (a, b, x), (c, o, y)


def clear(outputs):
    for t in outputs:
        fill = np.full(t.shape, SENTINEL, np.uint16) if t.numpy == np.uint16 else np.full(t.shape, np.nan, t.numpy)
        t.copy_from(fill)


def read(outputs):
    return [t.to_host() for t in outputs]


def test_every_replay_matches_the_eager_launches(device):
    rng = np.random.default_rng(31)
    step, _, outputs = pipeline(device, rng)
    clear(outputs)
    step()
    want = read(outputs)
    assert not np.isnan(bf16_values(want[0])).any()
    clear(outputs)
    graph = device.graph(step)
    # eager work of the same program on other buffers between replays, and a synchronization after each
    other_step, _, other_outputs = pipeline(device, np.random.default_rng(32))
    for replay in range(4):
        clear(outputs)
        graph()
        other_step()
        got = read(outputs)
        for g, w in zip(got, want):
            np.testing.assert_array_equal(g, w, err_msg=f"replay {replay}")
        device.sync()


def test_a_replay_reads_the_current_contents_of_recorded_tensors(device):
    rng = np.random.default_rng(33)
    step, inputs, outputs = pipeline(device, rng)
    graph = device.graph(step)
    a, b, x = inputs
    for trial in range(3):
        a.copy_from(bf16_normal(rng, a.shape)[0])
        x.copy_from(rng.standard_normal(x.shape).astype(np.float32))
        clear(outputs)
        step()
        want = read(outputs)
        clear(outputs)
        graph()
        for g, w in zip(read(outputs), want):
            np.testing.assert_array_equal(g, w, err_msg=f"trial {trial}")


def test_new_arguments_raise_target_error(device):
    rng = np.random.default_rng(34)
    (aw, _), (bw, _) = bf16_normal(rng, (128, 64)), bf16_normal(rng, (128, 64))
    a, b = device.to_device(aw, T.bf16), device.to_device(bw, T.bf16)
    c, other = device.empty(T.bf16, 128, 128), device.empty(T.bf16, 128, 128)

    def product(out):
        programs.gemm_nt[programs.Tiling(bm=64, bn=64, bk=32)](a, b, out)

    graph = device.graph(product, c)
    graph(c)
    with pytest.raises(TargetError):
        graph(other)


def test_the_nn_product_scratch_outlives_the_recording(device):
    """krn's NN GEMM example (b is K x N) transposes b into scratch the launch allocates; the graph keeps it."""
    rng = np.random.default_rng(35)
    m, n, k = 192, 256, 128
    a = rng.uniform(-1, 1, (m, k)).astype(np.float16)
    b = rng.uniform(-1, 1, (k, n)).astype(np.float16)
    da, db = device.to_device(a), device.to_device(b)
    c = device.empty(T.f16, m, n)

    def product():
        programs.matmul[programs.Tiling(bm=64, bn=64, bk=32)](da, db, c)

    product()
    want = c.to_host()
    graph = device.graph(product)
    device.sync()
    gc.collect()
    for replay in range(3):
        c.copy_from(np.full((m, n), np.nan, np.float16))
        graph()
        np.testing.assert_array_equal(c.to_host(), want, err_msg=f"replay {replay}")


def test_krn_graphs_0_replays_as_plain_launches(device, monkeypatch):
    monkeypatch.setenv("KRN_GRAPHS", "0")
    rng = np.random.default_rng(36)
    step, _, outputs = pipeline(device, rng)
    clear(outputs)
    step()
    want = read(outputs)
    graph = device.graph(step)
    clear(outputs)
    graph()
    for g, w in zip(read(outputs), want):
        np.testing.assert_array_equal(g, w)
