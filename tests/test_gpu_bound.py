"""`Launcher.bind` on gfx950 (reference src/krn/runtime/api.py:176-204 `Bound`): a bound launch marshals its
arguments once and replays only the library call, so it must give the direct call's result on every replay, read the
current contents of its tensors, write to new arguments after `rebind`, and keep per-launch scratch (the NN
product's transposed operand) alive until the launch is done."""

import math

import numpy as np
import pytest

from krn_amd import Blocks, T
from tests.helpers import bf16_normal
from tests.kernels import tile_programs as programs

pytestmark = pytest.mark.gpu


def test_bound_w8a8_replays_match_the_direct_call_and_read_new_contents(device):
    rng = np.random.default_rng(51)
    m, n, k = 16, 320, 256
    a = device.to_device(rng.integers(-127, 128, (m, k), dtype=np.int8), T.i8)
    w = device.to_device(rng.integers(-127, 128, (n, k), dtype=np.int8), T.i8)
    sa = device.to_device(rng.uniform(0.5, 2, (m, 1)).astype(np.float32))
    sw = device.to_device(rng.uniform(0.5, 2, (1, n)).astype(np.float32) / 127)
    c, other = device.empty(T.bf16, m, n), device.empty(T.bf16, m, n)
    launcher = programs.gemm_w8a8[programs.Tiling(bm=64, bn=64, bk=32)]
    launcher(a, w, sa, sw, c)
    want = c.to_host()
    bound = launcher.bind(a, w, sa, sw, c)
    for replay in range(3):
        c.copy_from(np.zeros((m, n), np.uint16))
        bound()
        np.testing.assert_array_equal(c.to_host(), want, err_msg=f"replay {replay}")
    a.copy_from(rng.integers(-127, 128, (m, k), dtype=np.int8))
    launcher(a, w, sa, sw, other)
    bound.submit().wait()
    np.testing.assert_array_equal(c.to_host(), other.to_host())
    other.copy_from(np.zeros((m, n), np.uint16))
    bound.rebind(a, w, sa, sw, other)
    bound()
    np.testing.assert_array_equal(other.to_host(), c.to_host())


def test_bound_nn_product_keeps_its_scratch(device):
    rng = np.random.default_rng(52)
    m, n, k = 130, 192, 96
    da = device.to_device(rng.uniform(-1, 1, (m, k)).astype(np.float16))
    db = device.to_device(rng.uniform(-1, 1, (k, n)).astype(np.float16))
    c = device.empty(T.f16, m, n)
    launcher = programs.matmul[programs.Tiling(bm=64, bn=64, bk=32)]
    launcher(da, db, c)
    want = c.to_host()
    bound = launcher.bind(da, db, c)
    for replay in range(4):
        c.copy_from(np.full((m, n), np.nan, np.float16))
        bound()
        np.testing.assert_array_equal(c.to_host(), want, err_msg=f"replay {replay}")


def test_bound_nn_replays_with_event_waits_only_keep_memory_flat(device):
    """A bound NN product replayed many times on a side stream, waiting only on its own events (never a stream
    synchronization): the transposed-operand scratch is allocated once per stream and reused, and the stream releases
    the launches' arguments as their markers complete, so neither device memory nor held launches grow."""
    from krn_amd.runtime import hipapi

    rng = np.random.default_rng(54)
    m, n, k = 256, 2048, 2048  # 8 MiB of scratch per transposed operand
    da = device.to_device(rng.uniform(-1, 1, (m, k)).astype(np.float16))
    db = device.to_device(rng.uniform(-1, 1, (k, n)).astype(np.float16))
    c = device.empty(T.f16, m, n)
    launcher = programs.matmul[programs.Tiling(bm=64, bn=64, bk=32)]
    launcher(da, db, c)
    want = c.to_host()
    side = device.stream()
    with side:
        bound = launcher.bind(da, db, c)
        bound.submit().wait()
        before = hipapi.memory_free()
        for _ in range(400):
            event = bound.submit()
        event.wait()
        after = hipapi.memory_free()
        side.record().wait()
    assert before - after < 64 << 20, f"device memory fell by {(before - after) >> 20} MiB over 400 replays"
    assert side.pending_launches() == ()
    np.testing.assert_array_equal(c.to_host(side), want)


def test_bound_attention_and_softmax_match_direct_calls(device):
    rng = np.random.default_rng(53)
    heads, seq, d = 2, 200, 64
    qkv = [device.to_device(bf16_normal(rng, (heads, seq, d))[0], T.bf16) for _ in range(3)]
    o = device.empty(T.bf16, heads, seq, d)
    scale = math.log2(math.e) / math.sqrt(d)
    attention = device.launcher(programs.flash_attention_bf16, Blocks(-(-seq // 64), heads))
    config = programs.Attention(bq=64, bk=64, d=d, causal=True)
    attention(config, *qkv, o, scale)
    want_o = o.to_host()
    x = device.to_device((rng.standard_normal((9, 3000)) * 3).astype(np.float16))
    y = device.empty(T.f16, 9, 3000)
    softmax = device.launcher(programs.softmax_long_rows, Blocks(3))
    tiling = programs.RowTiling(rows=4, cols=1024)
    softmax(tiling, x, y)
    want_y = y.to_host()
    bound_o, bound_y = attention.bind(config, *qkv, o, scale), softmax.bind(tiling, x, y)
    for replay in range(2):
        o.copy_from(np.zeros(o.shape, np.uint16))
        y.copy_from(np.zeros(y.shape, np.float16))
        bound_o()
        bound_y()
        np.testing.assert_array_equal(o.to_host(), want_o, err_msg=f"replay {replay}")
        np.testing.assert_array_equal(y.to_host(), want_y, err_msg=f"replay {replay}")
