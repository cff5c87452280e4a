"""krn's own `Kernel` objects launch through this backend unchanged.

krn's `Kernel` carries only `fn` and `name` (reference src/krn/frontend/kernel.py:38-40); its `SourceLauncher` takes
the parameter names from `inspect.signature(kernel.fn)` (reference src/krn/runtime/runtime.py:469), `Const` fields
from `@struct` dataclasses, element types as parametrised classes (`fp[L[8], L[7], ieee]`) and geometry as
`Blocks` / `Tiles` records. The stand-ins in `tests/kernels/krn_style.py` have exactly those public fields.

The CPU tests go `BACKEND.device(Target) -> .launcher(kernel) -> .explain(...)` with tensors that only carry a shape,
an element type and a pointer (nothing is launched); the GPU tests launch a GEMM and a flash attention that way and
check them against float64.
"""

import math
from types import SimpleNamespace

import numpy as np
import pytest

from krn_amd import dtypes as D
from krn_amd.compiler.capture import TargetError
from krn_amd.frontend import const_fields, is_const
from krn_amd.runtime import hip
from tests.kernels import krn_style as krn
from tests.test_runtime_host import Target


def tensor(dtype, *shape):
    """A device tensor record for planning only: never freed, never read."""
    t = object.__new__(hip.HIPTensor)
    t.device, t.pointer, t.dtype, t.shape = None, 1 << 20, D.of(dtype), tuple(shape)
    t.numpy, t._owner, t._stream = D.NUMPY[t.dtype], None, None
    return t


@pytest.fixture
def device(monkeypatch):
    monkeypatch.setattr(hip, "HIPDevice", lambda arch: SimpleNamespace(arch=arch))
    monkeypatch.setattr(hip, "BACKEND", hip.HIPBackend())
    found = hip.BACKEND.device(Target("gfx950"))
    return SimpleNamespace(arch=found.arch, launcher=lambda kernel, launch=None: hip.HIPLauncher(found, kernel, launch))


def test_the_stand_in_has_only_krns_fields():
    assert set(krn.Kernel.__slots__) == {"fn", "name", "_shape"}
    assert not hasattr(krn.gemm_nt, "parameters")


def test_krn_element_types_and_const_fields_are_read_by_structure():
    assert [D.of(t) for t in (krn.bf16, krn.f16, krn.f32, krn.f8e4m3fn, krn.i8, krn.i32)] == [
        D.BF16, D.F16, D.F32, D.F8E4M3, D.I8, D.I32]
    assert is_const(krn.Const[int]) and not is_const(int)
    assert const_fields(krn.Tiling()) == {"bm": 256, "bn": 256, "bk": 64}
    with pytest.raises(TypeError):
        D.of(krn.fp[krn.L[3], krn.L[3], krn.ieee])


def test_a_krn_kernel_plans_through_device_launcher_explain(device):
    m = n = k = 1024
    launcher = device.launcher(krn.gemm_nt)
    assert launcher.parameters == ("t", "a", "b", "c")
    explained = launcher.explain(krn.Tiling(), tensor(krn.bf16, m, k), tensor(krn.bf16, n, k), tensor(krn.bf16, m, n))
    assert explained["plan"] == "GemmPlan" and explained["kernel"] == "gemm_nt"
    # keyword arguments are placed by the signature's names
    again = launcher.explain(krn.Tiling(), c=tensor(krn.bf16, m, n), b=tensor(krn.bf16, n, k), a=tensor(krn.bf16, m, k))
    assert again["plan"] == "GemmPlan"
    with pytest.raises(TypeError, match="missing the argument"):
        launcher.explain(krn.Tiling(), tensor(krn.bf16, m, k))


def test_krn_geometry_records_are_taken_by_their_fields(device):
    m = n = k = 512
    args = (krn.Tiling(), tensor(krn.bf16, m, k), tensor(krn.bf16, n, k), tensor(krn.bf16, m, n))
    tiles = device.launcher(krn.gemm_nt, krn.Tiles((m, n), (256, 256)))
    assert tiles.launch == hip.Blocks(2, 2, 1) and tiles.explain(*args)["plan"] == "GemmPlan"
    larger = device.launcher(krn.gemm_nt, krn.Blocks(3, 2))
    assert larger.explain(*args)["plan"] == "GenericPlan"  # one block column more than the output: generic
    with pytest.raises(TargetError, match="not a tile launch geometry"):
        device.launcher(krn.gemm_nt, SimpleNamespace(count=5))


def test_krn_flash_attention_kernel_plans_as_attention(device):
    bh, s, d = 8, 512, 128
    q, kk, v, o = (tensor(krn.bf16, bh, s, d) for _ in range(4))
    explained = device.launcher(krn.flash_attention, krn.Blocks(s // 128, bh)).explain(krn.Attention(), q, kk, v, o, 0.1)
    assert explained["plan"] == "AttentionPlan"
    # the grid inferred from `block.tile(t.bq)` alone has one head: not the whole problem, so the generic lowering
    assert device.launcher(krn.flash_attention).explain(krn.Attention(), q, kk, v, o, 0.1)["plan"] == "GenericPlan"


@pytest.mark.gpu
def test_a_krn_kernel_launches_a_gemm_on_gfx950():
    from krn_amd.runtime.api import device_of
    from oracle.numerics import bf16_values, bf16_words
    from tests.helpers import assert_agrees

    gpu = hip.BACKEND.device(Target("gfx950"))
    assert device_of("gfx950") is gpu
    m, n, k = 768, 512, 1024
    rng = np.random.default_rng(3)
    aw = bf16_words(rng.standard_normal((m, k)).astype(np.float32))
    bw = bf16_words(rng.standard_normal((n, k)).astype(np.float32))
    a, b = gpu.to_device(aw, krn.bf16), gpu.to_device(bw, krn.bf16)
    c = gpu.empty(krn.bf16, m, n)
    launcher = gpu.launcher(krn.gemm_nt, krn.Tiles((m, n), (256, 256)))
    assert launcher.explain(krn.Tiling(), a, b, c)["plan"] == "GemmPlan"
    launcher(krn.Tiling(), a, b, c)
    assert_agrees(bf16_values(c.to_host()), bf16_values(aw), bf16_values(bw).T, k, "bf16")


@pytest.mark.gpu
def test_a_krn_kernel_launches_flash_attention_on_gfx950():
    from oracle.numerics import bf16_values, bf16_words

    gpu = hip.BACKEND.device(Target("gfx950"))
    bh, s, d = 4, 384, 128
    rng = np.random.default_rng(5)
    words = [bf16_words(rng.standard_normal((bh, s, d)).astype(np.float32)) for _ in range(3)]
    q, kk, v = (gpu.to_device(w, krn.bf16) for w in words)
    o = gpu.empty(krn.bf16, bh, s, d)
    scale = math.log2(math.e) / math.sqrt(d)
    launcher = gpu.launcher(krn.flash_attention, krn.Blocks(s // 128, bh))
    assert launcher.explain(krn.Attention(), q, kk, v, o, scale)["plan"] == "AttentionPlan"
    launcher(krn.Attention(), q, kk, v, o, scale)
    qf, kf, vf = (bf16_values(w).astype(np.float64) for w in words)
    scores = np.einsum("hqd,hkd->hqk", qf, kf) * scale
    scores = np.where(np.arange(s)[None, :] <= np.arange(s)[:, None], scores, -np.inf)
    p = np.exp2(scores - scores.max(axis=-1, keepdims=True))
    want = np.einsum("hqk,hkd->hqd", p / p.sum(axis=-1, keepdims=True), vf)
    np.testing.assert_allclose(bf16_values(o.to_host()), want, atol=2e-2)
