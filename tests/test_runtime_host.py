"""Host-side runtime contract (no GPU): the backend seam keyed by krn's `Target`, stream-ordered argument keeping,
event time-outs, and launches that must fall back to the generic lowering. The HIP runtime is replaced by a fake
whose events complete when the test says so."""

import dataclasses
from dataclasses import dataclass, field
from types import SimpleNamespace
from typing import ClassVar

import pytest

from krn_amd.runtime import api, hip, hipapi


@dataclass(frozen=True)
class Target:
    """A stand-in with the fields of krn's `Target` / `AMD` (reference src/krn/facts/targets.py:90-108, 214-237)."""

    vendor: ClassVar[str] = "amd"
    arch: str
    warp_size: int = 64
    shared_bytes: int = 160 * 1024
    features: frozenset = field(default_factory=frozenset)
    storage: frozenset = field(default_factory=frozenset)
    mma: frozenset = field(default_factory=frozenset)
    scaled: frozenset = frozenset({"mxfp4", "mxfp8"})


@dataclass(frozen=True)
class NvidiaTarget(Target):
    vendor: ClassVar[str] = "nvidia"


class FakeApi:
    """hipEventRecord / hipEventQuery / hipStreamIsCapturing / hipStreamSynchronize over events the test finishes."""

    def __init__(self) -> None:
        self.finished: set[int] = set()
        self.recorded: list[int] = []
        self.synced = 0
        fake = self

        class Lib:
            @staticmethod
            def hipEventQuery(handle):
                return 0 if handle.value in fake.finished else 600

            @staticmethod
            def hipEventDestroy(handle):
                return 0

        self.lib = Lib()

    def hipEventRecord(self, event, stream):
        self.recorded.append(event.value)

    def hipStreamSynchronize(self, stream):
        self.synced += 1

    def hipStreamIsCapturing(self, stream, status):
        pass  # leaves the status at 0: not capturing

    def hipEventSynchronize(self, event):
        self.finished.add(event.value)


@pytest.fixture
def fake(monkeypatch):
    fake = FakeApi()
    counter = iter(range(1000, 10**6))
    monkeypatch.setattr(hipapi, "api", lambda: fake)
    monkeypatch.setattr(hipapi, "event_create", lambda timing=True: next(counter))
    return fake


def test_backend_device_takes_krn_target_objects_and_arch_names(monkeypatch):
    """`device_of(Target.of("gfx950"))` is how krn asks (reference runtime/api.py:341-354): the backend reads the
    target's arch, builds one device per arch, and refuses other archs and other vendors."""
    made = []

    class FakeDevice:
        def __init__(self, arch):
            made.append(arch)
            self.arch = arch

    monkeypatch.setattr(hip, "HIPDevice", FakeDevice)
    backend = hip.HIPBackend()
    by_target = backend.device(Target("gfx950"))
    assert by_target.arch == "gfx950" and backend.device("gfx950") is by_target and made == ["gfx950"]
    with pytest.raises(api.BackendUnavailable, match="serves gfx950, not gfx942"):
        backend.device(Target("gfx942"))
    with pytest.raises(TypeError, match="AMD targets"):
        backend.device(NvidiaTarget("gfx950"))
    with pytest.raises(TypeError):
        api.arch_of(3)


def test_device_of_with_a_target_reaches_the_amd_backend(monkeypatch):
    """The binding a maintainer adds upstream is `src/krn/runtime/hip.py: from krn_amd.runtime.hip import BACKEND`;
    krn's `device_of(target)` then calls `BACKEND.device(target)` with its Target. Both spellings give one device."""
    monkeypatch.setattr(hip, "HIPDevice", lambda arch: SimpleNamespace(arch=arch))
    monkeypatch.setattr(hip, "BACKEND", hip.HIPBackend())
    monkeypatch.setattr(api, "_devices", {})
    device = api.device_of(Target("gfx950"))
    assert device.arch == "gfx950"
    assert api.device_of(Target("gfx950")) is device
    assert hip.BACKEND.device(Target("gfx950")) is device
    with pytest.raises(api.BackendUnavailable, match="no backend"):
        api.device_of(NvidiaTarget("sm_90a"))


def test_a_stream_holds_launch_arguments_until_a_later_marker_completes(fake):
    """The Keeper contract (reference runtime/completion.py:99-131): arguments of a launch stay referenced until
    a marker recorded after it is done; pending_launches lists launches under unfinished markers, then unmarked."""
    stream = hip.HIPStream(SimpleNamespace(), 1)
    stream.note("a", ("tensor a",))
    first = stream.record()
    stream.note("b", ("tensor b",))
    assert stream.pending_launches() == ("a", "b")
    second = stream.record()
    assert stream.pending_launches() == ("a", "b")
    fake.finished.add(first.handle)
    assert stream.pending_launches() == ("b",)
    stream.note("c", ())
    fake.finished.add(second.handle)
    third = stream.record()  # releases both finished markers
    assert len(stream._marks) == 1 and stream.pending_launches() == ("c",)
    fake.finished.add(third.handle)
    assert stream.pending_launches() == ()
    stream.note("d", ())
    stream.sync()
    assert stream.pending_launches() == () and not stream._marks and fake.synced == 1


def test_a_stream_that_never_synchronizes_holds_a_bounded_number_of_launches(fake):
    """A replay loop that only waits on its own events (never `sync`) must not accumulate arguments: after
    KEEP_LIMIT open launches the stream marks them itself, and completed markers are dropped."""
    stream = hip.HIPStream(SimpleNamespace(), 1)
    for i in range(10 * hip.KEEP_LIMIT):
        stream.note("k", (i,))
        fake.finished.update(fake.recorded)  # the device keeps up
    held = len(stream._open) + sum(len(launches) for _, launches in stream._marks)
    assert held <= 2 * hip.KEEP_LIMIT
    assert len(fake.recorded) >= 9


def test_event_wait_times_out_when_the_device_never_finishes(fake):
    """reference runtime/cuda_backend.py:132-142: a wait with a timeout polls until the deadline, then raises."""
    event = hip.HIPEvent(SimpleNamespace(), 77)
    with pytest.raises(TimeoutError):
        event.wait(timeout=0.05)
    fake.finished.add(77)
    event.wait(timeout=0.05)
    assert event.done()


def test_a_gemm_with_more_epilogue_operations_than_the_library_takes_lowers_generically(monkeypatch):
    """krn_gemm_nt takes at most four epilogue operations; a longer chain must keep the generic lowering instead of
    failing at launch."""
    from krn_amd import Blocks
    from krn_amd.compiler import cdna4
    from krn_amd.compiler.capture import capture
    from krn_amd.runtime import library
    from tests.conftest import KERNELS

    monkeypatch.setattr(library, "gemm_nt_call", lambda *a: (lambda stream: None))
    kernel = capture(KERNELS, "gemm_w8a8", consts={"t": {"bm": 64, "bn": 64, "bk": 32}})
    plan = cdna4.lower(kernel)
    op = plan.ops[0]
    long_plan = dataclasses.replace(plan, ops=(op,) * (library.MAX_OPS + 1))
    launch = hip.Launch(kernel, long_plan)
    m, n, k = 16, 200, 256
    params = {"a": SimpleNamespace(shape=(m, k), pointer=1), "w": SimpleNamespace(shape=(n, k), pointer=2),
              "scale_a": SimpleNamespace(shape=(m, 1), pointer=3, dtype=library.F32),
              "scale_w": SimpleNamespace(shape=(1, n), pointer=4, dtype=library.F32),
              "c": SimpleNamespace(shape=(m, n), pointer=5)}
    assert launch._gemm(long_plan, params, Blocks(4, 1)) is None
    assert launch._gemm(plan, params, Blocks(4, 1)) is not None


def test_a_kernel_parameter_table_keeps_its_parameters_alive():
    """A prepared generic launch keeps only the kernelParams table; the parameter objects whose addresses it holds
    must live as long as the table, or a later replay would pass freed memory as kernel arguments."""
    import ctypes
    import gc

    def prepared():
        return hip.Program.table([ctypes.c_int64(1111 * i) for i in range(6)] + [ctypes.c_void_p(0xABC)])

    table = prepared()
    gc.collect()
    _ = [ctypes.c_int64(-1) for _ in range(1000)]  # reuse of freed memory would show here
    assert [ctypes.c_int64.from_address(a).value for a in table] == [1111 * i for i in range(6)] + [0xABC]
