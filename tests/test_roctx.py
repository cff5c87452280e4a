"""ROCTx ranges (reference src/krn/profile/providers/amd/tracer.py:31-56; its test tests/profile/test_vendors.py:
46-69): the tracer closes exactly the range it opened, refuses native activity collection, names ROCm when the
library is missing, and calls the real ROCTx library (a no-op outside a profiler). On CPU."""

from types import SimpleNamespace
from unittest.mock import Mock

import pytest

from krn_amd.compiler.capture import TargetError
from krn_amd.hw import FILENAMES, Libraries, LibraryNotFound
from krn_amd.runtime import roctx


def test_start_returns_the_closer_of_its_own_range(monkeypatch):
    closed: list[int] = []
    ids = iter((7, 8, 9))
    handle = SimpleNamespace(roctxRangeStartA=Mock(side_effect=lambda name: next(ids)),
                             roctxRangeStop=Mock(side_effect=closed.append))
    monkeypatch.setattr(roctx, "_handle", lambda: handle)
    outer = roctx.ROCTxTracer().start("outer")
    inner = roctx.ROCTxTracer().start("inner")
    inner()
    outer()
    assert closed == [8, 7]
    assert [c.args[0] for c in handle.roctxRangeStartA.call_args_list] == [b"outer", b"inner"]
    with roctx.span("body"):
        pass
    assert closed == [8, 7, 9] and handle.roctxRangeStartA.call_count == 3


def test_span_closes_on_error(monkeypatch):
    closed: list[int] = []
    handle = SimpleNamespace(roctxRangeStartA=Mock(return_value=3), roctxRangeStop=Mock(side_effect=closed.append))
    monkeypatch.setattr(roctx, "_handle", lambda: handle)
    with pytest.raises(ValueError):
        with roctx.span("failing"):
            raise ValueError
    assert closed == [3]


def test_native_activity_is_refused():
    with pytest.raises(TargetError):
        roctx.ROCTxTracer().collect()


def test_a_missing_library_names_rocm(monkeypatch):
    monkeypatch.setitem(FILENAMES, "roctx", ("libroctx64-not-here.so",))
    Libraries.clear_cache()
    try:
        assert not roctx.ROCTxTracer.is_available()
        with pytest.raises(LibraryNotFound, match="ROCm"):
            Libraries.load("roctx")
    finally:
        Libraries.clear_cache()


@pytest.mark.skipif(Libraries.find("roctx") is None, reason="no ROCTx library on this machine")
def test_the_real_library_opens_and_closes_ranges():
    roctx._handle.cache_clear()
    with roctx.span("krn_amd test range"):
        roctx.ROCTxTracer().start("nested")()


def test_launch_ranges_switch():
    before = roctx.launch_ranges()
    try:
        assert roctx.launch_ranges(True) is True and roctx.launch_ranges() is True
        assert roctx.launch_ranges(False) is False
    finally:
        roctx.launch_ranges(before)
