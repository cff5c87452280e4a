"""A thin ctypes layer over the HIP runtime, the HIP module API and hiprtc: the C ABI the AMD backend drives.

Every call checks its hipError_t and raises `HIPError` with the driver's name and message
(the pattern of `CUDAError`/`check`, reference src/krn/runtime/cuda_backend.py:97-105). Nothing here needs PyTorch.
"""

import ctypes
from ctypes import POINTER, byref, c_char_p, c_float, c_int, c_size_t, c_uint, c_void_p

from krn_amd.hw import Libraries

hipStream_t = c_void_p
hipEvent_t = c_void_p

H2D, D2H, D2D = 1, 2, 3  # hipMemcpyKind


class HIPError(RuntimeError):
    """A HIP runtime or hiprtc call that failed: the function, the error name and the driver's message."""

    def __init__(self, function: str, code: int, name: str, message: str) -> None:
        self.function, self.code = function, code
        super().__init__(f"{function} failed with {name} ({code}): {message}")


CAPTURE_RELAXED = 2  # hipStreamCaptureModeRelaxed: allocation calls stay legal while a stream records


class _Api:
    """The resolved entry points of libamdhip64; built once on first use."""

    def __init__(self) -> None:
        lib = Libraries.load("hip").handle
        self.lib = lib
        lib.hipGetErrorName.restype = c_char_p
        lib.hipGetErrorString.restype = c_char_p
        signatures = {
            "hipInit": [c_uint],
            "hipGetDeviceCount": [POINTER(c_int)],
            "hipSetDevice": [c_int],
            "hipGetDevice": [POINTER(c_int)],
            "hipDeviceSynchronize": [],
            "hipDeviceGetAttribute": [POINTER(c_int), c_int, c_int],
            "hipDeviceGetName": [c_char_p, c_int, c_int],
            "hipMalloc": [POINTER(c_void_p), c_size_t],
            "hipFree": [c_void_p],
            "hipMemGetInfo": [POINTER(c_size_t), POINTER(c_size_t)],
            "hipMallocAsync": [POINTER(c_void_p), c_size_t, hipStream_t],
            "hipFreeAsync": [c_void_p, hipStream_t],
            "hipDeviceGetDefaultMemPool": [POINTER(c_void_p), c_int],
            "hipMemPoolSetAttribute": [c_void_p, c_int, c_void_p],
            "hipStreamIsCapturing": [hipStream_t, POINTER(c_int)],
            "hipHostMalloc": [POINTER(c_void_p), c_size_t, c_uint],
            "hipHostFree": [c_void_p],
            "hipMemcpy": [c_void_p, c_void_p, c_size_t, c_int],
            "hipMemcpyAsync": [c_void_p, c_void_p, c_size_t, c_int, hipStream_t],
            "hipMemsetAsync": [c_void_p, c_int, c_size_t, hipStream_t],
            "hipStreamCreate": [POINTER(hipStream_t)],
            "hipStreamDestroy": [hipStream_t],
            "hipStreamSynchronize": [hipStream_t],
            "hipStreamWaitEvent": [hipStream_t, hipEvent_t, c_uint],
            "hipEventCreateWithFlags": [POINTER(hipEvent_t), c_uint],
            "hipEventDestroy": [hipEvent_t],
            "hipEventRecord": [hipEvent_t, hipStream_t],
            "hipEventSynchronize": [hipEvent_t],
            "hipEventQuery": [hipEvent_t],
            "hipEventElapsedTime": [POINTER(c_float), hipEvent_t, hipEvent_t],
            "hipModuleLoadData": [POINTER(c_void_p), c_void_p],
            "hipModuleUnload": [c_void_p],
            "hipModuleGetFunction": [POINTER(c_void_p), c_void_p, c_char_p],
            "hipModuleLaunchKernel": [
                c_void_p, c_uint, c_uint, c_uint, c_uint, c_uint, c_uint, c_uint, hipStream_t,
                POINTER(c_void_p), POINTER(c_void_p),
            ],
            "hipFuncSetAttribute": [c_void_p, c_int, c_int],
            "hipGetLastError": [],
            "hipStreamBeginCapture": [hipStream_t, c_int],
            "hipStreamEndCapture": [hipStream_t, POINTER(c_void_p)],
            "hipGraphInstantiate": [POINTER(c_void_p), c_void_p, c_void_p, c_char_p, c_size_t],
            "hipGraphLaunch": [c_void_p, hipStream_t],
            "hipGraphExecDestroy": [c_void_p],
            "hipGraphDestroy": [c_void_p],
        }  # fmt: skip
        for name, argtypes in signatures.items():
            function = getattr(lib, name)
            function.argtypes, function.restype = argtypes, c_int

    def check(self, name: str, code: int) -> None:
        if code != 0:
            error = self.lib.hipGetErrorName(code).decode()
            message = self.lib.hipGetErrorString(code).decode()
            raise HIPError(name, code, error, message)

    def raw(self, name: str, *args) -> int:
        """Call a HIP function and return its status instead of raising (clean-up paths)."""
        return getattr(self.lib, name)(*args)

    def __getattr__(self, name: str):  # only called for names not set in __init__: the HIP functions
        function = getattr(self.lib, name)

        def call(*args):
            self.check(name, function(*args))

        call.__name__ = name
        setattr(self, name, call)
        return call


_api: _Api | None = None


def api() -> _Api:
    global _api
    if _api is None:
        _api = _Api()
    return _api


def device_count() -> int:
    """How many HIP devices this process sees; 0 when the runtime reports none (a machine without a GPU)."""
    try:
        lib = api()
    except OSError:
        return 0
    count = c_int(0)
    if lib.lib.hipGetDeviceCount(byref(count)) != 0:
        return 0
    return count.value


def malloc(nbytes: int) -> int:
    pointer = c_void_p()
    api().hipMalloc(byref(pointer), max(nbytes, 1))
    return pointer.value or 0


def free(pointer: int) -> None:
    api().hipFree(c_void_p(pointer))


def malloc_async(nbytes: int, stream: int) -> int:
    """Device memory from the device's default pool, ordered on `stream`: usable by work queued after this call on
    that stream, or on a stream that waited for an event recorded after it."""
    pointer = c_void_p()
    api().hipMallocAsync(byref(pointer), max(nbytes, 1), c_void_p(stream))
    return pointer.value or 0


def free_async(pointer: int, stream: int) -> None:
    """Return memory to its pool once the work queued on `stream` so far has run."""
    api().hipFreeAsync(c_void_p(pointer), c_void_p(stream))


RELEASE_THRESHOLD = 4  # hipMemPoolAttrReleaseThreshold


def keep_pool(ordinal: int) -> None:
    """Let the default pool of a device keep freed memory instead of returning it to the driver at every
    synchronization, so that stream-ordered allocation of a recently freed size costs no driver allocation."""
    pool = c_void_p()
    api().hipDeviceGetDefaultMemPool(byref(pool), ordinal)
    threshold = ctypes.c_uint64(2**64 - 1)
    api().hipMemPoolSetAttribute(pool, RELEASE_THRESHOLD, ctypes.cast(byref(threshold), c_void_p))


def capturing(stream: int) -> bool:
    """Is `stream` recording a graph (hipStreamCaptureStatusActive) right now?"""
    status = c_int(0)
    api().hipStreamIsCapturing(c_void_p(stream), byref(status))
    return status.value == 1


def memory_free() -> int:
    """Bytes of device memory the driver reports free (hipMemGetInfo)."""
    free_bytes, total = c_size_t(), c_size_t()
    api().hipMemGetInfo(byref(free_bytes), byref(total))
    return free_bytes.value


def stream_create() -> int:
    stream = hipStream_t()
    api().hipStreamCreate(byref(stream))
    return stream.value or 0


def event_create(timing: bool = True) -> int:
    event = hipEvent_t()
    api().hipEventCreateWithFlags(byref(event), 0 if timing else 2)  # 2 = hipEventDisableTiming
    return event.value or 0


def elapsed_ms(start: int, end: int) -> float:
    ms = c_float()
    api().hipEventElapsedTime(byref(ms), c_void_p(start), c_void_p(end))
    return ms.value


def device_name(ordinal: int = 0) -> str:
    buffer = ctypes.create_string_buffer(256)
    api().hipDeviceGetName(buffer, 256, ordinal)
    return buffer.value.decode()


class _Rtc:
    """The hiprtc entry points: compile generated HIP source to a gfx950 code object at run time."""

    def __init__(self) -> None:
        lib = Libraries.load("hiprtc").handle
        self.lib = lib
        lib.hiprtcGetErrorString.restype = c_char_p
        lib.hiprtcGetErrorString.argtypes = [c_int]
        signatures = {
            "hiprtcCreateProgram": [POINTER(c_void_p), c_char_p, c_char_p, c_int, c_void_p, c_void_p],
            "hiprtcCompileProgram": [c_void_p, c_int, POINTER(c_char_p)],
            "hiprtcGetProgramLogSize": [c_void_p, POINTER(c_size_t)],
            "hiprtcGetProgramLog": [c_void_p, c_char_p],
            "hiprtcGetCodeSize": [c_void_p, POINTER(c_size_t)],
            "hiprtcGetCode": [c_void_p, c_char_p],
            "hiprtcDestroyProgram": [POINTER(c_void_p)],
        }
        for name, argtypes in signatures.items():
            function = getattr(lib, name)
            function.argtypes, function.restype = argtypes, c_int

    def compile(self, source: str, name: str, options: list[str]) -> bytes:
        """The code object of `source`; a compile error raises HIPError carrying the compiler log."""
        program = c_void_p()
        code = self.lib.hiprtcCreateProgram(byref(program), source.encode(), f"{name}.hip".encode(), 0, None, None)
        if code:
            raise HIPError("hiprtcCreateProgram", code, "HIPRTC_ERROR", self.lib.hiprtcGetErrorString(code).decode())
        try:
            encoded = [option.encode() for option in options]
            array = (c_char_p * len(encoded))(*encoded)
            code = self.lib.hiprtcCompileProgram(program, len(encoded), array)
            if code:
                size = c_size_t()
                self.lib.hiprtcGetProgramLogSize(program, byref(size))
                log = ctypes.create_string_buffer(size.value + 1)
                self.lib.hiprtcGetProgramLog(program, log)
                raise HIPError("hiprtcCompileProgram", code, "HIPRTC_ERROR_COMPILATION", log.value.decode())
            size = c_size_t()
            self.lib.hiprtcGetCodeSize(program, byref(size))
            blob = ctypes.create_string_buffer(size.value)
            self.lib.hiprtcGetCode(program, blob)
            return blob.raw
        finally:
            self.lib.hiprtcDestroyProgram(byref(program))


_rtc: _Rtc | None = None


def rtc() -> _Rtc:
    global _rtc
    if _rtc is None:
        _rtc = _Rtc()
    return _rtc
