"""Throughput of krn's tile contraction path on one MI355X: bf16 GEMM 8192^3 (the headline), causal bf16 flash
attention, fp8 e4m3 and W8A8 int8 GEMMs, each run as an unchanged krn tile program through krn_amd.

`python bench.py [--gpus 1] [--steps K] [--warmup W]` prints ONE JSON line. A step is one launch of the headline
program (C = A @ B^T, M = N = K = 8192, bf16 in, fp32 accumulate, bf16 out) on inputs already resident in HBM,
timed with HIP events on the launch stream over exactly K steps after W warm-up steps, with a device
synchronization on both sides. The other configurations are reported under "extra" with the same method. The CPU
baseline is the oracle C backend (krn's CPU clang lowering restated) on a bounded sample of the same program.
"""

import argparse
import json
import math
import os
import sys
import time
from ctypes import c_void_p

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK = {"bf16": 2500.0, "fp8": 5000.0, "int8": 5000.0}  # dense MFMA TFLOP/s (TOP/s) of MI355X
HBM_PEAK = 8000.0  # GB/s


def events_ms(stream, run, steps: int) -> float:
    """Average milliseconds per step of `run()` over `steps` steps, by HIP events on `stream`."""
    from krn_amd.runtime import hipapi

    api = hipapi.api()
    start, end = hipapi.event_create(), hipapi.event_create()
    api.hipDeviceSynchronize()
    api.hipEventRecord(c_void_p(start), c_void_p(stream.handle))
    for _ in range(steps):
        run()
    api.hipEventRecord(c_void_p(end), c_void_p(stream.handle))
    api.hipEventSynchronize(c_void_p(end))
    api.hipDeviceSynchronize()
    return hipapi.elapsed_ms(start, end) / steps


def bf16_words(x: np.ndarray) -> np.ndarray:
    bits = x.astype(np.float32).view(np.uint32)
    return ((bits + np.uint32(0x7FFF) + ((bits >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)).astype(np.uint16)


def gemm_bf16(device, steps, warmup, rng, n=8192):
    from krn_amd import T
    from tests.kernels import tile_programs as programs

    a = device.to_device(bf16_words(rng.standard_normal((n, n), dtype=np.float32)), T.bf16)
    b = device.to_device(bf16_words(rng.standard_normal((n, n), dtype=np.float32)), T.bf16)
    c = device.empty(T.bf16, n, n)
    bound = programs.gemm_nt[programs.Tiling(bm=256, bn=256, bk=64)].bind(a, b, c)
    for _ in range(warmup):
        bound()
    ms = events_ms(device.default_stream, bound, steps)
    return ms, 2.0 * n**3, (a, b, c)


def attention_bf16(device, steps, warmup, rng, batch=4, heads=32, seq=4096, d=128):
    from krn_amd import T, Blocks
    from tests.kernels import tile_programs as programs

    shape = (batch * heads, seq, d)
    q, k, v = (device.to_device(bf16_words(rng.standard_normal(shape, dtype=np.float32)), T.bf16) for _ in range(3))
    o = device.empty(T.bf16, *shape)
    tiling = programs.Attention(bq=128, bk=64, d=d, causal=True)
    launcher = device.launcher(programs.flash_attention_bf16, Blocks(seq // 128, batch * heads))
    bound = launcher.bind(tiling, q, k, v, o, math.log2(math.e) / math.sqrt(d))
    for _ in range(warmup):
        bound()
    ms = events_ms(device.default_stream, bound, steps)
    return ms, 2.0 * batch * heads * seq * seq * d  # causal: half of 4 B H S^2 D


def transpose_copy(device, steps, warmup, rng, n=8192):
    """The calibration kernel for HBM byte counters: an n x n 16-bit transpose reads and writes 2 n^2 bytes each."""
    from krn_amd import T
    from krn_amd.runtime import library

    src = device.to_device(rng.integers(0, 1 << 16, (n, n), dtype=np.uint16), T.bf16)
    dst = device.empty(T.bf16, n, n)
    stream = device.default_stream

    def run():
        library.transpose16(src.pointer, dst.pointer, n, n, stream.handle)

    for _ in range(warmup):
        run()
    ms = events_ms(stream, run, steps)
    return ms, 2 * n * n


def softmax_f16(device, steps, warmup, rng, rows=32768, cols=4096):
    """krn's row softmax (the kernel its softmax tile programs lower to) over rows x cols f16: 256 MiB read and
    256 MiB written, twice the 256 MiB last-level cache, so every step streams from HBM."""
    from krn_amd import T
    from krn_amd.dtypes import F16
    from krn_amd.runtime import library

    x = device.to_device((rng.standard_normal((rows, cols), dtype=np.float32) * 4).astype(np.float16))
    y = device.empty(T.f16, rows, cols)
    stream = device.default_stream

    def run():
        library.softmax_rows(F16, x.pointer, y.pointer, rows, cols, cols, cols, stream.handle)

    for _ in range(warmup):
        run()
    return events_ms(stream, run, steps), 2 * 2 * rows * cols


def lib_matmul_bf16(device, steps, warmup, rng, library, n=8192):
    """krn's `lib.matmul` (C = A @ B with B stored K x N, the reference's NN form) on bf16 8192^3 through one named
    candidate: "hipblaslt" (the vendor library, the first of the reference's AMD order) or "ours" (krn's
    matmul_epilogue tile program on the MFMA GEMM)."""
    from krn_amd import T
    from krn_amd.lib import lib

    a = device.to_device(bf16_words(rng.standard_normal((n, n), dtype=np.float32)), T.bf16)
    b = device.to_device(bf16_words(rng.standard_normal((n, n), dtype=np.float32)), T.bf16)
    c = device.empty(T.bf16, n, n)

    def run():
        lib.matmul(a, b, out=c, library=library)

    for _ in range(warmup):
        run()
    return events_ms(device.default_stream, run, steps)


def quantize_e4m3(x: np.ndarray) -> tuple[np.ndarray, np.float32]:
    from krn_amd.formats import e4m3_encode

    scale = np.float32(np.abs(x).max() / 448.0)
    return e4m3_encode(x / scale), scale


def gemm_fp8(device, steps, warmup, rng, m, n=8192, k=8192):
    from krn_amd import T
    from tests.kernels import tile_programs as programs

    a, sa = quantize_e4m3(rng.standard_normal((m, k), dtype=np.float32))
    b, sb = quantize_e4m3(rng.standard_normal((n, k), dtype=np.float32))
    da, db = device.to_device(a, T.f8e4m3fn), device.to_device(b, T.f8e4m3fn)
    c = device.empty(T.bf16, m, n)
    bound = programs.gemm_fp8[programs.Tiling(bm=256, bn=256, bk=128)].bind(da, db, c, sa, sb)
    for _ in range(warmup):
        bound()
    ms = events_ms(device.default_stream, bound, steps)
    return ms, 2.0 * m * n * k, k * n + m * k + 2 * m * n


def gemm_w8a8(device, steps, warmup, rng, m, n=14336, k=4096):
    from krn_amd import T
    from tests.kernels import tile_programs as programs

    a = device.to_device(rng.integers(-127, 128, (m, k), dtype=np.int8))
    w = device.to_device(rng.integers(-127, 128, (n, k), dtype=np.int8))
    sa = device.to_device((rng.uniform(0.5, 1.5, (m, 1)) / 127).astype(np.float32))
    sw = device.to_device((rng.uniform(0.5, 1.5, (1, n)) / 127).astype(np.float32))
    c = device.empty(T.bf16, m, n)
    bound = programs.gemm_w8a8[programs.Tiling(bm=256, bn=256, bk=128)].bind(a, w, sa, sw, c)
    for _ in range(warmup):
        bound()
    ms = events_ms(device.default_stream, bound, steps)
    return ms, 2.0 * m * n * k, n * k + m * k + 4 * (m + n) + 2 * m * n


def cpu_model() -> str:
    """The host CPU's model name, as /proc/cpuinfo gives it."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(a_words: np.ndarray, b_words: np.ndarray, budget_s: float = 12.0, threads: int = 1) -> dict:
    """The oracle C backend (krn's CPU lowering: one thread per block, fmaf in k order) running the same gemm_nt
    program with 128 x 128 tiles over whole output tiles of the 8192^3 problem until `budget_s`: on one core (the
    reference's own execution model, one C call on one core), or with the block range split over `threads` host
    threads (the same per-block code, in batches of `threads` blocks)."""
    import ctypes

    from krn_amd.compiler.capture import capture
    from oracle.cbackend import Program
    from tests.conftest import KERNELS

    n = a_words.shape[0]
    tile = 128
    kernel = capture(KERNELS, "gemm_nt", consts={"t": {"bm": tile, "bn": tile, "bk": 32}})
    program = Program(kernel)
    c = np.zeros((n, n), np.uint16)
    native = program.arguments([a_words, b_words, c])
    grid = [ctypes.c_longlong(n // tile), ctypes.c_longlong(n // tile), ctypes.c_longlong(1)]
    blocks, elapsed = 0, 0.0
    start = time.perf_counter()
    while elapsed < budget_s and blocks < (n // tile) ** 2:
        step = min(threads, (n // tile) ** 2 - blocks)
        program.run_range(native, grid, blocks, blocks + step, threads)
        blocks += step
        elapsed = time.perf_counter() - start
    flops = 2.0 * tile * tile * n * blocks
    return {
        "value": flops / elapsed / 1e12,
        "unit": "TFLOP/s",
        "cores": threads,
        "cpu": cpu_model(),
        "kind": "port",
        "sample": f"{blocks} of {(n // tile) ** 2} 128x128 output tiles of the 8192^3 bf16 gemm_nt program "
                  f"(full K), oracle C backend, {threads} thread{'s' if threads > 1 else ''}, {elapsed:.1f} s",
    }


def main() -> None:
    parser = argparse.ArgumentParser(description=__doc__)
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=50)
    parser.add_argument("--warmup", type=int, default=5)
    parser.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    parser.add_argument("--only", default="", help="comma list of extra legs to run (fa, fp8, int8, softmax, copy, "
                        "blas; default all but copy); copy (the known-size calibration kernel for HBM byte counters) "
                        "runs only when named; blas is lib.matmul bf16 8192^3 NN through the hipBLASLt candidate and "
                        "through ours")
    args = parser.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (the tile kernels shard by output "
              "tiles or heads with no exchange; see DESIGN.md). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    os.environ.setdefault("KRN_TARGET", "gfx950")
    from krn_amd.runtime.api import device_of

    device = device_of("gfx950")
    rng = np.random.default_rng(0)
    print("[bench] bf16 gemm 8192^3", file=sys.stderr, flush=True)
    ms, flops, (a, b, c) = gemm_bf16(device, args.steps, args.warmup, rng)
    tflops = flops / ms / 1e9
    legs = set(filter(None, args.only.split(","))) or {"fa", "fp8", "int8", "softmax", "blas"}
    extra = {}
    if "fa" in legs:
        print("[bench] causal bf16 flash attention", file=sys.stderr, flush=True)
        fa_ms, fa_flops = attention_bf16(device, max(args.steps // 2, 5), args.warmup, rng)
        extra["flash_attn_causal_bf16_B4_H32_S4096_D128"] = {
            "ms": round(fa_ms, 4), "tflops": round(fa_flops / fa_ms / 1e9, 1),
            "frac_of_bf16_peak": round(fa_flops / fa_ms / 1e9 / PEAK["bf16"], 4)}
    if "fp8" in legs:
        for m in (8192, 128, 16, 1):
            print(f"[bench] fp8 gemm M={m}", file=sys.stderr, flush=True)
            f_ms, f_flops, f_bytes = gemm_fp8(device, args.steps, args.warmup, rng, m)
            extra[f"fp8_e4m3_gemm_M{m}_N8192_K8192"] = {
                "ms": round(f_ms, 4), "tflops": round(f_flops / f_ms / 1e9, 1),
                "frac_of_fp8_peak": round(f_flops / f_ms / 1e9 / PEAK["fp8"], 4),
                "gbps": round(f_bytes / f_ms / 1e6, 1), "frac_of_hbm": round(f_bytes / f_ms / 1e6 / HBM_PEAK, 4)}
    if "int8" in legs:
        for m in (4096, 16):
            print(f"[bench] w8a8 int8 gemm M={m}", file=sys.stderr, flush=True)
            i_ms, i_ops, i_bytes = gemm_w8a8(device, args.steps, args.warmup, rng, m)
            extra[f"w8a8_int8_gemm_M{m}_N14336_K4096"] = {
                "ms": round(i_ms, 4), "tops": round(i_ops / i_ms / 1e9, 1),
                "frac_of_int8_peak": round(i_ops / i_ms / 1e9 / PEAK["int8"], 4),
                "gbps": round(i_bytes / i_ms / 1e6, 1), "frac_of_hbm": round(i_bytes / i_ms / 1e6 / HBM_PEAK, 4)}
    if "softmax" in legs:
        print("[bench] f16 row softmax 32768x4096", file=sys.stderr, flush=True)
        s_ms, s_bytes = softmax_f16(device, args.steps, args.warmup, rng)
        extra["softmax_rows_f16_32768x4096"] = {"ms": round(s_ms, 4), "gbps": round(s_bytes / s_ms / 1e6, 1),
                                                "frac_of_hbm": round(s_bytes / s_ms / 1e6 / HBM_PEAK, 4)}
    if "copy" in legs:
        print("[bench] 16-bit transpose 8192^2 (counter calibration)", file=sys.stderr, flush=True)
        c_ms, c_bytes = transpose_copy(device, args.steps, args.warmup, rng)
        extra["transpose16_8192x8192"] = {"ms": round(c_ms, 4), "bytes_read": c_bytes, "bytes_written": c_bytes,
                                          "gbps": round(2 * c_bytes / c_ms / 1e6, 1)}
    if "blas" in legs:
        for library in ("hipblaslt", "ours"):
            print(f"[bench] lib.matmul bf16 8192^3 (NN) through {library}", file=sys.stderr, flush=True)
            v_ms = lib_matmul_bf16(device, args.steps, args.warmup, rng, library)
            extra[f"lib_matmul_bf16_nn_8192_{library}"] = {"ms": round(v_ms, 4),
                                                            "tflops": round(flops / v_ms / 1e9, 1)}
    baseline = None
    if not args.no_cpu:
        print("[bench] CPU baseline (oracle C backend, bounded sample)", file=sys.stderr, flush=True)
        baseline = cpu_baseline(a.to_host(), b.to_host())
        # the same port over the host's cores (at most 16: a GPU box's CPU share), reported beside the 1-core figure
        cores = max(1, min(16, os.cpu_count() or 1))
        print(f"[bench] CPU baseline on {cores} threads (bounded sample)", file=sys.stderr, flush=True)
        extra["cpu_baseline_all_cores"] = cpu_baseline(a.to_host(), b.to_host(), budget_s=8.0, threads=cores)
    traffic = None
    traffic_file = os.path.join(ROOT, "profiles", "gemm_bf16_8192_traffic.json")
    if os.path.exists(traffic_file):
        with open(traffic_file) as f:
            traffic = json.load(f).get("hbm_bytes_per_launch")
    line = {
        "metric": "TFLOP/s + % MFMA peak: fp8/bf16 tile GEMM 8192^3, causal bf16 flash-attn fwd",
        "value": round(tflops, 1),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: A, B ~ N(0,1) rounded to bf16 (seed 0), resident in HBM",
        "config": {"workload": "krn tile GEMM C = A @ B^T, M=N=K=8192, bf16 in, fp32 accumulate, bf16 out",
                   "program": "tests/kernels/tile_programs.py:gemm_nt", "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "achieved": round(tflops, 1), "peak": PEAK["bf16"], "unit": "TFLOP/s",
                     "frac": round(tflops / PEAK["bf16"], 4), "traffic": traffic},
        "cpu_baseline": baseline,
        "extra": extra,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
