// Row softmax for gfx950: y[r, c] = exp(x[r, c] - max_r) / sum_r exp(x[r, :] - max_r) over the first `width`
// columns of every row, in float32, rounded once to the element type of y.
//
// This is the lowering of krn's softmax tile programs (reference examples/02_tiles_and_types/01_softmax_rows.py
// :27-40, the long rows in column chunks with a running maximum and sum; tests/helpers/example_softmax.py:12-24,
// one tile per row block, `.softmax(axis=1)` or its spelled-out steps). Both compute the same function: the
// running form and the one-tile form differ only in rounding. Columns past `width` (the one-tile program's lanes
// past its tile) are neither read nor written; a row is a run of valid lanes, so no padding value enters the
// maximum or the sum.
//
// Layout (HBM-bound: one read, one write per element). One wave per row, four rows per workgroup, no LDS and no
// barriers (or, for at most 4096 rows longer than 2048 columns, four waves per row): lane l owns the 8-element
// chunks l, l + 64, ...; it keeps a running maximum m and sum s of its chunks (s rescaled by exp(m_old - m_new)
// when m grows), the wave combines the 64 pairs by shuffles, and a second pass writes exp(x - m) * (1 / s). Up to
// CACHE chunks per lane stay in registers between the passes, so those rows are read from HBM once; longer rows
// are read again (from L2).
#include "common.h"

namespace krn {

constexpr float LOG2E = 1.4426950408889634f;

// Eight elements of row `row` from chunk `c` as float32; lanes at or past `width` read -infinity (they then add
// exp(-inf) = 0 to the sum and never win the maximum)
template <int KIND>
__device__ __forceinline__ void load8(const void* X, int64_t row, int64_t ld, int64_t c, int64_t width, bool vec,
                                      float* v) {
  const int64_t col = c * 8;
  if (vec && col + 8 <= width) {
    if constexpr (KIND == F32) {
      const f32x4* p = reinterpret_cast<const f32x4*>(static_cast<const float*>(X) + row * ld + col);
      const f32x4 a = p[0], b = p[1];
      v[0] = a[0], v[1] = a[1], v[2] = a[2], v[3] = a[3], v[4] = b[0], v[5] = b[1], v[6] = b[2], v[7] = b[3];
    } else {
      const u32x4 w = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(X) + row * ld + col);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint16_t lo = (uint16_t)(w[q] & 0xffff), hi = (uint16_t)(w[q] >> 16);
        v[2 * q] = KIND == F16 ? h2f(lo) : bf2f(lo);
        v[2 * q + 1] = KIND == F16 ? h2f(hi) : bf2f(hi);
      }
    }
    return;
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int64_t at = col + e;
    if (at < width) {
      if constexpr (KIND == F32) v[e] = static_cast<const float*>(X)[row * ld + at];
      else {
        const uint16_t h = static_cast<const uint16_t*>(X)[row * ld + at];
        v[e] = KIND == F16 ? h2f(h) : bf2f(h);
      }
    } else {
      v[e] = -INFINITY;
    }
  }
}

// Whole 16-bit chunks (one 16-byte store per lane, lanes contiguous) are stored non-temporally: the output is not read
// again by this kernel, and keeping it out of the caches' way lifts f16 32768 x 4096 from 5.0 to 6.5 TB/s. float32
// chunks are two 16-byte stores 32 bytes apart per lane, half lines per instruction, which are slower non-temporal
// (8192 x 4096: 0.047 -> 0.067 ms), so they keep ordinary stores.
template <int KIND>
__device__ __forceinline__ void store8(void* Y, int64_t row, int64_t ld, int64_t c, int64_t width, bool vec,
                                       const float* v) {
  const int64_t col = c * 8;
  if (vec && col + 8 <= width) {
    if constexpr (KIND == F32) {
      f32x4* p = reinterpret_cast<f32x4*>(static_cast<float*>(Y) + row * ld + col);
      p[0] = f32x4{v[0], v[1], v[2], v[3]};
      p[1] = f32x4{v[4], v[5], v[6], v[7]};
    } else {
      uint32_t w[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t lo = KIND == F16 ? f2h(v[2 * q]) : f2bf(v[2 * q]);
        const uint32_t hi = KIND == F16 ? f2h(v[2 * q + 1]) : f2bf(v[2 * q + 1]);
        w[q] = lo | (hi << 16);
      }
      __builtin_nontemporal_store(u32x4{w[0], w[1], w[2], w[3]},
                                  reinterpret_cast<u32x4*>(static_cast<uint16_t*>(Y) + row * ld + col));
    }
    return;
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int64_t at = col + e;
    if (at < width) {
      if constexpr (KIND == F32) static_cast<float*>(Y)[row * ld + at] = v[e];
      else static_cast<uint16_t*>(Y)[row * ld + at] = KIND == F16 ? f2h(v[e]) : f2bf(v[e]);
    }
  }
}

// (m, s) += the eight values: m the running maximum, s the sum of exp(x - m)
__device__ __forceinline__ void accumulate(float& m, float& s, const float* v) {
  float top = v[0];
#pragma unroll
  for (int e = 1; e < 8; ++e) top = fmaxf(top, v[e]);
  const float m_new = fmaxf(m, top);
  if (m_new == -INFINITY) return;  // nothing valid yet
  float add = 0.0f;
#pragma unroll
  for (int e = 0; e < 8; ++e) add += __builtin_amdgcn_exp2f((v[e] - m_new) * LOG2E);
  s = s * __builtin_amdgcn_exp2f((m - m_new) * LOG2E) + add;
  m = m_new;
}

// SPLIT waves share one row (4 / SPLIT rows per workgroup): lane t of the row's 64 * SPLIT owns chunks t, t + 64 *
// SPLIT, ...; with SPLIT > 1 the waves' (m, s) pairs meet in LDS. One wave per row fills the chip when rows are
// many; a whole workgroup per row keeps enough loads in flight when few long rows are all there is.
// (m, s) and (m2, s2) merged: both sums rescaled to the larger maximum
__device__ __forceinline__ void combine(float& m, float& s, float m2, float s2) {
  const float m_new = fmaxf(m, m2);
  if (m_new != -INFINITY)
    s = s * __builtin_amdgcn_exp2f((m - m_new) * LOG2E) + s2 * __builtin_amdgcn_exp2f((m2 - m_new) * LOG2E);
  m = m_new;
}

template <int KIND, int CACHE, int SPLIT>
__global__ __launch_bounds__(256) void softmax_rows(const void* __restrict__ X, void* __restrict__ Y, int64_t rows,
                                                   int64_t width, int64_t ldx, int64_t ldy) {
  constexpr int STRIDE = 64 * SPLIT;
  const int lane = threadIdx.x % STRIDE;
  const int64_t row = (int64_t)blockIdx.x * (4 / SPLIT) + threadIdx.x / STRIDE;
  if constexpr (SPLIT == 1) {
    if (row >= rows) return;  // a whole wave leaves together; no barrier follows
  }
  const int64_t chunks = (width + 7) / 8;
  const int esize = KIND == F32 ? 4 : 2;
  const bool vec = (ldx * esize) % 16 == 0 && (ldy * esize) % 16 == 0 && (uintptr_t)X % 16 == 0 &&
                   (uintptr_t)Y % 16 == 0;
  float m = -INFINITY, s = 0.0f;
  float kept[CACHE][8];
#pragma unroll
  for (int i = 0; i < CACHE; ++i) {
    const int64_t c = lane + STRIDE * i;
    if (c < chunks) load8<KIND>(X, row, ldx, c, width, vec, kept[i]);
#pragma unroll
    for (int e = 0; e < 8; ++e) kept[i][e] = c < chunks ? kept[i][e] : -INFINITY;
    accumulate(m, s, kept[i]);
  }
  for (int64_t c = lane + STRIDE * CACHE; c < chunks; c += STRIDE) {
    float v[8];
    load8<KIND>(X, row, ldx, c, width, vec, v);
    accumulate(m, s, v);
  }
  // the wave's maximum and sum: pairs combined by shuffles
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) combine(m, s, __shfl_xor(m, off), __shfl_xor(s, off));
  if constexpr (SPLIT > 1) {
    __shared__ float part[2][4];
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) part[0][wave] = m, part[1][wave] = s;
    __syncthreads();
    m = part[0][0], s = part[1][0];
#pragma unroll
    for (int w = 1; w < SPLIT; ++w) combine(m, s, part[0][w], part[1][w]);
  }
  const float inv = 1.0f / s;
#pragma unroll
  for (int i = 0; i < CACHE; ++i) {
    const int64_t c = lane + STRIDE * i;
    if (c < chunks) {
      float y[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) y[e] = __builtin_amdgcn_exp2f((kept[i][e] - m) * LOG2E) * inv;
      store8<KIND>(Y, row, ldy, c, width, vec, y);
    }
  }
  for (int64_t c = lane + STRIDE * CACHE; c < chunks; c += STRIDE) {
    float v[8], y[8];
    load8<KIND>(X, row, ldx, c, width, vec, v);
#pragma unroll
    for (int e = 0; e < 8; ++e) y[e] = __builtin_amdgcn_exp2f((v[e] - m) * LOG2E) * inv;
    store8<KIND>(Y, row, ldy, c, width, vec, y);
  }
}

}  // namespace krn

using namespace krn;

template <int KIND>
static int launch_softmax(const void* x, void* y, int64_t rows, int64_t width, int64_t ldx, int64_t ldy,
                          hipStream_t stream) {
  const dim3 block(256);
  if (rows <= 4096 && width > 2048) {
    // few long rows: a workgroup per row; up to 16384 columns stay in registers between the passes
    hipLaunchKernelGGL((softmax_rows<KIND, 8, 4>), dim3((unsigned)rows), block, 0, stream, x, y, rows, width, ldx,
                       ldy);
  } else {
    // a wave per row; up to 2048 (4096) columns stay in registers, longer rows are read again from L2
    const dim3 grid((unsigned)((rows + 3) / 4));
    if (width <= 8 * 64 * 4)
      hipLaunchKernelGGL((softmax_rows<KIND, 4, 1>), grid, block, 0, stream, x, y, rows, width, ldx, ldy);
    else
      hipLaunchKernelGGL((softmax_rows<KIND, 8, 1>), grid, block, 0, stream, x, y, rows, width, ldx, ldy);
  }
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    krn_set_error("softmax launch: %s", hipGetErrorString(err));
    return (int)err;
  }
  return 0;
}

extern "C" int krn_softmax_rows(int kind, const void* x, void* y, int64_t rows, int64_t width, int64_t ldx,
                                int64_t ldy, void* stream) {
  if (kind != F32 && kind != F16 && kind != BF16) {
    krn_set_error("softmax: element kind %d; f32, f16 or bf16 only", kind);
    return -1;
  }
  if (rows < 0 || width < 0 || ldx < width || ldy < width) {
    krn_set_error("softmax: %lld rows of %lld columns with row strides %lld and %lld", (long long)rows,
                  (long long)width, (long long)ldx, (long long)ldy);
    return -1;
  }
  if (rows == 0 || width == 0) return 0;
  if ((rows + 3) / 4 > 0x7fffffff) {
    krn_set_error("softmax: %lld rows exceed the grid limit", (long long)rows);
    return -1;
  }
  hipStream_t s = (hipStream_t)stream;
  if (kind == F32) return launch_softmax<F32>(x, y, rows, width, ldx, ldy, s);
  if (kind == F16) return launch_softmax<F16>(x, y, rows, width, ldx, ldy, s);
  return launch_softmax<BF16>(x, y, rows, width, ldx, ldy, s);
}
