// Tile GEMM for gfx950: C[m, n] = epilogue(sum_k A[m, k] * B[n, k]) with both operands K-contiguous.
//
// This is the lowering of krn's tile contraction `acc += a[rows, ks] @ b[cols, ks].transpose()` followed by
// `c[rows, cols] = f(acc).to(dtype)` (reference compiler/ir.py:309-315 Accumulate, compiler/emit.py:788-821). One
// workgroup owns a BM x BN output tile, four waves split it 2 x 2, and every wave keeps its accumulators in
// registers as 32x32 MFMA blocks. The K loop stages 128-byte slices of both operands through LDS, double buffered:
// the global loads of slice k+1 are in flight while the MFMAs of slice k run.
//
// One byte-oriented main loop serves three operand formats, because each MFMA consumes the same 16 bytes per lane
// per half-wave:
//   bf16 / f16 : v_mfma_f32_32x32x16_{bf16,f16}   16 elements = 32 bytes of K per step
//   int8       : v_mfma_i32_32x32x32_i8           32 elements = 32 bytes of K per step
//   fp8 e4m3   : v_mfma_scale_f32_32x32x64_f8f6f4 64 elements = 64 bytes of K per step (unit E8M0 scales)
// The K order inside one instruction is the hardware's; A and B fragments are read with the same byte layout, so
// every lane pairs A[m, k] with B[n, k] for the same k.
//
// LDS layout: a tile row is 128 bytes = 8 chunks of 16 bytes; chunk c of row r lives at slot c ^ (r & 7), so the
// 16-byte fragment reads of 8 consecutive rows touch 8 different bank groups (no conflicts).
#include <type_traits>

#include "common.h"

namespace krn {

enum Op : int { MUL_SCALAR = 0, MUL_ROW = 1, MUL_COL = 2, ADD_SCALAR = 3, ADD_ROW = 4, ADD_COL = 5 };

struct Epilogue {
  int out_kind;          // F32, F16, BF16 or I32 (I32 only for an int8 product with no operations)
  int nops;              // elementwise operations applied in order, each rounded to float32
  int op[4];
  float scalar[4];
  const float* vec[4];   // per-row (length M) or per-column (length N) vectors
};

enum Format : int { FMT_BF16 = 0, FMT_F16 = 1, FMT_I8 = 2, FMT_FP8 = 3 };

template <int FMT>
struct Mfma;

template <>
struct Mfma<FMT_BF16> {
  typedef f32x16 Acc;
  static constexpr int kBytes = 32;  // bytes of K one instruction consumes per row
  __device__ static void step(Acc& c, const u32x4* a, const u32x4* b) {
    c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a[0]), __builtin_bit_cast(bf16x8, b[0]),
                                               c, 0, 0, 0);
  }
};

template <>
struct Mfma<FMT_F16> {
  typedef f32x16 Acc;
  static constexpr int kBytes = 32;
  __device__ static void step(Acc& c, const u32x4* a, const u32x4* b) {
    c = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a[0]), __builtin_bit_cast(f16x8, b[0]), c,
                                              0, 0, 0);
  }
};

template <>
struct Mfma<FMT_I8> {
  typedef i32x16 Acc;
  static constexpr int kBytes = 32;
  __device__ static void step(Acc& c, const u32x4* a, const u32x4* b) {
    c = __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(i32x4, a[0]), __builtin_bit_cast(i32x4, b[0]), c, 0,
                                             0, 0);
  }
};

template <>
struct Mfma<FMT_FP8> {
  typedef f32x16 Acc;
  static constexpr int kBytes = 64;
  __device__ static void step(Acc& c, const u32x4* a, const u32x4* b) {
    i32x8 av, bv;
    i32x4 a0 = __builtin_bit_cast(i32x4, a[0]), a1 = __builtin_bit_cast(i32x4, a[1]);
    i32x4 b0 = __builtin_bit_cast(i32x4, b[0]), b1 = __builtin_bit_cast(i32x4, b[1]);
    av = (i32x8){a0[0], a0[1], a0[2], a0[3], a1[0], a1[1], a1[2], a1[3]};
    bv = (i32x8){b0[0], b0[1], b0[2], b0[3], b1[0], b1[1], b1[2], b1[3]};
    // format 0 = e4m3 for both operands; E8M0 scale 127 = 2^0
    c = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(av, bv, c, 0, 0, 0, 127, 0, 127);
  }
};

__device__ __forceinline__ float apply_ops(float v, const Epilogue& e, int64_t m, int64_t n) {
  for (int i = 0; i < e.nops; ++i) {
    float s;
    switch (e.op[i] % 3) {
      case 0: s = e.scalar[i]; break;
      case 1: s = e.vec[i][m]; break;
      default: s = e.vec[i][n]; break;
    }
    v = e.op[i] < 3 ? __fmul_rn(v, s) : __fadd_rn(v, s);
  }
  return v;
}

// Write one 32x32 block of results from a wave's LDS patch (row stride 33 words): lane l takes row l/2 and 16
// consecutive columns, applies the epilogue and converts. Not inlined: the loop is over LDS, not registers.
template <bool INT>
__device__ __noinline__ void store_patch(const uint32_t* patch, void* C, int64_t ldc, int64_t row0, int64_t col0,
                                         int64_t M, int64_t N, const Epilogue& e, int lane) {
  const int r = lane >> 1, c0 = (lane & 1) * 16;
  const int64_t m = row0 + r;
  if (m >= M) return;
  for (int c = c0; c < c0 + 16; ++c) {
    const int64_t n = col0 + c;
    if (n >= N) break;
    const uint32_t bits = patch[r * 33 + c];
    if (INT && e.out_kind == I32) {
      static_cast<int32_t*>(C)[m * ldc + n] = (int32_t)bits;
      continue;
    }
    const float v = apply_ops(INT ? (float)(int32_t)bits : __uint_as_float(bits), e, m, n);
    switch (e.out_kind) {
      case BF16: static_cast<uint16_t*>(C)[m * ldc + n] = f2bf(v); break;
      case F16: static_cast<uint16_t*>(C)[m * ldc + n] = f2h(v); break;
      default: static_cast<float*>(C)[m * ldc + n] = v; break;
    }
  }
}

// 16 bytes of row `base` starting at byte `kb`, zero past the row's end or for a row outside the matrix. VEC: the
// row is 16-byte aligned and its length a multiple of 16, so one dwordx4 load does it.
template <bool VEC>
__device__ __forceinline__ u32x4 load16(const uint8_t* __restrict__ p, int64_t base, int64_t kb, bool inside,
                                        int64_t kbytes) {
  if constexpr (VEC) {
    return (inside && kb < kbytes) ? *reinterpret_cast<const u32x4*>(p + base + kb) : u32x4{};
  } else {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint32_t v = 0;
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const int64_t at = kb + i * 4 + b;
        v |= (inside && at < kbytes) ? (uint32_t)p[base + at] << (8 * b) : 0u;
      }
      w[i] = v;
    }
    return u32x4{w[0], w[1], w[2], w[3]};
  }
}

// Tile index of this workgroup. Workgroups are dispatched round-robin over the 8 XCDs, so consecutive ids are
// first regrouped per XCD (each XCD gets one contiguous range of tiles and its own L2 sees a compact panel), then
// ordered in groups of GROUP_M tile rows so neighbours share A rows and B columns.
__device__ __forceinline__ void tile_of(int tiles_m, int tiles_n, int& tm, int& tn) {
  constexpr int GROUP_M = 8;
  int nb = tiles_m * tiles_n;
  int bid = blockIdx.x;
  if (nb % 8 == 0) bid = (bid % 8) * (nb / 8) + bid / 8;
  int per_group = GROUP_M * tiles_n;
  int group = bid / per_group;
  int first = group * GROUP_M;
  int size = min(tiles_m - first, GROUP_M);
  int local = bid % per_group;
  tm = first + local % size;
  tn = local / size;
}

// BM x BN tile, WM x WN waves, K sliced 128 bytes at a time. `kbytes` is K times the element size; rows of A and B
// are `lda`/`ldb` bytes apart. VEC: every row is 16-byte aligned and kbytes % 16 == 0, so 16-byte loads are legal.
template <int FMT, int BM, int BN, int WM, int WN, bool VEC>
__global__ __launch_bounds__(256, 1) void gemm_tile(const uint8_t* __restrict__ A, const uint8_t* __restrict__ B,
                                                    void* __restrict__ C, int64_t M, int64_t N, int64_t kbytes,
                                                    int64_t lda, int64_t ldb, int64_t ldc, Epilogue e) {
  typedef Mfma<FMT> Unit;
  typedef typename Unit::Acc Acc;
  constexpr int BKB = 128;             // bytes of K per slice
  constexpr int TM = BM / WM / 32;     // 32x32 blocks per wave along M
  constexpr int TN = BN / WN / 32;
  constexpr int STEP = Unit::kBytes;   // bytes of K per MFMA
  constexpr int CH = STEP / 32;        // 16-byte chunks per lane per MFMA operand
  constexpr int PA = BM / 32, PB = BN / 32;  // load passes (32 rows of 8 chunks per pass)
  static_assert(WM * WN == 4, "four waves");

  __shared__ u32x4 lds[2][(BM + BN) * 8];

  int tm, tn;
  tile_of((int)((M + BM - 1) / BM), (int)((N + BN - 1) / BN), tm, tn);
  const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int lrow = t >> 3, lchunk = t & 7;

  Acc acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = Acc{};

  u32x4 ra[PA], rb[PB];
  const int nk = (int)((kbytes + BKB - 1) / BKB);

  // Global -> registers for K slice `kt`, registers -> LDS stage `s`. Written as macros, not lambdas: a lambda
  // capturing the staging arrays by reference takes their address and sends them to scratch memory.
#define KRN_LOAD(kt)                                                                                            \
  do {                                                                                                          \
    const int64_t kb = (int64_t)(kt) * BKB + lchunk * 16;                                                       \
    _Pragma("unroll") for (int p = 0; p < PA; ++p) {                                                            \
      const int64_t row = m0 + lrow + 32 * p;                                                                   \
      ra[p] = load16<VEC>(A, row * lda, kb, row < M, kbytes);                                                   \
    }                                                                                                           \
    _Pragma("unroll") for (int p = 0; p < PB; ++p) {                                                            \
      const int64_t row = n0 + lrow + 32 * p;                                                                   \
      rb[p] = load16<VEC>(B, row * ldb, kb, row < N, kbytes);                                                   \
    }                                                                                                           \
  } while (0)
#define KRN_STORE(s)                                                                                            \
  do {                                                                                                          \
    _Pragma("unroll") for (int p = 0; p < PA; ++p) {                                                            \
      const int row = lrow + 32 * p;                                                                            \
      lds[s][row * 8 + (lchunk ^ (row & 7))] = ra[p];                                                           \
    }                                                                                                           \
    _Pragma("unroll") for (int p = 0; p < PB; ++p) {                                                            \
      const int row = BM + lrow + 32 * p;                                                                       \
      lds[s][row * 8 + (lchunk ^ (row & 7))] = rb[p];                                                           \
    }                                                                                                           \
  } while (0)

  KRN_LOAD(0);
  KRN_STORE(0);
  __syncthreads();
  const int half = lane >> 5, r32 = lane & 31;
  for (int kt = 0; kt < nk; ++kt) {
    const int s = kt & 1;
    if (kt + 1 < nk) KRN_LOAD(kt + 1);
#pragma unroll
    for (int k = 0; k < BKB / STEP; ++k) {
      u32x4 fa[TM][CH], fb[TN][CH];
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int row = wm * (BM / WM) + i * 32 + r32;
#pragma unroll
        for (int c = 0; c < CH; ++c) {
          const int chunk = (k * STEP + half * (STEP / 2)) / 16 + c;
          fa[i][c] = lds[s][row * 8 + (chunk ^ (row & 7))];
        }
      }
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int row = BM + wn * (BN / WN) + j * 32 + r32;
#pragma unroll
        for (int c = 0; c < CH; ++c) {
          const int chunk = (k * STEP + half * (STEP / 2)) / 16 + c;
          fb[j][c] = lds[s][row * 8 + (chunk ^ (row & 7))];
        }
      }
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) Unit::step(acc[i][j], fa[i], fb[j]);
    }
    if (kt + 1 < nk) KRN_STORE(s ^ 1);
    __syncthreads();
  }

  // C layout of a 32x32 MFMA block: lane holds column (lane & 31) and rows (r/4)*8 + (lane/32)*4 + r%4. Each block
  // goes through a per-wave 32x33-word LDS patch so the global stores run along rows; only the register -> LDS
  // copy is unrolled, which keeps every accumulator index a compile-time constant (a runtime index would send the
  // whole accumulator array to scratch memory).
  typedef std::remove_cv_t<std::remove_reference_t<decltype(acc[0][0][0])>> Elem;  // float or int
  Elem* patch = reinterpret_cast<Elem*>(&lds[0][0]) + wave * (32 * 33);
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) {
#pragma unroll
      for (int r = 0; r < 16; ++r)
        patch[((r >> 2) * 8 + half * 4 + (r & 3)) * 33 + r32] = acc[i][j][r];
      __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the patch is written before any lane reads it
      __builtin_amdgcn_wave_barrier();
      store_patch<FMT == FMT_I8>((const uint32_t*)patch, C, ldc, m0 + wm * (BM / WM) + i * 32, n0 + wn * (BN / WN) + j * 32, M, N,
                                 e, lane);
      __builtin_amdgcn_wave_barrier();
    }
}

}  // namespace krn

using namespace krn;

template <int FMT, int BM, int BN, int WM, int WN>
static int launch_gemm(const void* a, const void* b, void* c, int64_t m, int64_t n, int64_t kbytes, int64_t lda,
                       int64_t ldb, int64_t ldc, const Epilogue& e, hipStream_t stream) {
  const int64_t tiles = ((m + BM - 1) / BM) * ((n + BN - 1) / BN);
  if (tiles == 0) return 0;
  if (tiles > 0x7fffffff) {
    krn_set_error("gemm: %lld tiles exceed the grid limit", (long long)tiles);
    return -1;
  }
  const bool vec = kbytes % 16 == 0 && lda % 16 == 0 && ldb % 16 == 0 && (uintptr_t)a % 16 == 0 &&
                   (uintptr_t)b % 16 == 0;
  dim3 grid((unsigned)tiles), block(256);
  if (vec) {
    hipLaunchKernelGGL((gemm_tile<FMT, BM, BN, WM, WN, true>), grid, block, 0, stream, (const uint8_t*)a,
                       (const uint8_t*)b, c, m, n, kbytes, lda, ldb, ldc, e);
  } else if constexpr (BM <= 128) {  // the byte-wise loads need the registers a 256-row tile would take
    hipLaunchKernelGGL((gemm_tile<FMT, BM, BN, WM, WN, false>), grid, block, 0, stream, (const uint8_t*)a,
                       (const uint8_t*)b, c, m, n, kbytes, lda, ldb, ldc, e);
  } else {
    krn_set_error("gemm: a %dx%d tile needs 16-byte aligned rows", BM, BN);
    return -1;
  }
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    krn_set_error("gemm launch: %s", hipGetErrorString(err));
    return (int)err;
  }
  return 0;
}

static int gemm_dispatch(int fmt, const void* a, const void* b, void* c, int64_t m, int64_t n, int64_t k,
                         int64_t elem, const Epilogue& e, hipStream_t stream) {
  const int64_t kbytes = k * elem, lda = k * elem, ldb = k * elem;
  const int64_t ldc = n;
  // Tile selection for 256 CUs: a 256x256 tile when that still gives every CU a tile, else 128x128.
  const int64_t big = ((m + 255) / 256) * ((n + 255) / 256);
  const bool vec = kbytes % 16 == 0 && (uintptr_t)a % 16 == 0 && (uintptr_t)b % 16 == 0;
  const bool large = big >= 256 && vec;
#define KRN_GEMM(F)                                                                                    \
  return large ? launch_gemm<F, 256, 256, 2, 2>(a, b, c, m, n, kbytes, lda, ldb, ldc, e, stream)      \
               : launch_gemm<F, 128, 128, 2, 2>(a, b, c, m, n, kbytes, lda, ldb, ldc, e, stream)
  switch (fmt) {
    case FMT_BF16: KRN_GEMM(FMT_BF16);
    case FMT_F16: KRN_GEMM(FMT_F16);
    case FMT_I8: KRN_GEMM(FMT_I8);
    case FMT_FP8: KRN_GEMM(FMT_FP8);
  }
#undef KRN_GEMM
  krn_set_error("gemm: unknown operand format %d", fmt);
  return -1;
}

extern "C" {

// See include/krn_amd.h for the contract of each entry point.
int krn_gemm_nt(int in_kind, const void* a, const void* b, void* c, int out_kind, int64_t m, int64_t n, int64_t k,
                int nops, const int* ops, const float* scalars, const float* const* vectors, void* stream) {
  Epilogue e{};
  e.out_kind = out_kind;
  if (nops < 0 || nops > 4) {
    krn_set_error("gemm: %d epilogue operations, at most 4", nops);
    return -1;
  }
  e.nops = nops;
  for (int i = 0; i < nops; ++i) {
    e.op[i] = ops[i];
    e.scalar[i] = scalars ? scalars[i] : 0.0f;
    e.vec[i] = vectors ? vectors[i] : nullptr;
    if (ops[i] < 0 || ops[i] > 5) {
      krn_set_error("gemm: unknown epilogue operation %d", ops[i]);
      return -1;
    }
    if (ops[i] % 3 != 0 && e.vec[i] == nullptr) {
      krn_set_error("gemm: epilogue operation %d needs a vector", i);
      return -1;
    }
  }
  if (m < 0 || n < 0 || k < 0) {
    krn_set_error("gemm: negative extent");
    return -1;
  }
  int fmt;
  int64_t elem;
  switch (in_kind) {
    case BF16: fmt = FMT_BF16; elem = 2; break;
    case F16: fmt = FMT_F16; elem = 2; break;
    case I8: fmt = FMT_I8; elem = 1; break;
    case F8E4M3: fmt = FMT_FP8; elem = 1; break;
    default: krn_set_error("gemm: operand kind %d has no matrix unit product", in_kind); return -1;
  }
  if (out_kind == I32 && (fmt != FMT_I8 || nops != 0)) {
    krn_set_error("gemm: an int32 result needs int8 operands and no epilogue operations");
    return -1;
  }
  if (out_kind != F32 && out_kind != F16 && out_kind != BF16 && out_kind != I32) {
    krn_set_error("gemm: output kind %d is not stored by the tile GEMM", out_kind);
    return -1;
  }
  return gemm_dispatch(fmt, a, b, c, m, n, k, elem, e, (hipStream_t)stream);
}

}  // extern "C"

// out[c, r] = in[r, c] for 16-bit elements, through a 64x65-word LDS tile: the B operand of a `b[ks, cols]`
// product is turned K-contiguous before the NT main loop reads it.
__global__ __launch_bounds__(256) void transpose16(const uint16_t* __restrict__ in, uint16_t* __restrict__ out,
                                                   int64_t rows, int64_t cols) {
  __shared__ uint16_t tile[64][65];
  const int64_t r0 = (int64_t)blockIdx.y * 64, c0 = (int64_t)blockIdx.x * 64;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  for (int i = ty; i < 64; i += 4) {
    const int64_t r = r0 + i, c = c0 + tx;
    tile[i][tx] = (r < rows && c < cols) ? in[r * cols + c] : 0;
  }
  __syncthreads();
  for (int i = ty; i < 64; i += 4) {
    const int64_t c = c0 + i, r = r0 + tx;
    if (c < cols && r < rows) out[c * rows + r] = tile[tx][i];
  }
}

extern "C" int krn_transpose16(const void* in, void* out, int64_t rows, int64_t cols, void* stream) {
  if (rows < 0 || cols < 0) {
    krn_set_error("transpose: negative extent");
    return -1;
  }
  if (rows == 0 || cols == 0) return 0;
  const int64_t gx = (cols + 63) / 64, gy = (rows + 63) / 64;
  if (gx > 0x7fffffff || gy > 65535) {
    krn_set_error("transpose: %lld x %lld exceeds the grid limit", (long long)rows, (long long)cols);
    return -1;
  }
  hipLaunchKernelGGL(transpose16, dim3((unsigned)gx, (unsigned)gy), dim3(256), 0, (hipStream_t)stream,
                     (const uint16_t*)in, (uint16_t*)out, rows, cols);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    krn_set_error("transpose launch: %s", hipGetErrorString(err));
    return (int)err;
  }
  return 0;
}
