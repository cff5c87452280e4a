// Tile GEMM for gfx950: C[m, n] = epilogue(sum_k A[m, k] * B[n, k]) with both operands K-contiguous.
//
// This is the lowering of krn's tile contraction `acc += a[rows, ks] @ b[cols, ks].transpose()` followed by
// `c[rows, cols] = f(acc).to(dtype)` (reference compiler/ir.py:309-315 Accumulate, compiler/emit.py:788-821). One
// workgroup owns a BM x BN output tile split among its waves, and every wave keeps its accumulators in registers as
// 32x32 MFMA blocks (`gemm_quad16`: 16x16 blocks of the transposed product). Main loops: `gemm_quad16` (every
// format, also the bf16/f16 NN form, 16x16 MFMAs) for whole 256 x 256 tiles of two K slices or more, `gemm_pipe`
// and `gemm_pp` (fp8) for one slice and, `gemm_pipe`, on 128 x 128 and 128 x 256 tiles for mid-size products,
// `gemm_skinny` for M <= 128 (rings of direct-to-LDS slices per wave), and `gemm_tile` for the rest (128-byte
// slices staged through registers, bounds-checked, double buffered). All end in `store_tile` (`gemm_quad16`:
// `store_tile16t`): whole blocks straight from the accumulators (the direct epilogue), the rest through an LDS patch.
//
// One byte-oriented main loop serves three operand formats, because each MFMA consumes the same 16 bytes per lane
// per half-wave:
//   bf16 / f16 : v_mfma_f32_32x32x16_{bf16,f16}   16 elements = 32 bytes of K per step
//   int8       : v_mfma_i32_32x32x32_i8           32 elements = 32 bytes of K per step
//   fp8 e4m3   : v_mfma_scale_f32_32x32x64_f8f6f4 64 elements = 64 bytes of K per step (unit E8M0 scales)
// The K order inside one instruction is the hardware's; A and B fragments are read with the same byte layout, so
// every lane pairs A[m, k] with B[n, k] for the same k.
//
// LDS layout: a tile row of a K slice is 64 or 128 bytes (4 or 8 chunks of 16 bytes), swizzled per row so that
// the 16-byte fragment reads of 16 consecutive rows hit distinct banks (swz4 / swz8 below).
#include <mutex>
#include <type_traits>

#include "common.h"

namespace krn {

// Epilogue operations. Codes 0-5 take a float32 scalar or a row/column vector; 6-8 are the activations of krn's
// `lib.matmul` (reference src/krn/lib/lib_kernels.py:31-48, formulas of compiler/emit.py:112-114). A vector's
// element kind rides in bits 4-5 of the code: 0 float32, 1 f16, 2 bf16.
enum Op : int {
  MUL_SCALAR = 0, MUL_ROW = 1, MUL_COL = 2, ADD_SCALAR = 3, ADD_ROW = 4, ADD_COL = 5, RELU = 6, GELU = 7, SILU = 8
};
constexpr int VEC_KIND_SHIFT = 4;

struct Epilogue {
  int out_kind;          // F32, F16, BF16 or I32 (I32 only for an int8 product with no operations)
  int nops;              // elementwise operations applied in order, each rounded to float32
  int op[4];
  float scalar[4];
  const void* vec[4];    // per-row (length M) or per-column (length N) vectors
};

__device__ __forceinline__ float activation(int op, float x) {
  if (op == RELU) return x < 0.0f ? 0.0f : x;
  if (op == GELU) return __fmul_rn(__fmul_rn(0.5f, x), __fadd_rn(1.0f, erff(__fmul_rn(x, 0.7071067811865476f))));
  return __fdiv_rn(x, __fadd_rn(1.0f, expf(-x)));  // SILU
}

enum Format : int { FMT_BF16 = 0, FMT_F16 = 1, FMT_I8 = 2, FMT_FP8 = 3 };

typedef short v4s16 __attribute__((ext_vector_type(4)));  // the result type of ds_read_b64_tr_b16

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

// The 16x16 forms, which consume twice the K per instruction for 16-bit and int8 operands. On gfx950 they sustain
// more throughput than the 32x32 forms under the same power limit (MFMA-only loops on random operands: bf16
// 16x16x32 0.93 of the per-clock peak at 1.71 GHz against 0.84 at 1.62 GHz for 32x32x16). Operand lane L holds row
// (or column) L & 15 and 16 bytes of K from (L >> 4) * 16; accumulator lane L holds column L & 15 of rows
// 4 (L >> 4) .. + 3.
template <int FMT>
struct Mfma16;

template <>
struct Mfma16<FMT_BF16> {
  typedef f32x4 Acc;
  __device__ static void step(Acc& c, u32x4 a, u32x4 b) {
    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0,
                                                0, 0);
  }
  // the same as assembly with the accumulator tied to one AGPR tuple (the allocator otherwise moves 4-register
  // accumulators between AGPRs and VGPRs around the loop)
  __device__ static void step_agpr(Acc& c, u32x4 a, u32x4 b) {
    asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+a"(c) : "v"(a), "v"(b));
  }
};

template <>
struct Mfma16<FMT_F16> {
  typedef f32x4 Acc;
  __device__ static void step(Acc& c, u32x4 a, u32x4 b) {
    c = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0,
                                               0);
  }
  __device__ static void step_agpr(Acc& c, u32x4 a, u32x4 b) {
    asm volatile("v_mfma_f32_16x16x32_f16 %0, %1, %2, %0" : "+a"(c) : "v"(a), "v"(b));
  }
};

template <>
struct Mfma16<FMT_I8> {
  typedef i32x4 Acc;
  __device__ static void step_agpr(Acc& c, u32x4 a, u32x4 b) {
    asm volatile("v_mfma_i32_16x16x64_i8 %0, %1, %2, %0" : "+a"(c) : "v"(a), "v"(b));
  }
};

template <>
struct Mfma16<FMT_FP8> {
  typedef f32x4 Acc;
  // v_mfma_scale_f32_16x16x128_f8f6f4 on e4m3 operands (format 0) with unit E8M0 scales (127 = 2^0, in `one`)
  __device__ static void step_agpr(Acc& c, i32x8 a, i32x8 b, int one) {
    asm volatile("v_mfma_scale_f32_16x16x128_f8f6f4 %0, %1, %2, %0, %3, %3 op_sel_hi:[0,0,0]"
                 : "+a"(c)
                 : "v"(a), "v"(b), "v"(one));
  }
};

template <typename V>
struct Elem;
template <>
struct Elem<f32x16> {
  typedef float T;
};
template <>
struct Elem<i32x16> {
  typedef int T;
};

template <typename V16, typename V4>
__device__ __forceinline__ V16 join16(const V4& s00, const V4& s01, const V4& s10, const V4& s11) {
  V16 t;
#pragma unroll
  for (int R = 0; R < 2; ++R)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t x0 = __builtin_bit_cast(uint32_t, R ? s10[q] : s00[q]);
      const uint32_t x1 = __builtin_bit_cast(uint32_t, R ? s11[q] : s01[q]);
      const auto p = __builtin_amdgcn_permlane16_swap(x0, x1, false, false);
      const auto w = __builtin_amdgcn_permlane32_swap(p[0], p[1], false, false);
      t[8 * R + q] = __builtin_bit_cast(typename Elem<V16>::T, (uint32_t)w[0]);
      t[8 * R + 4 + q] = __builtin_bit_cast(typename Elem<V16>::T, (uint32_t)w[1]);
    }
  return t;
}

// Store one 32x32 accumulator block (the C layout of a 32x32 MFMA: lane holds column lane & 31 and rows
// (r/4)*8 + (lane/32)*4 + r%4) through a per-wave LDS patch with a 36-word row stride, so that each lane then owns
// 16 consecutive elements of one row: lane l takes row l/2, columns (l&1)*16 .. +16, applies the epilogue and
// writes them with 16-byte stores. Everything indexed by the register array is unrolled, so the accumulators stay
// in registers; the patch is then read with 16-byte LDS loads.
constexpr int PATCH_STRIDE = 36;
constexpr int PATCH_WORDS = 32 * PATCH_STRIDE;

// Register half: copy one accumulator block into the wave's patch. Small and fully unrolled, so that the
// accumulator index is a constant and the accumulators never leave registers.
template <bool INT, typename V>
__device__ __forceinline__ void patch_put(const V& block, uint32_t* patch, int lane) {
  const int half = lane >> 5, r32 = lane & 31;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    if constexpr (INT)
      patch[((r >> 2) * 8 + half * 4 + (r & 3)) * PATCH_STRIDE + r32] = (uint32_t)block[r];
    else
      patch[((r >> 2) * 8 + half * 4 + (r & 3)) * PATCH_STRIDE + r32] = __float_as_uint(block[r]);
  }
}

// Entry i of a vector of float32 (`kind` 0) or 16-bit values (1 = f16, 2 = bf16) as raw bits, and their value
__device__ __forceinline__ uint32_t vec_bits(const void* v, int kind, int64_t i) {
  return kind == 0 ? static_cast<const uint32_t*>(v)[i] : static_cast<const uint16_t*>(v)[i];
}

__device__ __forceinline__ float bits_value(int kind, uint32_t b) {
  return kind == 0 ? __uint_as_float(b) : kind == 1 ? h2f((uint16_t)b) : bf2f((uint16_t)b);
}

// Columns n .. n + 7 from raw bits, zero from N on; one branch on the kind for all eight
__device__ __forceinline__ void decode8(int kind, const uint32_t* b, int64_t n, int64_t N, float* s) {
  if (kind == 0) {
#pragma unroll
    for (int c = 0; c < 8; ++c) s[c] = __uint_as_float(b[c]);
  } else if (kind == 1) {
#pragma unroll
    for (int c = 0; c < 8; ++c) s[c] = h2f((uint16_t)b[c]);
  } else {
#pragma unroll
    for (int c = 0; c < 8; ++c) s[c] = bf2f((uint16_t)b[c]);
  }
#pragma unroll
  for (int c = 0; c < 8; ++c) s[c] = n + c < N ? s[c] : 0.0f;
}

// The vector operands of a 32 x 32 block's epilogue, fetched ahead by every lane of the storing wave: for a per-row
// operation i the entry of the lane's row (row0 + lane / 2, as the memory half stores), for a per-column one the
// entry of column col0 + lane % 32. Every load is unconditional (a 32-bit and a 16-bit one per operation, the unused
// ones reading the valid address `dummy`) and only raw bits are kept, so that no branch merge or decode waits on
// these loads before the epilogue.
struct EpiPre {
  uint32_t w32[4], w16[4];
};

__device__ __forceinline__ void epi_prefetch(EpiPre& p, const Epilogue& e, const void* dummy, int64_t row0,
                                             int64_t col0, int64_t M, int64_t N, int lane) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int op = e.op[i] & ((1 << VEC_KIND_SHIFT) - 1), kind = e.op[i] >> VEC_KIND_SHIFT;
    const bool row = i < e.nops && op < RELU && op % 3 == 1, col = i < e.nops && op < RELU && op % 3 == 2;
    const int64_t at = row ? min(row0 + (lane >> 1), M - 1) : col ? min(col0 + (lane & 31), N - 1) : 0;
    p.w32[i] = static_cast<const uint32_t*>((row || col) && kind == 0 ? e.vec[i] : dummy)[(row || col) && kind == 0 ? at : 0];
    p.w16[i] = static_cast<const uint16_t*>((row || col) && kind != 0 ? e.vec[i] : dummy)[(row || col) && kind != 0 ? at : 0];
  }
}

// Memory half: the patch through the epilogue to C. ACT = false: the caller has checked that no operation is an
// activation, and their code (erff, expf and a divide for each of 16 values) stays out. PRE: the vector operands
// were fetched ahead by `epi_prefetch` (one value per lane and operation) and reach the lanes that need them by
// cross-lane permutes; the whole wave must then be active.
template <bool INT, bool ACT = true, bool PRE = false>
__device__ __forceinline__ void patch_store_inline(uint32_t* patch, void* C, int64_t ldc, int64_t row0, int64_t col0,
                                                   int64_t M, int64_t N, const Epilogue& e, int lane,
                                                   const EpiPre* pre = nullptr) {
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the patch is written before any lane reads it
  __builtin_amdgcn_wave_barrier();
  const int rr = lane >> 1, c0 = (lane & 1) * 16;
  uint32_t bits[16];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const u32x4 w = *reinterpret_cast<const u32x4*>(patch + rr * PATCH_STRIDE + c0 + 4 * q);
    bits[4 * q] = w[0], bits[4 * q + 1] = w[1], bits[4 * q + 2] = w[2], bits[4 * q + 3] = w[3];
  }
  __builtin_amdgcn_s_waitcnt(0xc07f);
  __builtin_amdgcn_wave_barrier();  // the next block may overwrite the patch
  const int64_t m = row0 + rr, n = col0 + c0;
  const bool live = m < M;
  if (!PRE && !live) return;
  const bool whole = n + 16 <= N && (ldc % 8) == 0 && (uintptr_t)C % 16 == 0;
  if (INT && e.out_kind == I32) {
    if (!live) return;
    int32_t* out = static_cast<int32_t*>(C) + m * ldc + n;
    if (whole && (ldc % 4) == 0) {
#pragma unroll
      for (int q = 0; q < 4; ++q)
        reinterpret_cast<u32x4*>(out)[q] = u32x4{bits[4 * q], bits[4 * q + 1], bits[4 * q + 2], bits[4 * q + 3]};
    } else {
      for (int c = 0; c < 16 && n + c < N; ++c) out[c] = (int32_t)bits[c];
    }
    return;
  }
  float v[16];
#pragma unroll
  for (int c = 0; c < 16; ++c) v[c] = INT ? (float)(int32_t)bits[c] : __uint_as_float(bits[c]);
  auto apply = [&](int i, auto row_value, auto col_values) {
    const int op = e.op[i] & ((1 << VEC_KIND_SHIFT) - 1);
    if (op >= RELU) {
      if constexpr (ACT) {
#pragma unroll
        for (int c = 0; c < 16; ++c) v[c] = activation(op, v[c]);
      }
    } else if (op % 3 == 0) {
#pragma unroll
      for (int c = 0; c < 16; ++c) v[c] = op < 3 ? __fmul_rn(v[c], e.scalar[i]) : __fadd_rn(v[c], e.scalar[i]);
    } else if (op % 3 == 1) {
      const float s = row_value();
#pragma unroll
      for (int c = 0; c < 16; ++c) v[c] = op < 3 ? __fmul_rn(v[c], s) : __fadd_rn(v[c], s);
    } else {
#pragma unroll
      for (int h = 0; h < 2; ++h) {  // eight columns at a time keeps the store's register use small
        float s[8];
        col_values(s, h * 8);
#pragma unroll
        for (int c = 0; c < 8; ++c)
          v[h * 8 + c] = op < 3 ? __fmul_rn(v[h * 8 + c], s[c]) : __fadd_rn(v[h * 8 + c], s[c]);
      }
    }
  };
  if constexpr (PRE) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (i < e.nops) {
        const int kind = e.op[i] >> VEC_KIND_SHIFT;
        const uint32_t mine = kind == 0 ? pre->w32[i] : pre->w16[i];
        apply(i, [&] { return bits_value(kind, mine); }, [&](float* s, int c8) {
          uint32_t b[8];  // column n + c was fetched by lane c0 + c; all permutes out before any result is used
#pragma unroll
          for (int c = 0; c < 8; ++c) b[c] = (uint32_t)__shfl((int)mine, c0 + c8 + c);
          decode8(kind, b, n + c8, N, s);
        });
      }
    }
    if (!live) return;
  } else {
    for (int i = 0; i < e.nops; ++i) {
      const int kind = e.op[i] >> VEC_KIND_SHIFT;
      apply(i, [&] { return bits_value(kind, vec_bits(e.vec[i], kind, m)); }, [&](float* s, int c8) {
        uint32_t b[8];  // clamped indices: the loads issue back to back
#pragma unroll
        for (int c = 0; c < 8; ++c) b[c] = vec_bits(e.vec[i], kind, min(n + c8 + c, N - 1));
        decode8(kind, b, n + c8, N, s);
      });
    }
  }
  if (e.out_kind == F32) {
    float* out = static_cast<float*>(C) + m * ldc + n;
    if (whole) {
#pragma unroll
      for (int q = 0; q < 4; ++q)
        reinterpret_cast<f32x4*>(out)[q] = f32x4{v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]};
    } else {
      for (int c = 0; c < 16 && n + c < N; ++c) out[c] = v[c];
    }
    return;
  }
  uint32_t h[8];
#pragma unroll
  for (int c = 0; c < 8; ++c)
    h[c] = e.out_kind == BF16 ? f2bf2(v[2 * c], v[2 * c + 1])
                              : ((uint32_t)f2h(v[2 * c]) | ((uint32_t)f2h(v[2 * c + 1]) << 16));
  uint16_t* out = static_cast<uint16_t*>(C) + m * ldc + n;
  if (whole) {
    // C is written once and not read here: non-temporal stores keep it from displacing operand panels in L2
    // (bf16 8192^3 +0.3 %, fp8 +1.5 %, bf16 M = 4096 +2 %)
    __builtin_nontemporal_store(u32x4{h[0], h[1], h[2], h[3]}, reinterpret_cast<u32x4*>(out));
    __builtin_nontemporal_store(u32x4{h[4], h[5], h[6], h[7]}, reinterpret_cast<u32x4*>(out) + 1);
  } else {
    for (int c = 0; c < 16 && n + c < N; ++c) out[c] = (uint16_t)(h[c >> 1] >> ((c & 1) * 16));
  }
}

template <bool INT>
__device__ __noinline__ void patch_store(uint32_t* patch, void* C, int64_t ldc, int64_t row0, int64_t col0, int64_t M,
                                         int64_t N, const Epilogue& e, int lane) {
  patch_store_inline<INT>(patch, C, ldc, row0, col0, M, N, e, lane);
}

// One accumulator block to C through the out-of-line store: the tiles' loops over their blocks must unroll
// completely, and an inlined store in each copy would not fit. (The skinny kernel, with at most four blocks and the
// vectors fetched ahead, inlines the store instead.)
template <bool INT, typename V>
__device__ __forceinline__ void store_block(const V& block, uint32_t* patch, void* C, int64_t ldc, int64_t row0,
                                            int64_t col0, int64_t M, int64_t N, const Epilogue& e, int lane) {
  patch_put<INT>(block, patch, lane);
  patch_store<INT>(patch, C, ldc, row0, col0, M, N, e, lane);
}

// The direct epilogue: whole 32 x 32 blocks straight from the MFMA accumulator layout to 16-bit C, without the LDS
// patch, for epilogues of at most two operations that are float32 scalars or row/column vectors (no activation):
// the headline bf16 product, the fp8 product's `acc * (scale_a * scale_b)`, the W8A8 dequantisation
// `acc * scale_a[m] * scale_w[n]`. Lane L holds column c = L & 31 at rows R(r) = (r / 4) * 8 + (L / 32) * 4 + r % 4;
// neighbouring lanes hold columns c and c ^ 1 of the same rows. The operations and their rounding are the patch
// path's, so the result is the same bit for bit.
constexpr int DIRECT_OPS = 2;

__device__ __forceinline__ bool direct_epilogue(const Epilogue& e) {
  if (e.out_kind != BF16 && e.out_kind != F16) return false;
  if (e.nops > DIRECT_OPS) return false;
  for (int i = 0; i < e.nops; ++i)
    if ((e.op[i] & ((1 << VEC_KIND_SHIFT) - 1)) >= RELU) return false;
  return true;
}

// The vector operands of a wave's TM x TN blocks, fetched for all blocks at once before any is stored: for a per-row
// operation the 16 rows R(r) of each row block, for a per-column one the lane's column of each column block.
template <int TM, int TN>
struct DirectVectors {
  float row[DIRECT_OPS][TM][16];
  float col[DIRECT_OPS][TN];
};

template <int TM, int TN>
__device__ __forceinline__ void direct_vectors(DirectVectors<TM, TN>& dv, const Epilogue& e, int64_t row0,
                                               int64_t col0, int lane) {
  const int c = lane & 31, half = lane >> 5;
#pragma unroll
  for (int q = 0; q < DIRECT_OPS; ++q) {
    if (q >= e.nops) break;
    const int op = e.op[q] & ((1 << VEC_KIND_SHIFT) - 1), kind = e.op[q] >> VEC_KIND_SHIFT;
    // every element is assigned on every path, so the arrays stay in registers
    const bool per_row = op % 3 == 1, per_col = op % 3 == 2;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        dv.row[q][i][r] =
            per_row ? bits_value(kind, vec_bits(e.vec[q], kind, row0 + i * 32 + (r >> 2) * 8 + half * 4 + (r & 3)))
                    : 0.0f;
#pragma unroll
    for (int j = 0; j < TN; ++j)
      dv.col[q][j] = per_col ? bits_value(kind, vec_bits(e.vec[q], kind, col0 + j * 32 + c)) : 0.0f;
  }
}

// One block's 16 accumulators through the epilogue operations, in float32 (the patch path's operations and
// rounding).
template <bool INT, int TM, int TN, typename V>
__device__ __forceinline__ void direct_ops(float (&v)[16], const V& block, const DirectVectors<TM, TN>& dv, int i,
                                           int j, const Epilogue& e) {
#pragma unroll
  for (int r = 0; r < 16; ++r) v[r] = INT ? (float)(int32_t)block[r] : (float)block[r];
#pragma unroll
  for (int q = 0; q < DIRECT_OPS; ++q) {
    if (q >= e.nops) break;
    const int op = e.op[q] & ((1 << VEC_KIND_SHIFT) - 1);
    const bool mul = op < 3;
    if (op % 3 == 0) {
      const float s = e.scalar[q];
#pragma unroll
      for (int r = 0; r < 16; ++r) v[r] = mul ? __fmul_rn(v[r], s) : __fadd_rn(v[r], s);
    } else if (op % 3 == 1) {
#pragma unroll
      for (int r = 0; r < 16; ++r) v[r] = mul ? __fmul_rn(v[r], dv.row[q][i][r]) : __fadd_rn(v[r], dv.row[q][i][r]);
    } else {
      const float s = dv.col[q][j];
#pragma unroll
      for (int r = 0; r < 16; ++r) v[r] = mul ? __fmul_rn(v[r], s) : __fadd_rn(v[r], s);
    }
  }
}

// One block (i, j): one DPP swap per register pair (2k, 2k + 1) gives the even lane both columns c, c + 1 of row
// R(2k) and the odd lane both of row R(2k + 1); each store instruction writes 64-byte row segments (half lines).
template <bool INT, bool BF, int TM, int TN, typename V>
__device__ __forceinline__ void store_block_direct(const V& block, const DirectVectors<TM, TN>& dv, int i, int j,
                                                   __amdgpu_buffer_rsrc_t out, uint32_t lane_off, int64_t ldc,
                                                   const Epilogue& e, int lane) {
  float v[16];
  direct_ops<INT>(v, block, dv, i, j, e);
  const int odd = lane & 1;
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const float send = odd ? v[2 * k] : v[2 * k + 1];
    const float recv = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(send), 0xB1, 0xF, 0xF, true));
    const float lo = odd ? recv : v[2 * k], hi = odd ? v[2 * k + 1] : recv;
    const uint32_t pair = BF ? f2bf2(lo, hi) : ((uint32_t)f2h(lo) | ((uint32_t)f2h(hi) << 16));
    // register 2k + odd holds row ((2k + odd) >> 2) * 8 + half * 4 + ((2k + odd) & 3): the lane's part
    // (half * 4 + odd) is in lane_off, the rest is a scalar offset
    const int step = (k >> 1) * 8 + (k & 1) * 2 + i * 32;
    const int soff = __builtin_amdgcn_readfirstlane((int)(((int64_t)step * ldc + j * 32) * 2));
    __builtin_amdgcn_raw_buffer_store_b32(pair, out, (int)lane_off, soff, 2 /* nt */);
  }
}

// A wave's TM x TN accumulator blocks to C. When the wave's whole region lies inside C and the epilogue is one the
// direct path takes, every block goes straight from registers; otherwise each block goes through the LDS patch (all
// operations, ragged edges, int32 and float32 outputs).

// A block of accumulators held in AGPRs (the four-wave loop's 256 of them), copied to VGPRs right before it is
// stored, by ordered reads; left to itself the compiler copies all of them at the end of the loop and spills most of
// them to private memory.
template <typename V>
__device__ __forceinline__ V agpr_block(const V& x) {
  V y;
#pragma unroll
  for (int r = 0; r < (int)(sizeof(V) / 4); ++r)
    asm volatile("v_accvgpr_read_b32 %0, %1" : "=v"(y[r]) : "a"(x[r]) : "memory");
  return y;
}

// `fetch(i, j)` hands over block (i, j) in the 32x32 accumulator layout.
template <bool INT, int TM, int TN, typename Fetch>
__device__ __forceinline__ void store_tile_by(Fetch fetch, uint32_t* patch, void* C, int64_t ldc, int64_t row0,
                                              int64_t col0, int64_t M, int64_t N, const Epilogue& e, int lane) {
  const bool direct = direct_epilogue(e) && (ldc % 2) == 0 && (uintptr_t)C % 4 == 0 && row0 + 32 * TM <= M &&
                      col0 + 32 * TN <= N && (int64_t)32 * TM * ldc * 2 <= 0x7fffffff;
  if (direct) {
    DirectVectors<TM, TN> dv;
    direct_vectors(dv, e, row0, col0, lane);
    // the wave's region of C as a buffer resource; each lane stores a column pair at (c & ~1) of rows
    // half * 4 + odd, plus wave-uniform steps
    const int c = lane & 31;
    // (readfirstlane returns int: each word goes through uint32_t, so the low word is never sign-extended into
    // the high one)
    const uint64_t base = (uint64_t)(static_cast<uint16_t*>(C) + row0 * ldc + col0);
    const uint32_t base_lo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)base);
    const uint32_t base_hi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(base >> 32));
    const void* region = (const void*)(((uint64_t)base_hi << 32) | (uint64_t)base_lo);
    const __amdgpu_buffer_rsrc_t out = panel_rsrc(region, (int64_t)32 * TM * ldc * 2);
    // block by block: row half * 4 + (c & 1), column pair c & ~1 (measured 3 % faster for W8A8 on the eight-wave
    // int8 loop, whose registers are tighter, than pairs of blocks stored as whole lines)
    const uint32_t lane_off = (uint32_t)((((lane >> 5) * 4 + (c & 1)) * ldc + (c & ~1)) * 2);
#define KRN_DIRECT(BF)                                                                                       \
  _Pragma("unroll") for (int i = 0; i < TM; ++i) _Pragma("unroll") for (int j = 0; j < TN; ++j)              \
      store_block_direct<INT, BF>(fetch(i, j), dv, i, j, out, lane_off, ldc, e, lane);
    if (e.out_kind == BF16) {
      KRN_DIRECT(true)
    } else {
      KRN_DIRECT(false)
    }
#undef KRN_DIRECT
    return;
  }
  // The out-of-line store takes the epilogue by address. Passing the kernel argument itself would copy it to private
  // memory at kernel entry, in every wave, whichever path the wave takes (80 bytes a lane, 42 MB per bf16 8192^3
  // launch); this copy is made only on this path.
  const Epilogue local = e;
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) store_block<INT>(fetch(i, j), patch, C, ldc, row0 + i * 32, col0 + j * 32, M, N, local, lane);
}

template <bool INT, int TM, int TN, typename Acc>
__device__ __forceinline__ void store_tile(const Acc (&acc)[TM][TN], uint32_t* patch, void* C, int64_t ldc,
                                           int64_t row0, int64_t col0, int64_t M, int64_t N, const Epilogue& e,
                                           int lane) {
  store_tile_by<INT, TM, TN>([&](int i, int j) { return acc[i][j]; }, patch, C, ldc, row0, col0, M, N, e, lane);
}

// Register half of the patch path for a block held transposed: `block` is the 32x32 accumulator layout of the
// transpose of a C block (lane holds C row lane & 31 and C columns (r/4)*8 + (lane/32)*4 + r%4), written into the
// patch in C's row-major order.
template <bool INT, typename V>
__device__ __forceinline__ void patch_put_t(const V& block, uint32_t* patch, int lane) {
  const int half = lane >> 5, r32 = lane & 31;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const uint32_t bits = INT ? (uint32_t)block[r] : __float_as_uint(block[r]);
    patch[r32 * PATCH_STRIDE + (r >> 2) * 8 + half * 4 + (r & 3)] = bits;
  }
}

// The four-wave loop's 8 x 8 blocks of 16 x 16, computed transposed (B A^T, so that C's rows lie along the lanes):
// lane L of block (i, j) holds row 16 i + (L & 15) of the wave's 128 x 128 region and its columns
// 16 j + 4 (L >> 4) .. + 3, one per register. The four lanes L & 15 + 16 s that share a row exchange 8-byte pieces
// (two permlane swaps per word), so that each holds 16 contiguous columns of one block and writes them as two
// 16-byte pieces: per store instruction 64 bytes of each of 16 rows. The untransposed 32x32 layout needs a DPP
// exchange and three selects per register for whole-line pieces; 8-byte pieces without the exchange were slower
// (quarter lines). `ops` applies the epilogue's operations to one block's four values (Quad16Generic,
// Quad16RowCol below), with the patch path's rounding. 32-bit outputs have their own direct store
// (store32t_direct); everything else (ragged edges, activations, more than two operations) goes through the patch:
// four blocks are joined into the 32x32 layout of the transposed block and written into the patch transposed.
// Against the 32x32 direct store (same box, bench legs): bf16 8192^3 equal, fp8 8192^3 0.440 -> 0.424 ms,
// W8A8 M = 4096 0.272 -> 0.247 ms; write-back instead of non-temporal stores: bf16 1.5 % slower.
template <bool INT, bool BF, typename V4, typename Ops>
__device__ __forceinline__ void store16t_direct(const V4 (&acc)[8][8], Ops ops, void* C, int64_t ldc, int64_t row0,
                                                int64_t col0, int lane) {
  const int r16 = lane & 15, g = lane >> 4;
  const uint64_t base = (uint64_t)(static_cast<uint16_t*>(C) + row0 * ldc + col0);
  const uint32_t base_lo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)base);
  const uint32_t base_hi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(base >> 32));
  const void* region = (const void*)(((uint64_t)base_hi << 32) | (uint64_t)base_lo);
  const __amdgpu_buffer_rsrc_t out = panel_rsrc(region, (int64_t)128 * ldc * 2);
  // after the exchange below, lane group g holds the 16 columns of block 4 jj + g of its row: two 16-byte pieces
  const uint32_t lane_off = (uint32_t)((r16 * ldc + 16 * g) * 2);
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      uint32_t w[4][2];  // [block jb][word]: columns 16 (4 jj + jb) + 4 g + 2 word .. + 1
#pragma unroll
      for (int jb = 0; jb < 4; ++jb) {
        const int j = 4 * jj + jb;
        const V4 b = agpr_block(acc[i][j]);
        float v[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) v[c] = INT ? (float)(int32_t)b[c] : (float)b[c];
        ops(v, i, j);
        w[jb][0] = BF ? f2bf2(v[0], v[1]) : ((uint32_t)f2h(v[0]) | ((uint32_t)f2h(v[1]) << 16));
        w[jb][1] = BF ? f2bf2(v[2], v[3]) : ((uint32_t)f2h(v[2]) | ((uint32_t)f2h(v[3]) << 16));
      }
      // a 4 x 4 transpose of 8-byte pieces over the four lane groups (16-lane rows) that share a C row: piece
      // (group s, block jb) goes to group jb, slot s. permlane16_swap(x, y) leaves [x0 y0 x2 y2] in x and
      // [x1 y1 x3 y3] in y (16-lane rows), permlane32_swap(x, y) [x0 x1 y0 y1] and [x2 x3 y2 y3].
      uint32_t t[4][2];  // [slot s][word]: columns 16 (4 jj + g) + 4 s + 2 word .. + 1
#pragma unroll
      for (int x = 0; x < 2; ++x) {
        const auto p01 = __builtin_amdgcn_permlane16_swap(w[0][x], w[1][x], false, false);
        const auto p23 = __builtin_amdgcn_permlane16_swap(w[2][x], w[3][x], false, false);
        const auto q02 = __builtin_amdgcn_permlane32_swap(p01[0], p23[0], false, false);
        const auto q13 = __builtin_amdgcn_permlane32_swap(p01[1], p23[1], false, false);
        t[0][x] = q02[0];
        t[2][x] = q02[1];
        t[1][x] = q13[0];
        t[3][x] = q13[1];
      }
      const int soff = __builtin_amdgcn_readfirstlane((int)(((int64_t)16 * i * ldc + 64 * jj) * 2));
      __builtin_amdgcn_raw_buffer_store_b128(u32x4{t[0][0], t[0][1], t[1][0], t[1][1]}, out, (int)lane_off, soff,
                                             2 /* nt */);
      __builtin_amdgcn_raw_buffer_store_b128(u32x4{t[2][0], t[2][1], t[3][0], t[3][1]}, out, (int)lane_off + 16,
                                             soff, 2 /* nt */);
    }
}

// The direct store's operations on one block's four values (row 16 i + (lane & 15), columns 16 j + 4 (lane >> 4)
// + c). Generic: any chain of at most two scalar, row and column multiplies and adds, as two fused multiply-adds
// each (x * s + (-0) = x * s or x * 1 + s = x + s, and the identity x * 1 + (-0) for the other of the pair: each exact
// or rounded once, signed zeros included, so the result is the patch path's bit for bit).
struct Quad16Generic {
  float rm[DIRECT_OPS][8], ra[DIRECT_OPS][8], cm[DIRECT_OPS][8][4], ca[DIRECT_OPS][8][4];
  int nops;
  __device__ void operator()(float (&v)[4], int i, int j) const {
#pragma unroll
    for (int q = 0; q < DIRECT_OPS; ++q) {
      if (q >= nops) break;
#pragma unroll
      for (int c = 0; c < 4; ++c)
        v[c] = __builtin_fmaf(__builtin_fmaf(v[c], rm[q][i], ra[q][i]), cm[q][j][c], ca[q][j][c]);
    }
  }
};

__device__ __forceinline__ void quad16_generic(Quad16Generic& qv, const Epilogue& e, int64_t row0, int64_t col0,
                                               int lane) {
  const int r16 = lane & 15, g = lane >> 4;
  qv.nops = e.nops;
  // per operation: the multiplier and addend of a fused multiply-add per row block (row and scalar operations) and
  // per column of each column block (column operations); the other of the two is the identity x * 1 + (-0), exact
  // for every x, so each operation is two fused multiply-adds and no selection
#pragma unroll
  for (int q = 0; q < DIRECT_OPS; ++q) {
    if (q >= e.nops) break;
    const int op = e.op[q] & ((1 << VEC_KIND_SHIFT) - 1), kind = e.op[q] >> VEC_KIND_SHIFT;
    const bool mul = op < 3, col = op % 3 == 2;
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const float s = col ? bits_value(kind, vec_bits(e.vec[q], kind, col0 + 16 * j + 4 * g + c)) : 0.0f;
        qv.cm[q][j][c] = col && mul ? s : 1.0f;
        qv.ca[q][j][c] = col && !mul ? s : -0.0f;
      }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float s = col ? 0.0f
                          : op % 3 == 1 ? bits_value(kind, vec_bits(e.vec[q], kind, row0 + 16 * i + r16)) : e.scalar[q];
      qv.rm[q][i] = !col && mul ? s : 1.0f;
      qv.ra[q][i] = !col && !mul ? s : -0.0f;
    }
  }
}

// W8A8's dequantisation `acc * scale_a[m] * scale_w[n]` (a row multiply, then a column multiply, float32 vectors):
// the lane's 8 row and 32 column values, fetched before the loop's last slices, and two multiplies per value.
struct Quad16RowCol {
  float r[8], c[8][4];
  __device__ void operator()(float (&v)[4], int i, int j) const {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      v[q] = __fmul_rn(__fmul_rn(v[q], r[i]), c[j][q]);
      // opaque to the compiler, which would otherwise fuse the last multiply into the f16 conversion (a mixed
      // multiply-add with a +0 addend, rounded once: -0 becomes +0 and the float32 rounding is skipped)
      asm("" : "+v"(v[q]));
    }
  }
};

__device__ __forceinline__ bool quad16_is_rowcol(const Epilogue& e) {
  return e.nops == 2 && e.op[0] == MUL_ROW && e.op[1] == MUL_COL;  // kind 0: float32 vectors
}

__device__ __forceinline__ void quad16_rowcol(Quad16RowCol& rc, const Epilogue& e, int64_t row0, int64_t col0,
                                              int lane) {
  const int r16 = lane & 15, g = lane >> 4;
  const float* rv = static_cast<const float*>(e.vec[0]);
  const float* cv = static_cast<const float*>(e.vec[1]);
#pragma unroll
  for (int i = 0; i < 8; ++i) rc.r[i] = rv[row0 + 16 * i + r16];
#pragma unroll
  for (int j = 0; j < 8; ++j)
#pragma unroll
    for (int c = 0; c < 4; ++c) rc.c[j][c] = cv[col0 + 16 * j + 4 * g + c];
}

// Whether a wave's 128 x 128 region at (row0, col0) takes the direct store.
__device__ __forceinline__ bool quad16_direct(const Epilogue& e, const void* C, int64_t ldc, int64_t row0,
                                              int64_t col0, int64_t M, int64_t N) {
  return direct_epilogue(e) && (ldc % 4) == 0 && (uintptr_t)C % 8 == 0 && row0 + 128 <= M && col0 + 128 <= N &&
         (int64_t)128 * ldc * 2 <= 0x7fffffff;
}

// 32-bit outputs (int32 from an int8 product with no operations, float32 with at most two scalar, row and column
// operations) of the transposed blocks: a lane's four values are 16 contiguous bytes of one row, so each block is
// one 16-byte store per lane (64 bytes of each of 16 rows per instruction), no exchange between lanes.
__device__ __forceinline__ bool quad16_direct32(const Epilogue& e, const void* C, int64_t ldc, int64_t row0,
                                                int64_t col0, int64_t M, int64_t N) {
  bool ops_ok = e.nops <= DIRECT_OPS;
  for (int i = 0; i < e.nops; ++i) ops_ok &= (e.op[i] & ((1 << VEC_KIND_SHIFT) - 1)) < RELU;
  const bool kind = (e.out_kind == I32 && e.nops == 0) || (e.out_kind == F32 && ops_ok);
  return kind && (ldc % 4) == 0 && (uintptr_t)C % 16 == 0 && row0 + 128 <= M && col0 + 128 <= N &&
         (int64_t)128 * ldc * 4 <= 0x7fffffff;
}

template <bool INT, typename V4, typename Ops>
__device__ __forceinline__ void store32t_direct(const V4 (&acc)[8][8], Ops ops, bool raw_int, void* C, int64_t ldc,
                                                int64_t row0, int64_t col0, int lane) {
  const int r16 = lane & 15, g = lane >> 4;
  const uint64_t base = (uint64_t)(static_cast<uint32_t*>(C) + row0 * ldc + col0);
  const uint32_t base_lo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)base);
  const uint32_t base_hi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(base >> 32));
  const void* region = (const void*)(((uint64_t)base_hi << 32) | (uint64_t)base_lo);
  const __amdgpu_buffer_rsrc_t out = panel_rsrc(region, (int64_t)128 * ldc * 4);
  const uint32_t lane_off = (uint32_t)((r16 * ldc + 4 * g) * 4);
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const V4 b = agpr_block(acc[i][j]);
      u32x4 w;
      if (INT && raw_int) {
#pragma unroll
        for (int c = 0; c < 4; ++c) w[c] = (uint32_t)b[c];
      } else {
        float v[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) v[c] = INT ? (float)(int32_t)b[c] : (float)b[c];
        ops(v, i, j);
#pragma unroll
        for (int c = 0; c < 4; ++c) w[c] = __float_as_uint(v[c]);
      }
      const int soff = __builtin_amdgcn_readfirstlane((int)(((int64_t)16 * i * ldc + 16 * j) * 4));
      __builtin_amdgcn_raw_buffer_store_b128(w, out, (int)lane_off, soff, 2 /* nt */);
    }
}

// `direct`: quad16_direct of the region; `rowcol`: the epilogue is W8A8's, with its vectors already in `rc`.
template <bool INT, typename V16, typename V4>
__device__ __forceinline__ void store_tile16t(const V4 (&acc)[8][8], bool direct, bool rowcol,
                                              const Quad16RowCol& rc, uint32_t* patch, void* C, int64_t ldc,
                                              int64_t row0, int64_t col0, int64_t M, int64_t N, const Epilogue& e,
                                              int lane) {
  if (direct) {
    const bool bf = e.out_kind == BF16;
    if (rowcol) {
      if (bf) store16t_direct<INT, true>(acc, rc, C, ldc, row0, col0, lane);
      else store16t_direct<INT, false>(acc, rc, C, ldc, row0, col0, lane);
    } else {
      Quad16Generic qv;
      quad16_generic(qv, e, row0, col0, lane);
      if (bf) store16t_direct<INT, true>(acc, qv, C, ldc, row0, col0, lane);
      else store16t_direct<INT, false>(acc, qv, C, ldc, row0, col0, lane);
    }
    return;
  }
  if (quad16_direct32(e, C, ldc, row0, col0, M, N)) {
    Quad16Generic qv;
    quad16_generic(qv, e, row0, col0, lane);
    store32t_direct<INT>(acc, qv, e.out_kind == I32, C, ldc, row0, col0, lane);
    return;
  }
  const Epilogue local = e;  // taken by address by the out-of-line store
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      // the transposed 32x32 block's quarter (h, k) is the transpose of C's quarter (k, h)
      const V16 blk = join16<V16>(agpr_block(acc[2 * i][2 * j]), agpr_block(acc[2 * i + 1][2 * j]),
                                  agpr_block(acc[2 * i][2 * j + 1]), agpr_block(acc[2 * i + 1][2 * j + 1]));
      patch_put_t<INT>(blk, patch, lane);
      patch_store<INT>(patch, C, ldc, row0 + 32 * i, col0 + 32 * j, M, N, local, lane);
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

// LDS swizzles. gfx950's LDS serves 16 lanes of a 16-byte read per cycle from 64 banks (256 bytes), so the 16
// rows a read touches must land on 16 different 16-byte positions modulo 256 bytes. With 128-byte rows (8 chunks)
// rows of equal parity share a window half, so chunk c of row r goes to slot c ^ ((r >> 1) & 7); with 64-byte rows
// (4 chunks) rows of equal r & 3 share a quarter, so slot c ^ ((r >> 2) & 3).
__device__ __forceinline__ int swz8(int row) { return (row >> 1) & 7; }
__device__ __forceinline__ int swz4(int row) { return (row >> 2) & 3; }

// Tile index of this workgroup. Workgroups are dispatched round-robin over the 8 XCDs, so consecutive ids are
// first regrouped per XCD (each XCD gets one contiguous range of tiles and its own L2 sees a compact panel), then
// ordered in groups of GROUP_M tile rows so neighbours share A rows and B columns.
__device__ __forceinline__ void tile_of(int tiles_m, int tiles_n, int& tm, int& tn) {
#ifndef KRN_GROUP_M
#define KRN_GROUP_M 4
#endif
#ifndef KRN_XCD_REMAP
#define KRN_XCD_REMAP 1
#endif
  constexpr int GROUP_M = KRN_GROUP_M;  // bf16 8192^3, eight-wave ring: 0.5-1.5 % faster than 8 (2: -6 %, 6: -1 %,
                                        // 16: -9 %); fp8 equal; four-wave register-staged 32x32 loop: 8 equal, 2
                                        // -1.5 % (1.5 times the bytes read)
  int nb = tiles_m * tiles_n;
  int bid = blockIdx.x;
  if (KRN_XCD_REMAP && nb % 8 == 0) bid = (bid % 8) * (nb / 8) + bid / 8;
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
      lds[s][row * 8 + (lchunk ^ swz8(row))] = ra[p];                                                           \
    }                                                                                                           \
    _Pragma("unroll") for (int p = 0; p < PB; ++p) {                                                            \
      const int row = BM + lrow + 32 * p;                                                                       \
      lds[s][row * 8 + (lchunk ^ swz8(row))] = rb[p];                                                           \
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
          fa[i][c] = lds[s][row * 8 + (chunk ^ swz8(row))];
        }
      }
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int row = BM + wn * (BN / WN) + j * 32 + r32;
#pragma unroll
        for (int c = 0; c < CH; ++c) {
          const int chunk = (k * STEP + half * (STEP / 2)) / 16 + c;
          fb[j][c] = lds[s][row * 8 + (chunk ^ swz8(row))];
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
  uint32_t* patch = reinterpret_cast<uint32_t*>(&lds[0][0]) + wave * PATCH_WORDS;
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
      store_block<FMT == FMT_I8>(acc[i][j], patch, C, ldc, m0 + wm * (BM / WM) + i * 32,
                                 n0 + wn * (BN / WN) + j * 32, M, N, e, lane);
}

// The pipelined main loop for 256 x 256 tiles (the last row and column of tiles may be ragged; K a multiple of the
// BKB-byte slice, rows 16-byte aligned). Operand slices go straight from global memory into LDS (global_load_lds_dwordx4, no register staging)
// through a ring of STAGES buffers, so the loads of slice k + STAGES - 1 are in flight while slice k multiplies.
// One barrier per slice publishes the landed slice and frees the oldest buffer; it is a bare s_barrier, because the
// workgroup fence of __syncthreads() would wait for every outstanding load and drain the ring. A wave's load
// instruction fills 1 KiB of LDS contiguously (lane i -> slot i), so each lane fetches the global chunk that belongs
// at its swizzled slot. Fragments are double-buffered in registers: the LDS reads of step s + 1 (and, at the end of
// a slice, of the next slice) are issued before the MFMAs of step s, and the scheduler is told to interleave one
// LDS read or one global load with each MFMA, so the memory instructions issue in the shadow of the matrix core.
template <int BKB>
__device__ __forceinline__ int swzk(int row) {
  return BKB == 128 ? swz8(row) : swz4(row);
}

template <int FMT, int BM, int BN, int WM, int WN, int STAGES, int BKB>
__global__ __launch_bounds__(WM * WN * 64, 1) void gemm_pipe(const uint8_t* __restrict__ A,
                                                             const uint8_t* __restrict__ B, void* __restrict__ C,
                                                             int64_t M, int64_t N, int64_t kbytes, int64_t lda,
                                                             int64_t ldb, int64_t ldc, Epilogue e) {
  typedef Mfma<FMT> Unit;
  typedef typename Unit::Acc Acc;
  constexpr int THREADS = WM * WN * 64;
  constexpr int CPR = BKB / 16;              // 16-byte chunks per row
  constexpr int TM = BM / WM / 32, TN = BN / WN / 32;
  constexpr int STEP = Unit::kBytes;         // bytes of K per MFMA
  constexpr int CH = STEP / 32;              // 16-byte chunks per lane per MFMA operand
  constexpr int KS = BKB / STEP;             // MFMA steps per slice
  constexpr int ROWS_PER_LOAD = 1024 / BKB;  // rows one wave load instruction fills
  constexpr int LOADS_A = BM / ROWS_PER_LOAD / (THREADS / 64), LOADS_B = BN / ROWS_PER_LOAD / (THREADS / 64);
  constexpr int LOADS = LOADS_A + LOADS_B;   // load instructions per wave per slice
  constexpr int STAGE_BYTES = (BM + BN) * BKB;
  constexpr int VMCNT = (STAGES - 2) * LOADS;
  // With three or more stages the A loads of a slice go between the first MFMAs and the B loads between the MFMAs
  // after the barrier, one load every four MFMAs: the workgroup's 32 loads of a slice no longer arrive at the
  // texture unit as one burst (bf16 8192^3 +2.5 %). At the barrier of slice kt the loads younger than slice kt + 1
  // are then slices kt + 2 .. kt + STAGES - 2 and the A loads of slice kt + STAGES - 1.
  constexpr bool SPREAD = STAGES >= 3;
  constexpr int VMCNT_SPLIT = SPREAD ? (STAGES - 3) * LOADS + LOADS_A : VMCNT;
  static_assert(KS % 2 == 0, "an even number of MFMA steps per slice");
  static_assert(LOADS_A * ROWS_PER_LOAD * (THREADS / 64) == BM && LOADS_B * ROWS_PER_LOAD * (THREADS / 64) == BN,
                "the tile splits into whole wave loads");
  static_assert(VMCNT <= 63, "vmcnt range");
  static_assert(STAGES * STAGE_BYTES <= 160 * 1024, "LDS of one CU");
  __shared__ __attribute__((aligned(1024))) uint8_t lds[STAGES * STAGE_BYTES];

  int tm, tn;
  tile_of((int)((M + BM - 1) / BM), (int)((N + BN - 1) / BN), tm, tn);
  const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
  const int t = threadIdx.x, lane = t & 63, wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int wm = wave / WN, wn = wave % WN;
  const int half = lane >> 5, r32 = lane & 31;

  // this lane's share of each wave load: its row within the 1 KiB block and the global chunk for its slot. Loads go
  // through buffer resources over this tile's A and B panels (base in SGPRs): a lane keeps one 32-bit panel offset
  // per load and the slice offset is an SGPR, so no address arithmetic runs per load (the host routes a tile here
  // only when its panel offsets fit in 31 bits). A panel's resource ends at the operand's last row: rows of a
  // ragged last tile past it load zeros, and their results are never stored.
  const int lrow = lane / CPR, lslot = lane % CPR;
  const __amdgpu_buffer_rsrc_t a_rsrc = panel_rsrc(A + m0 * lda, (M - m0) * lda),
                              b_rsrc = panel_rsrc(B + n0 * ldb, (N - n0) * ldb);
  uint32_t a_off_g[LOADS_A], b_off_g[LOADS_B];
#pragma unroll
  for (int j = 0; j < LOADS_A; ++j) {
    const int row = (wave * LOADS_A + j) * ROWS_PER_LOAD + lrow;
    a_off_g[j] = (uint32_t)(row * lda + (lslot ^ swzk<BKB>(row)) * 16);
  }
#pragma unroll
  for (int j = 0; j < LOADS_B; ++j) {
    const int row = (wave * LOADS_B + j) * ROWS_PER_LOAD + lrow;
    b_off_g[j] = (uint32_t)(row * ldb + (lslot ^ swzk<BKB>(row)) * 16);
  }
  // fragment offsets (16-byte units within a stage) of every MFMA operand this lane reads
  int a_off[TM][KS][CH], b_off[TN][KS][CH];
#pragma unroll
  for (int k = 0; k < KS; ++k)
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const int chunk = (k * STEP + half * (STEP / 2)) / 16 + c;
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int row = wm * (BM / WM) + i * 32 + r32;
        a_off[i][k][c] = row * CPR + (chunk ^ swzk<BKB>(row));
      }
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int row = wn * (BN / WN) + j * 32 + r32;
        b_off[j][k][c] = BM * CPR + row * CPR + (chunk ^ swzk<BKB>(row));
      }
    }
  const int nk = (int)(kbytes / BKB);

#define KRN_ISSUE(slice)                                                                                        \
  do {                                                                                                          \
    uint8_t* stage = lds + ((slice) % STAGES) * STAGE_BYTES;                                                    \
    const int koff = (slice) * BKB;                                                                             \
    _Pragma("unroll") for (int j = 0; j < LOADS_A; ++j)                                                         \
        buffer_to_lds16(a_rsrc, stage + (wave * LOADS_A + j) * 1024, a_off_g[j], koff);                         \
    _Pragma("unroll") for (int j = 0; j < LOADS_B; ++j)                                                         \
        buffer_to_lds16(b_rsrc, stage + BM * BKB + (wave * LOADS_B + j) * 1024, b_off_g[j], koff);              \
  } while (0)
  // vmcnt(n) with lgkmcnt and expcnt left alone (gfx9 s_waitcnt encoding), then every LDS read of this wave done
  // and the workgroup barrier
#define KRN_ISSUE_A(slice)                                                                                      \
  do {                                                                                                          \
    uint8_t* stage = lds + ((slice) % STAGES) * STAGE_BYTES;                                                    \
    const int koff = (slice) * BKB;                                                                             \
    _Pragma("unroll") for (int j = 0; j < LOADS_A; ++j)                                                         \
        buffer_to_lds16(a_rsrc, stage + (wave * LOADS_A + j) * 1024, a_off_g[j], koff);                         \
  } while (0)
#define KRN_ISSUE_B(slice)                                                                                      \
  do {                                                                                                          \
    uint8_t* stage = lds + ((slice) % STAGES) * STAGE_BYTES;                                                    \
    const int koff = (slice) * BKB;                                                                             \
    _Pragma("unroll") for (int j = 0; j < LOADS_B; ++j)                                                         \
        buffer_to_lds16(b_rsrc, stage + BM * BKB + (wave * LOADS_B + j) * 1024, b_off_g[j], koff);              \
  } while (0)
  // scheduling of the spread form: per load, MFMA read MFMA read MFMA load MFMA read (one load every four MFMAs)
#define KRN_SPREAD_A()                                                                                         \
  do {                                                                                                          \
    _Pragma("unroll") for (int q = 0; q < LOADS_A; ++q) {                                                       \
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0); __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);     \
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0); __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);     \
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0); __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);     \
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0); __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);     \
    }                                                                                                           \
  } while (0)
#define KRN_SPREAD_B()                                                                                         \
  do {                                                                                                          \
    _Pragma("unroll") for (int q = 0; q < LOADS_B; ++q) {                                                       \
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0); __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);     \
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0); __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);     \
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0); __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);     \
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0); __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);     \
    }                                                                                                           \
  } while (0)
#define KRN_PUBLISH(n)                                                                                          \
  do {                                                                                                          \
    __builtin_amdgcn_s_waitcnt(0x0070 | 0x0f00 | ((n) & 15) | (((n) >> 4) << 14));                              \
    __builtin_amdgcn_s_waitcnt(0xc07f & ~0x0f00);                                                               \
    __builtin_amdgcn_s_barrier();                                                                               \
  } while (0)
#define KRN_FRAGS(dst, slice, k)                                                                                \
  do {                                                                                                          \
    const u32x4* st = reinterpret_cast<const u32x4*>(lds + ((slice) % STAGES) * STAGE_BYTES);                   \
    _Pragma("unroll") for (int i = 0; i < TM; ++i) _Pragma("unroll") for (int c = 0; c < CH; ++c)              \
        dst##a[i][c] = st[a_off[i][k][c]];                                                                      \
    _Pragma("unroll") for (int j = 0; j < TN; ++j) _Pragma("unroll") for (int c = 0; c < CH; ++c)              \
        dst##b[j][c] = st[b_off[j][k][c]];                                                                      \
  } while (0)
#define KRN_MMA(src)                                                                                            \
  _Pragma("unroll") for (int i = 0; i < TM; ++i) _Pragma("unroll") for (int j = 0; j < TN; ++j)                 \
      Unit::step(acc[i][j], src##a[i], src##b[j])
  // scheduling hints: one LDS read (0x100) or one global load (0x020) between consecutive MFMAs (0x008)
#define KRN_WITH_READS()                                                                                        \
  _Pragma("unroll") for (int q = 0; q < (TM + TN) * CH; ++q) {                                                  \
    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);                                                          \
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                                                          \
  }
#define KRN_WITH_LOADS()                                                                                        \
  _Pragma("unroll") for (int q = 0; q < LOADS; ++q) {                                                           \
    __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);                                                          \
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                                                          \
  }

#pragma unroll
  for (int s = 0; s < STAGES - 1; ++s)
    if (s < nk) KRN_ISSUE(s);
  Acc acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = Acc{};
  u32x4 f0a[TM][CH], f0b[TN][CH], f1a[TM][CH], f1b[TN][CH];
  if (nk > STAGES - 2) {
    KRN_PUBLISH(VMCNT);
  } else {
    KRN_PUBLISH(0);
  }
  KRN_FRAGS(f0, 0, 0);
  int kt = 0;
  // steady state: every slice refills the ring (branch-free, so the scheduler can interleave)
  for (; kt + STAGES - 1 < nk; ++kt) {
#pragma unroll
    for (int k = 0; k < KS; k += 2) {
      KRN_FRAGS(f1, kt, k + 1);
      if constexpr (SPREAD) {
        if (k == 0) KRN_ISSUE_A(kt + STAGES - 1);
        KRN_MMA(f0);
        KRN_SPREAD_A();
      } else {
        if (k == 0) KRN_ISSUE(kt + STAGES - 1);
        KRN_MMA(f0);
        KRN_WITH_READS();
        if (k == 0) KRN_WITH_LOADS();
      }
      if (k + 2 < KS) {
        KRN_FRAGS(f0, kt, k + 2);
      } else {
        KRN_PUBLISH(VMCNT_SPLIT);
        KRN_FRAGS(f0, kt + 1, 0);
        if constexpr (SPREAD) KRN_ISSUE_B(kt + STAGES - 1);
      }
      KRN_MMA(f1);
      if constexpr (SPREAD) {
        KRN_SPREAD_B();
      } else {
        KRN_WITH_READS();
      }
    }
  }
  // drain: the last STAGES - 1 slices are already in flight
  for (; kt < nk; ++kt) {
#pragma unroll
    for (int k = 0; k < KS; k += 2) {
      KRN_FRAGS(f1, kt, k + 1);
      KRN_MMA(f0);
      KRN_WITH_READS();
      if (k + 2 < KS) {
        KRN_FRAGS(f0, kt, k + 2);
      } else if (kt + 1 < nk) {
        KRN_PUBLISH(0);
        KRN_FRAGS(f0, kt + 1, 0);
      }
      KRN_MMA(f1);
      KRN_WITH_READS();
    }
  }
#undef KRN_ISSUE
#undef KRN_PUBLISH
#undef KRN_FRAGS
#undef KRN_MMA
#undef KRN_WITH_READS
#undef KRN_WITH_LOADS
#undef KRN_ISSUE_A
#undef KRN_ISSUE_B
#undef KRN_SPREAD_A
#undef KRN_SPREAD_B
  __syncthreads();  // every wave is done with the ring before its LDS becomes the store patches

  uint32_t* patch = reinterpret_cast<uint32_t*>(lds) + wave * PATCH_WORDS;
  store_tile<FMT == FMT_I8>(acc, patch, C, ldc, m0 + wm * (BM / WM), n0 + wn * (BN / WN), M, N, e, lane);
}

// The four-wave main loop for whole 256 x 256 tiles with K a multiple of 128 bytes (bf16/f16 NT and NN, fp8, int8),
// on the 16x16 MFMA forms. Each wave owns a 128 x 128 quarter (wave w: rows 128 (w >> 1), columns 128 (w & 1)) as
// 8 x 8 accumulator blocks of 16 x 16 in AGPRs, each computed transposed (B A^T: the B fragment is the MFMA's first
// operand), so that a lane holds four columns of one row for the store (`store_tile16t`). 128-byte K slices go straight from global memory into LDS stages,
// two for A and three for B (5 x 32 KiB fill the 160 KiB), each stage a separate array so that the compiler can tell
// every fragment read from the loads in flight into the other stages; wave w loads rows 64 w .. 64 w + 63 of A and
// of B, 8 rows (1 KiB) per load, chunk c of row r at slot c ^ ((r >> 1) & 7).
//
// bf16/f16/int8: a slice is two steps of 64 bytes of K; fp8: one step of 128 (16x16x128). One set of fragments (A
// blocks 0-3 and B blocks 0-3 of 32 rows, each two 16-row halves) is refilled in place: steps alternate between
// running their 16 blocks of 32 x 32 row by row (block (I, J) is group 4 I + J of four MFMAs) and column by column,
// so a block's fragments are dead after its last group of the step and take the next step's at once (row order
// frees A block I after group 4 I + 3 and B block J after 12 + J; column order frees B block J after 4 J + 3 and A
// block I after 12 + I). The one barrier per slice sits after group 3 of its last step: by then this wave has read
// all of slice kt and its loads of slice kt + 1 have landed. B's slice kt + 2 is loaded during the slice, before
// and after the barrier (into the stage slice kt - 1 left, free since the last barrier), one load every other group;
// A's slice kt + 2 after the barrier, one load per group, into the stage slice kt leaves. Loads issued in a burst
// (the 16 of a slice in 8 groups) ask the vector memory path for twice what it delivers and stall the MFMA issue
// behind them (bf16 8192^3: 1452 TFLOP/s spread against 1392, MFMA busy 0.79 against 0.71; 0.84 with no loads).
//
// Measured against the 32x32 forms: MFMA-only loops on random operands sustain 16 % (bf16) and 25 % (int8) more
// on 16x16 at the same power limit; bf16 8192^3 on the register-staged 32x32 loop 1335 TFLOP/s, W8A8 M = 4096 on
// the eight-wave 32x32 loop 0.275 ms against 0.269; fp8 8192^3 equal (0.442 ms), the 16x16 form at a higher clock
// with proportionally less MFMA time.
template <int FMT, bool NN = false>
__global__ __launch_bounds__(256, 1) void gemm_quad16(const uint8_t* __restrict__ A, const uint8_t* __restrict__ B,
                                                     void* __restrict__ C, int64_t M, int64_t N, int64_t kbytes,
                                                     int64_t lda, int64_t ldb, int64_t ldc, Epilogue e) {
  constexpr int NA = 2, NB = 3;  // LDS stages of A and B
  typedef Mfma16<FMT> Unit;
  typedef typename Unit::Acc Acc;
  typedef typename Mfma<FMT>::Acc Acc32;
  // fp8: one 16x16x128 step per slice, 32 bytes of K per lane and operand; otherwise two steps of 16 bytes
  constexpr bool F8 = FMT == FMT_FP8;
  constexpr int NSTEP = F8 ? 1 : 2;
  typedef typename std::conditional<F8, i32x8, u32x4>::type Frag;
  static_assert(!NN || FMT == FMT_BF16 || FMT == FMT_F16, "NN: 16-bit operands");
  constexpr int BM = 256, BN = 256, BKB = 128;
  constexpr int HALF = BM * BKB;  // 32 KiB: one operand's rows of one slice
  constexpr int UNROLL = 6;  // slices per loop iteration: every stage index a constant
  __shared__ __attribute__((aligned(1024))) uint8_t la0[HALF];
  __shared__ __attribute__((aligned(1024))) uint8_t la1[HALF];
  __shared__ __attribute__((aligned(1024))) uint8_t lb0[HALF];
  __shared__ __attribute__((aligned(1024))) uint8_t lb1[HALF];
  __shared__ __attribute__((aligned(1024))) uint8_t lb2[HALF];
  int tm, tn;
  tile_of((int)((M + BM - 1) / BM), (int)((N + BN - 1) / BN), tm, tn);
  const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
  const int t = threadIdx.x, lane = t & 63, wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  auto uniform = [](const void* p) {
    const uint64_t v = (uint64_t)p;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return (const void*)(((uint64_t)hi << 32) | lo);
  };
  const int64_t a_bytes = __builtin_amdgcn_readfirstlane((int)min((M - m0) * lda, (int64_t)0x7fffffff));
  // NN: the panel is columns n0 .. n0 + 255 of every row of B (the host checks that it is addressable)
  const int64_t b_bytes = __builtin_amdgcn_readfirstlane(
      NN ? (int)((kbytes / 2 - 1) * ldb + BN * 2) : (int)min((N - n0) * ldb, (int64_t)0x7fffffff));
  const __amdgpu_buffer_rsrc_t a_rsrc = panel_rsrc(uniform(A + m0 * lda), a_bytes),
                              b_rsrc = panel_rsrc(uniform(B + (NN ? n0 * 2 : n0 * ldb)), b_bytes);
  // load item j of an operand: rows 64 wave + 8 j .. + 7; lane i takes row i / 8 and the global chunk that belongs at
  // slot i % 8. The swizzle of row 8 j + i / 8 depends on j only through j & 1.
  const int lrow = lane >> 3, lslot = lane & 7;
  uint32_t ga[2], gb[4];
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    const int row = wave * 64 + p * 8 + lrow;
    ga[p] = (uint32_t)(row * lda + ((lslot ^ swz8(row)) * 16));
    gb[p] = (uint32_t)(row * ldb + ((lslot ^ swz8(row)) * 16));
  }
  // NN: a slice of B is 64 k rows of 512 bytes ([k][n]); wave w loads k rows 16 w .. 16 w + 15, two per load (item
  // j: rows 16 w + 2 j + i / 32, lane i at slot i % 32). Chunk c of row k sits at slot c ^ nn_swz(k), which puts the
  // 8 rows a transposed fragment read serves per pass on 8 distinct 32-byte bank groups. The lane offsets depend on
  // j through j & 1 and j >> 2; the rest is the scalar offset 2 j ldb.
  auto nn_swz = [](int k) { return 2 * ((k & 3) | (((k >> 3) & 1) << 2)); };
  if constexpr (NN) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int j = (q >> 1) * 4 + (q & 1);
      const int krow = wave * 16 + 2 * j + (lane >> 5), slot = lane & 31;
      gb[q] = (uint32_t)((wave * 16 + (lane >> 5)) * ldb + ((slot ^ nn_swz(krow)) * 16));
    }
  }
  // NN fragment reads (ds_read_b64_tr_b16): lane L = 16 g + a reads k row 8 g + 4 p + a / 4 (part p) of the step's
  // 32 and columns 4 (a % 4) .. + 3 of its 16, and receives column a of the 16 at the four k of the part
  const int tg = lane >> 4, ta = lane & 15;
  const int tr_row = (8 * tg + (ta >> 2)) * 512, tr_swz = nn_swz(8 * tg + (ta >> 2));
  const int tr_col = wn * 128 + 4 * (ta & 3);
  const int wbase = wave * 8192;
  // fragment bases: lane L reads row L & 15 of a 16-row half, 16-byte chunk 4 x + (L >> 4) (step x), or for fp8
  // chunks 2 (L >> 4) + x (x = 0, 1: the lane's 32 bytes)
  int ra[2], rb[2];
#pragma unroll
  for (int x = 0; x < 2; ++x) {
    const int chunk = F8 ? 2 * (lane >> 4) + x : 4 * x + (lane >> 4);
    const int part = (lane & 15) * 128 + ((chunk ^ (((lane & 15) >> 1) & 7)) * 16);
    ra[x] = part + wm * 128 * 128;
    rb[x] = part + wn * 128 * 128;
  }
  const int one = 127;  // fp8: the unit E8M0 scale
  const int nk = (int)(kbytes / BKB);  // >= 2 (host)

  Frag F[16];  // A block I half R at 2 I + R, B block J half Q at 8 + 2 J + Q
  Acc acc[8][8];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[i][j] = Acc{};

#define KD_A(p) ((p) == 0 ? la0 : la1)
#define KD_B(p) ((p) == 0 ? lb0 : (p) == 1 ? lb1 : lb2)
#define KD_LOADA(j, sl, pa)                                                                                    \
  buffer_to_lds16(a_rsrc, KD_A(pa) + wbase + (j) * 1024, ga[(j) & 1], (int)((sl) * BKB + ((j) & 6) * 8 * lda))
#define KD_LOADB(j, sl, pb)                                                                                    \
  do {                                                                                                         \
    if constexpr (NN)                                                                                          \
      buffer_to_lds16(b_rsrc, KD_B(pb) + wbase + (j) * 1024, gb[((j) >> 2) * 2 + ((j) & 1)],                   \
                      (int)(((sl) * 64 + 2 * (j)) * ldb));                                                     \
    else                                                                                                       \
      buffer_to_lds16(b_rsrc, KD_B(pb) + wbase + (j) * 1024, gb[(j) & 1],                                      \
                      (int)((sl) * BKB + ((j) & 6) * 8 * ldb));                                                \
  } while (0)
#define KD_TR(pb, s, p, col)                                                                                   \
  __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4s16*)( \
                                KD_B(pb) + tr_row + ((s) * 32 + (p) * 4) * 512 +                               \
                                ((((col) >> 3) ^ tr_swz) * 16) + ((col) & 7) * 2)))
#define KD_READ(r, c, pa, pb, s)                                                                               \
  do {                                                                                                         \
    if constexpr (F8) {                                                                                        \
      const uint8_t* p8 = ((r) < 4 ? KD_A(pa) : KD_B(pb)) + (((r) & 3) * 32 + (c) * 16) * 128;                 \
      const u32x4 lo = *reinterpret_cast<const u32x4*>(p8 + ((r) < 4 ? ra[0] : rb[0]));                        \
      const u32x4 hi = *reinterpret_cast<const u32x4*>(p8 + ((r) < 4 ? ra[1] : rb[1]));                        \
      F[(r) * 2 + (c)] = Frag{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3],                                   \
                              (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};                                 \
    } else {                                                                                                   \
      if (NN && (r) >= 4) {                                                                                    \
        const int col = tr_col + ((r) - 4) * 32 + (c) * 16;                                                    \
        const u32x2 lo = KD_TR(pb, s, 0, col), hi = KD_TR(pb, s, 1, col);                                      \
        F[(r) * 2 + (c)] = u32x4{lo[0], lo[1], hi[0], hi[1]};                                                  \
      } else {                                                                                                 \
        F[(r) * 2 + (c)] = *reinterpret_cast<const u32x4*>(                                                    \
            ((r) < 4 ? KD_A(pa) + ra[s] : KD_B(pb) + rb[s]) + (((r) & 3) * 32 + (c) * 16) * 128);              \
      }                                                                                                        \
    }                                                                                                          \
  } while (0)
#define KD_FENCE() __builtin_amdgcn_sched_barrier(0)
#define KD_MMA(I, J)                                                                                           \
  _Pragma("unroll") for (int R = 0; R < 2; ++R) _Pragma("unroll") for (int Q = 0; Q < 2; ++Q) {               \
    if constexpr (F8)                                                                                          \
      Unit::step_agpr(acc[(I) * 2 + R][(J) * 2 + Q], F[8 + (J) * 2 + Q], F[(I) * 2 + R], one);                \
    else                                                                                                       \
      Unit::step_agpr(acc[(I) * 2 + R][(J) * 2 + Q], F[8 + (J) * 2 + Q], F[(I) * 2 + R]);                     \
  }
  // One step of slice kt (A stage PA, B stage PB). ORD 0: its 16 blocks row by row (group g = 4 I + J), 1: column
  // by column (g = 4 J + I); either way A block I is dead after its group with J = 3 and B block J after its group
  // with I = 3, and the next step's fragments of that block are read at once (ORD 0 reads A first, 1 reads B first).
  // The next step is step s + 1 of this slice, or (LAST) step 0 of slice kt + 1. In the last step, after group 3,
  // the barrier (this wave's loads of slice kt + 1 landed: only the loads of a three-stage operand's slice kt + 2,
  // issued last, may still be in flight), then the loads into the stages slice kt leaves, two-stage operands first
  // (past the end: the last slice again, into a stage nothing reads any more).
#define KD_STEP(PA, PB, ORD, LAST, kt, s)                                                                      \
  do {                                                                                                         \
    const int NA_ = (LAST) ? ((PA) + 1) % NA : (PA), NB_ = (LAST) ? ((PB) + 1) % NB : (PB);                    \
    const int NS_ = (LAST) ? 0 : (s) + 1;                                                                      \
    _Pragma("unroll") for (int g = 0; g < 16; ++g) {                                                           \
      const int I = (ORD) ? (g & 3) : (g >> 2), J = (ORD) ? (g >> 2) : (g & 3);                                \
      KD_MMA(I, J);                                                                                            \
      KD_FENCE();                                                                                              \
      if ((LAST) && g == 3) {                                                                                  \
        /* still in flight may be only B's slice kt + 2: its loads of step 0 (eight), or of this step's groups 0  \
           and 2 (fp8) */                                                                                      \
        if constexpr (NSTEP == 1)                                                                              \
          __builtin_amdgcn_s_waitcnt(0x0070 | 2); /* vmcnt(2) lgkmcnt(0) */                                     \
        else                                                                                                   \
          __builtin_amdgcn_s_waitcnt(0x0070 | 8); /* vmcnt(8) lgkmcnt(0) */                                     \
        __builtin_amdgcn_s_barrier();                                                                          \
        KD_FENCE();                                                                                            \
      }                                                                                                        \
      if ((NSTEP == 1 || !(LAST)) && (NSTEP == 1 ? (g & 1) == 0 : (g & 1))) {                                  \
        KD_LOADB(g >> 1, min((kt) + 2, nk - 1), ((PB) + 2) % NB);                                              \
        KD_FENCE();                                                                                            \
      }                                                                                                        \
      if ((LAST) && g >= 3 && g < 11) { /* (spread over groups 3-15 instead: 0.4 % slower) */                  \
        KD_LOADA(g - 3, min((kt) + 2, nk - 1), PA);                                                            \
        KD_FENCE();                                                                                            \
      }                                                                                                        \
      _Pragma("unroll") for (int o = 0; o < 2; ++o) {                                                          \
        if ((o == 0) == ((ORD) == 0) && J == 3) {                                                              \
          KD_READ(I, 0, NA_, NB_, NS_);                                                                        \
          KD_READ(I, 1, NA_, NB_, NS_);                                                                        \
          KD_FENCE();                                                                                          \
        }                                                                                                      \
        if ((o == 0) == ((ORD) == 1) && I == 3) {                                                              \
          KD_READ(4 + J, 0, NA_, NB_, NS_);                                                                    \
          KD_READ(4 + J, 1, NA_, NB_, NS_);                                                                    \
          KD_FENCE();                                                                                          \
        }                                                                                                      \
      }                                                                                                        \
    }                                                                                                          \
  } while (0)
  // slice u of an unrolled run (u even at the start of a run, so that the order alternates from step to step):
  // step 0 row by row, step 1 column by column; fp8's one step per slice alternates from slice to slice
#define KD_SLICE(u, kt)                                                                                        \
  do {                                                                                                         \
    if constexpr (NSTEP == 2) {                                                                                \
      KD_STEP((u) % NA, (u) % NB, 0, false, kt, 0);                                                            \
      KD_STEP((u) % NA, (u) % NB, 1, true, kt, 1);                                                             \
    } else {                                                                                                   \
      KD_STEP((u) % NA, (u) % NB, (u) & 1, true, kt, 0);                                                       \
    }                                                                                                          \
  } while (0)

  // the prologue: slices 0 and 1 of A and B (B's slice 2 loads during slice 0, as in the loop); once slice 0 has
  // landed everywhere, its step-0 fragments
#pragma unroll
  for (int sl = 0; sl < 2; ++sl) {
#pragma unroll
    for (int j = 0; j < 8; ++j) KD_LOADA(j, min(sl, nk - 1), sl);
#pragma unroll
    for (int j = 0; j < 8; ++j) KD_LOADB(j, min(sl, nk - 1), sl);
  }
#define KD_VMWAIT(n) __builtin_amdgcn_s_waitcnt(0x0070 | 0x0f00 | ((n) & 15) | (((n) >> 4) << 14))
  KD_VMWAIT(16);  // slice 0's 16 loads came first
  __builtin_amdgcn_s_barrier();
  KD_FENCE();
  // in the order step 1 reads them (B0 B1 B2 A0 A1 A2 B3 A3), so that the loop's first MFMAs wait on the same
  // partial LDS count whether they follow this or the loop's last step
#pragma unroll
  for (int x = 0; x < 8; ++x) {
    const int r = x < 3 ? 4 + x : x < 6 ? x - 3 : x == 6 ? 7 : 3;
    KD_READ(r, 0, 0, 0, 0);
    KD_READ(r, 1, 0, 0, 0);
    KD_FENCE();
  }
  int kt = 0;
  for (; kt + UNROLL <= nk; kt += UNROLL) {
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) KD_SLICE(u, kt + u);
  }
  // W8A8's scale vectors go out before the last (up to five) slices, so that their latency runs under MFMAs
  const int64_t row0 = m0 + wm * 128, col0 = n0 + wn * 128;
  const bool direct = quad16_direct(e, C, ldc, row0, col0, M, N), rowcol = direct && quad16_is_rowcol(e);
  Quad16RowCol rc;
  if (rowcol) quad16_rowcol(rc, e, row0, col0, lane);
#pragma unroll
  for (int u = 0; u < UNROLL - 1; ++u)
    if (kt + u < nk) KD_SLICE(u, kt + u);
#undef KD_A
#undef KD_B
#undef KD_LOADA
#undef KD_LOADB
#undef KD_READ
#undef KD_FENCE
#undef KD_MMA
#undef KD_STEP
#undef KD_SLICE
#undef KD_TR
#undef KD_VMWAIT
  __builtin_amdgcn_s_waitcnt(0x0070 | 0x0f00);  // vmcnt(0): no load still writes the stages
  // the MFMAs are assembly, so the compiler inserts no wait states between the last of them and the first read of
  // their results: 24 cycles cover the longest 16x16 form
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
  __syncthreads();  // every wave is done with the stages before their LDS becomes the store patches
  uint32_t* patch = reinterpret_cast<uint32_t*>(la0) + wave * PATCH_WORDS;
  store_tile16t<FMT == FMT_I8, Acc32>(acc, direct, rowcol, rc, patch, C, ldc, row0, col0, M, N, e, lane);
}

// Ping-pong main loop for whole 256 x 256 tiles with 64-byte K slices (bf16/f16: two 32x32x16 steps, int8: two
// 32x32x32 steps, fp8: one 32x32x64 step per slice -- 512 MFMA cycles per wave in every format). Eight waves form two
// groups of four: group g owns rows [128 g, 128 g + 128) of the tile, and within a group wave q owns the 64 x 128
// block (q >> 1, q & 1). Waves w and w + 4 run on the same SIMD, and group 1 starts one barrier late, so on every
// SIMD one wave issues its 16 MFMAs while the other reads its next fragments from LDS and issues direct-to-LDS loads:
// the matrix core is fed from one wave while the other's LDS and memory waits are hidden behind it.
//
// Every slot ends in a workgroup barrier. Per slice j a wave runs a memory phase (issue its part of the loads of
// slice j + STAGES - 1, read the fragments of slice j, wait for them and for its own loads of slice j + 1) and then
// a compute phase (the MFMAs of slice j). Group 0 loads the A rows of every slice, group 1 the B rows. Slice j is
// read by group 0 in slot 2j and by group 1 in slot 2j + 1, so its stage is free from slot 2j + 2 on, which is when
// the loads of slice j + STAGES (same stage) are issued at the earliest.
template <int FMT, int STAGES>
__global__ __launch_bounds__(512, 1) void gemm_pp(const uint8_t* __restrict__ A, const uint8_t* __restrict__ B,
                                                  void* __restrict__ C, int64_t M, int64_t N, int64_t kbytes,
                                                  int64_t lda, int64_t ldb, int64_t ldc, Epilogue e) {
  typedef Mfma<FMT> Unit;
  typedef typename Unit::Acc Acc;
  constexpr int BM = 256, BN = 256, BKB = 64, CPR = 4;  // 64-byte slice rows of four 16-byte chunks
  constexpr int TM = 2, TN = 4;                          // 32x32 blocks per wave
  constexpr int STEP = Unit::kBytes, CH = STEP / 32, KS = BKB / STEP;
  constexpr int PART = BM * BKB;                         // bytes of one operand's rows in a stage (16 KiB)
  constexpr int STAGE_BYTES = 2 * PART;
  constexpr int LOADS = PART / 1024 / 4;                 // 1 KiB wave loads per wave per slice (4)
  constexpr int VMWAIT = (STAGES - 2) * LOADS;
  static_assert(STAGES >= 3 && STAGES * STAGE_BYTES <= 160 * 1024, "LDS of one CU");
  static_assert(VMWAIT <= 63, "vmcnt range");
  __shared__ __attribute__((aligned(1024))) uint8_t lds[STAGES * STAGE_BYTES];

  int tm, tn;
  tile_of((int)((M + BM - 1) / BM), (int)((N + BN - 1) / BN), tm, tn);
  const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g = wave >> 2, q = wave & 3;
  const int half = lane >> 5, r32 = lane & 31;

  // loads: group 0 fills the A part of a stage, group 1 the B part; wave q the rows [64 q, 64 q + 64)
  const int lrow = lane / CPR, lslot = lane % CPR;
  // through a buffer resource over the group's panel, as in gemm_pipe
  const __amdgpu_buffer_rsrc_t rsrc = g ? panel_rsrc(B + n0 * ldb, (N - n0) * ldb) : panel_rsrc(A + m0 * lda, (M - m0) * lda);
  uint32_t src_off[LOADS];
  {
    const int64_t ld = g ? ldb : lda;
#pragma unroll
    for (int j = 0; j < LOADS; ++j) {
      const int row = (q * LOADS + j) * 16 + lrow;
      src_off[j] = (uint32_t)(row * ld + (lslot ^ swz4(row)) * 16);
    }
  }
  const int dst0 = g * PART + q * LOADS * 1024;
  // fragment offsets (16-byte units within a stage)
  const int wr = g * 128 + (q >> 1) * 64, wc = (q & 1) * 128;
  int a_off[TM][KS][CH], b_off[TN][KS][CH];
#pragma unroll
  for (int k = 0; k < KS; ++k)
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const int chunk = (k * STEP + half * (STEP / 2)) / 16 + c;
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int row = wr + i * 32 + r32;
        a_off[i][k][c] = row * CPR + (chunk ^ swz4(row));
      }
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int row = wc + j * 32 + r32;
        b_off[j][k][c] = BM * CPR + row * CPR + (chunk ^ swz4(row));
      }
    }
  const int nk = (int)(kbytes / BKB);

#define KRN_ISSUE(slice)                                                                                        \
  do {                                                                                                          \
    uint8_t* stage = lds + ((slice) % STAGES) * STAGE_BYTES + dst0;                                             \
    const int koff = (slice) * BKB;                                                                             \
    _Pragma("unroll") for (int j = 0; j < LOADS; ++j) buffer_to_lds16(rsrc, stage + j * 1024, src_off[j], koff); \
  } while (0)
#define KRN_VMWAIT(n) __builtin_amdgcn_s_waitcnt(0x0070 | 0x0f00 | ((n) & 15) | (((n) >> 4) << 14))
#define KRN_LGKWAIT() __builtin_amdgcn_s_waitcnt(0xc07f & ~0x0f00)

#pragma unroll
  for (int s = 0; s < STAGES - 1; ++s)
    if (s < nk) KRN_ISSUE(s);
  Acc acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = Acc{};
  if (nk > STAGES - 2) {
    KRN_VMWAIT(VMWAIT);
  } else {
    KRN_VMWAIT(0);
  }
  __builtin_amdgcn_s_barrier();
  if (g == 1) __builtin_amdgcn_s_barrier();
  u32x4 fa[KS][TM][CH], fb[KS][TN][CH];
  for (int kt = 0; kt < nk; ++kt) {
    // memory phase
    const bool refill = kt + STAGES - 1 < nk;
    if (refill) KRN_ISSUE(kt + STAGES - 1);
    {
      const u32x4* st = reinterpret_cast<const u32x4*>(lds + (kt % STAGES) * STAGE_BYTES);
#pragma unroll
      for (int k = 0; k < KS; ++k) {
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int c = 0; c < CH; ++c) fa[k][i][c] = st[a_off[i][k][c]];
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
          for (int c = 0; c < CH; ++c) fb[k][j][c] = st[b_off[j][k][c]];
      }
    }
    KRN_LGKWAIT();
    if (refill) {
      KRN_VMWAIT(VMWAIT);
    } else {
      KRN_VMWAIT(0);
    }
    __builtin_amdgcn_s_barrier();
    // compute phase
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int k = 0; k < KS; ++k)
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) Unit::step(acc[i][j], fa[k][i], fb[k][j]);
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_barrier();
  }
  if (g == 0) __builtin_amdgcn_s_barrier();
#undef KRN_ISSUE
#undef KRN_VMWAIT
#undef KRN_LGKWAIT
  __syncthreads();  // every wave is done with the ring before its LDS becomes the store patches

  uint32_t* patch = reinterpret_cast<uint32_t*>(lds) + wave * PATCH_WORDS;
  store_tile<FMT == FMT_I8>(acc, patch, C, ldc, m0 + wr, n0 + wc, M, N, e, lane);
}

// Skinny products (M <= 128), the HBM-bound shapes: B (N x K) is streamed from HBM once and A (M x K) is read by
// every workgroup from L2. A workgroup owns 32 output columns and all M rows (MT blocks of 32); its WAVES waves split
// K, wave w taking one contiguous run of 128-byte K slices (runs far apart in a row keep each wave's HBM requests on
// few DRAM pages). Each wave moves its slices of A and B into its own LDS ring with direct-to-LDS loads that cover 8
// whole 128-byte rows per instruction, then reads the MFMA operands from LDS: loads with one lane per row (32 rows x
// 16 bytes per instruction) would fetch every line four times. Row R of a staged slice holds its 16-byte chunk c at
// position c ^ ((R >> 1) & 7), so a ds_read_b128 of one chunk from 16 consecutive rows touches all 64 banks once.
// Lane (r32, half) takes chunks half * 4 + q of its row for A and for B alike, and MFMA step s the s-th 16 bytes of
// them (32 bytes for fp8): both operands see the same K permutation, so the dot products are unchanged. The ring has
// STAGES stages per wave, STAGES - 1 slices in flight while one is multiplied. The partial sums meet in LDS, and
// waves 0..MT-1 each store one 32 x 32 block through the common epilogue.
template <int FMT, int MT, int WAVES, int STAGES, bool ACT, int AL = MT * 4>
__global__ __launch_bounds__(WAVES * 64, 1) void gemm_skinny(const uint8_t* __restrict__ A,
                                                              const uint8_t* __restrict__ B, void* __restrict__ C,
                                                              int64_t M, int64_t N, int64_t kbytes, int64_t lda,
                                                              int64_t ldb, int64_t ldc, Epilogue e) {
  typedef Mfma<FMT> Unit;
  typedef typename Unit::Acc Acc;
  typedef std::conditional_t<FMT == FMT_I8, int, float> Elem;
  constexpr int CH = Unit::kBytes / 32;       // 16-byte registers per lane per MFMA step
  constexpr int STEPS = 4 / CH;               // MFMA steps per 128-byte slice
  constexpr int STAGE = (MT + 1) * 4096;      // one slice: MT * 32 rows of A, then 32 rows of B, 128 bytes each
  constexpr int LOADS = AL + 4;               // DMA instructions per slice: AL of A's rows (8 each), 4 of B's
  static_assert(AL >= 1 && AL <= MT * 4, "A loads cover at most the ring's A rows");
  constexpr int AHEAD = (STAGES - 1) * LOADS; // loads still in flight when the oldest slice is waited for
  constexpr int RING_WORDS = WAVES * STAGES * STAGE / 4;
  constexpr int RED_WORDS = WAVES * MT * 16 * 64;
  constexpr int W1 = RING_WORDS > RED_WORDS ? RING_WORDS : RED_WORDS;
  constexpr int LDS_WORDS = W1 > WAVES * PATCH_WORDS ? W1 : WAVES * PATCH_WORDS;
  static_assert(LDS_WORDS * 4 <= 160 * 1024, "the ring exceeds the LDS of a CU");
  __shared__ __attribute__((aligned(16))) uint32_t lds[LDS_WORDS];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int half = lane >> 5, r32 = lane & 31;
  const int64_t n0 = (int64_t)blockIdx.x * 32;
  // DMA instruction j fills rows 8 j .. 8 j + 7 of the stage (A's rows first, then B's); lane L lands at position
  // L & 7 of row 8 j + (L >> 3) and so fetches the chunk that the swizzle puts there. Rows past the end of A or B
  // read the last row: their results are never stored.
  // Only the first AL eight-row groups of A are loaded: the ring rows past them hold whatever the LDS held, and
  // their results (rows >= 8 AL >= M) are never stored.
  const uint8_t* src[LOADS];
  int dst[LOADS];
#pragma unroll
  for (int j = 0; j < LOADS; ++j) {
    const int g = j < AL ? j : MT * 4 + (j - AL);  // eight-row group of the stage
    const int chunk = (lane & 7) ^ (((g & 3) * 4 + (lane >> 4)) & 7);
    const int64_t row = g * 8 + (lane >> 3);  // row of the stage
    src[j] = j < AL ? A + min(row, M - 1) * lda + chunk * 16 : B + min(n0 + row - MT * 32, N - 1) * ldb + chunk * 16;
    dst[j] = g * 1024;
  }
  uint8_t* ring = reinterpret_cast<uint8_t*>(lds) + wave * STAGES * STAGE;
  int rd[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) rd[q] = r32 * 128 + (((half * 4 + q) ^ ((r32 >> 1) & 7)) * 16);
  const int nk = (int)(kbytes / 128);
  const int per = nk / WAVES, rem = nk % WAVES;
  const int begin = wave * per + min(wave, rem), cnt = per + (wave < rem ? 1 : 0);
  // the storing waves fetch the epilogue's vector operands now: loads issued at the very end of a workgroup would
  // wait behind the other workgroups' streams
  EpiPre pre;
  if (e.nops > 0) epi_prefetch(pre, e, A, (int64_t)wave * 32, n0, M, N, lane);
  Acc acc[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) acc[t] = Acc{};
  auto issue = [&](int slice, int stage) {
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's reads of the stage are done before it is refilled
    const int64_t off = (int64_t)slice * 128;
#pragma unroll
    for (int j = 0; j < AL; ++j)
      __builtin_amdgcn_global_load_lds((const void*)(src[j] + off),
                                       (__attribute__((address_space(3))) void*)(ring + stage * STAGE + dst[j]), 16,
                                       0, 0);
    // B (the weights, read once) streams non-temporally when M <= 32: fp8 M = 1 13.4 -> 11.8 us, M = 16 13.4 ->
    // 12.5 us, W8A8 M = 16 12.6 -> 12.0 us. With four row blocks (M = 128) it was 22 % slower, so A-heavy shapes
    // keep the default policy.
#pragma unroll
    for (int j = AL; j < LOADS; ++j)
      __builtin_amdgcn_global_load_lds((const void*)(src[j] + off),
                                       (__attribute__((address_space(3))) void*)(ring + stage * STAGE + dst[j]), 16,
                                       0, MT == 1 ? 2 : 0);
  };
  auto consume = [&](int stage) {
    const uint8_t* base = ring + stage * STAGE;
    u32x4 ra[MT][4], rb[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) rb[q] = *reinterpret_cast<const u32x4*>(base + MT * 4096 + rd[q]);
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
      for (int q = 0; q < 4; ++q) ra[t][q] = *reinterpret_cast<const u32x4*>(base + t * 4096 + rd[q]);
#pragma unroll
    for (int s = 0; s < STEPS; ++s)
#pragma unroll
      for (int t = 0; t < MT; ++t) Unit::step(acc[t], &ra[t][s * CH], &rb[s * CH]);
  };
#pragma unroll
  for (int p = 0; p < STAGES - 1; ++p)
    if (p < cnt) issue(begin + p, p);
  // steady state: STAGES slices per iteration, so every stage index is a constant and there are no branches (the
  // waits stay exact); vmcnt(AHEAD) = all but the newest STAGES - 1 slices have landed (gfx9 s_waitcnt encoding,
  // other counters left free)
  int i = 0;
  for (; i + 2 * STAGES - 2 < cnt; i += STAGES) {
#pragma unroll
    for (int j = 0; j < STAGES; ++j) {
      issue(begin + i + j + STAGES - 1, (j + STAGES - 1) % STAGES);
      __builtin_amdgcn_s_waitcnt(0x0070 | 0x0f00 | (AHEAD & 15) | ((AHEAD >> 4) << 14));
      consume(j);
    }
  }
  // at most 2 * STAGES - 2 slices are left, and i is a multiple of STAGES
#pragma unroll
  for (int j = 0; j < 2 * STAGES - 2; ++j) {
    if (i + j < cnt) {
      if (i + j + STAGES - 1 < cnt) issue(begin + i + j + STAGES - 1, (j + STAGES - 1) % STAGES);
      __builtin_amdgcn_s_waitcnt(0x0070 | 0x0f00);  // vmcnt(0)
      consume(j % STAGES);
    }
  }
  __syncthreads();  // the partial sums overwrite other waves' rings
  Elem* partial = reinterpret_cast<Elem*>(lds);
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) partial[((wave * MT + t) * 16 + r) * 64 + lane] = acc[t][r];
  __syncthreads();
  Acc sum = Acc{};
  if (wave < MT) {
    for (int v = 0; v < WAVES; ++v)
#pragma unroll
      for (int r = 0; r < 16; ++r) sum[r] += partial[((v * MT + wave) * 16 + r) * 64 + lane];
  }
  __syncthreads();
  if (wave < MT) {
    patch_put<FMT == FMT_I8>(sum, lds + wave * PATCH_WORDS, lane);
    patch_store_inline<FMT == FMT_I8, ACT, true>(lds + wave * PATCH_WORDS, C, ldc, (int64_t)wave * 32, n0, M, N, e,
                                                 lane, &pre);
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

template <int FMT, int BM, int BN, int WM, int WN, int STAGES, int BKB>
static int launch_pipe(const void* a, const void* b, void* c, int64_t m, int64_t n, int64_t kbytes, int64_t lda,
                       int64_t ldb, int64_t ldc, const Epilogue& e, hipStream_t stream) {
  const int64_t tiles = ((m + BM - 1) / BM) * ((n + BN - 1) / BN);
  if (tiles > 0x7fffffff) {
    krn_set_error("gemm: %lld tiles exceed the grid limit", (long long)tiles);
    return -1;
  }
  hipLaunchKernelGGL((gemm_pipe<FMT, BM, BN, WM, WN, STAGES, BKB>), dim3((unsigned)tiles), dim3(WM * WN * 64), 0, stream,
                     (const uint8_t*)a, (const uint8_t*)b, c, m, n, kbytes, lda, ldb, ldc, e);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    krn_set_error("gemm launch: %s", hipGetErrorString(err));
    return (int)err;
  }
  return 0;
}

template <int FMT>
static int launch_quad16(const void* a, const void* b, void* c, int64_t m, int64_t n, int64_t kbytes, int64_t lda,
                         int64_t ldb, int64_t ldc, const Epilogue& e, hipStream_t stream) {
  const int64_t tiles = ((m + 255) / 256) * ((n + 255) / 256);
  if (tiles > 0x7fffffff) {
    krn_set_error("gemm: %lld tiles exceed the grid limit", (long long)tiles);
    return -1;
  }
  hipLaunchKernelGGL((gemm_quad16<FMT>), dim3((unsigned)tiles), dim3(256), 0, stream, (const uint8_t*)a,
                     (const uint8_t*)b, c, m, n, kbytes, lda, ldb, ldc, e);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    krn_set_error("gemm launch: %s", hipGetErrorString(err));
    return (int)err;
  }
  return 0;
}

template <int FMT, int STAGES>
static int launch_pp(const void* a, const void* b, void* c, int64_t m, int64_t n, int64_t kbytes, int64_t lda,
                     int64_t ldb, int64_t ldc, const Epilogue& e, hipStream_t stream) {
  const int64_t tiles = ((m + 255) / 256) * ((n + 255) / 256);
  if (tiles > 0x7fffffff) {
    krn_set_error("gemm: %lld tiles exceed the grid limit", (long long)tiles);
    return -1;
  }
  hipLaunchKernelGGL((gemm_pp<FMT, STAGES>), dim3((unsigned)tiles), dim3(512), 0, stream, (const uint8_t*)a,
                     (const uint8_t*)b, c, m, n, kbytes, lda, ldb, ldc, e);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    krn_set_error("gemm launch: %s", hipGetErrorString(err));
    return (int)err;
  }
  return 0;
}

template <int FMT, int MT, int STAGES>
static int launch_skinny_mt(const void* a, const void* b, void* c, int64_t m, int64_t n, int64_t kbytes, int64_t lda,
                            int64_t ldb, int64_t ldc, const Epilogue& e, hipStream_t stream) {
  // an epilogue without activations gets a kernel without their code (a quarter of the size, and no instruction
  // cache misses in the epilogue)
  bool act = false;
  for (int i = 0; i < e.nops; ++i) act |= (e.op[i] & ((1 << VEC_KIND_SHIFT) - 1)) >= RELU;
  const dim3 grid((unsigned)((n + 31) / 32)), block(4 * 64);
  // one row block: only the eight-row groups of A that hold rows < M are loaded
#define KRN_SKINNY(AL)                                                                                          \
  do {                                                                                                          \
    if (act)                                                                                                    \
      hipLaunchKernelGGL((gemm_skinny<FMT, MT, 4, STAGES, true, AL>), grid, block, 0, stream, (const uint8_t*)a, \
                         (const uint8_t*)b, c, m, n, kbytes, lda, ldb, ldc, e);                                 \
    else                                                                                                        \
      hipLaunchKernelGGL((gemm_skinny<FMT, MT, 4, STAGES, false, AL>), grid, block, 0, stream, (const uint8_t*)a, \
                         (const uint8_t*)b, c, m, n, kbytes, lda, ldb, ldc, e);                                 \
  } while (0)
  if constexpr (MT == 1) {
    if (m <= 8) KRN_SKINNY(1);
    else if (m <= 16) KRN_SKINNY(2);
    else if (m <= 24) KRN_SKINNY(3);
    else KRN_SKINNY(4);
  } else {
    KRN_SKINNY(MT * 4);
  }
#undef KRN_SKINNY
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    krn_set_error("gemm launch: %s", hipGetErrorString(err));
    return (int)err;
  }
  return 0;
}

// M <= 128 rows with 16-byte aligned rows of a multiple of 128 bytes: one workgroup per 32 output columns, four
// waves (one per SIMD, all issuing MFMAs: fewer leave bf16 compute-bound at 128 rows). One row block and at most one
// workgroup per CU (N <= 8192): a four-stage ring per wave (128 KiB; fp8 M = 1 11.5 -> 11.2 us against two stages);
// more workgroups than CUs: two stages (64 KiB), so that two workgroups share a CU and one's reduction and epilogue
// overlap the other's stream (W8A8 M = 16, N = 14336: 15.4 us, against 18.7 us with four stages); more row blocks:
// two stages, 96 to 160 KiB.
template <int FMT>
static int launch_skinny(const void* a, const void* b, void* c, int64_t m, int64_t n, int64_t kbytes, int64_t lda,
                         int64_t ldb, int64_t ldc, const Epilogue& e, hipStream_t stream) {
  switch ((m + 31) / 32) {
    case 1:
      return (n + 31) / 32 <= 256 ? launch_skinny_mt<FMT, 1, 4>(a, b, c, m, n, kbytes, lda, ldb, ldc, e, stream)
                                  : launch_skinny_mt<FMT, 1, 2>(a, b, c, m, n, kbytes, lda, ldb, ldc, e, stream);
    case 2: return launch_skinny_mt<FMT, 2, 2>(a, b, c, m, n, kbytes, lda, ldb, ldc, e, stream);
    case 3: return launch_skinny_mt<FMT, 3, 2>(a, b, c, m, n, kbytes, lda, ldb, ldc, e, stream);
    case 4: return launch_skinny_mt<FMT, 4, 2>(a, b, c, m, n, kbytes, lda, ldb, ldc, e, stream);
  }
  krn_set_error("gemm: %lld rows are too many for the skinny kernel", (long long)m);
  return -1;
}

// 256 x 256 tiles (ragged at the edges).
template <int FMT>
static int launch_whole(const void* a, const void* b, void* c, int64_t m, int64_t n, int64_t kbytes, int64_t lda,
                        int64_t ldb, int64_t ldc, const Epilogue& e, hipStream_t stream) {
  // Two slices or more: the four-wave loop on 16x16 MFMAs (gemm_quad16). One slice (K = 128 bytes): fp8 the
  // eight-wave ping-pong, int8 and bf16/f16 the eight-wave direct-to-LDS ring.
  if (kbytes >= 256) return launch_quad16<FMT>(a, b, c, m, n, kbytes, lda, ldb, ldc, e, stream);
  if constexpr (FMT == FMT_FP8)
    return launch_pp<FMT, 4>(a, b, c, m, n, kbytes, lda, ldb, ldc, e, stream);
  else if constexpr (FMT == FMT_I8)
    return launch_pipe<FMT, 256, 256, 4, 2, 2, 128>(a, b, c, m, n, kbytes, lda, ldb, ldc, e, stream);
  else
    return launch_pipe<FMT, 256, 256, 4, 2, 4, 64>(a, b, c, m, n, kbytes, lda, ldb, ldc, e, stream);
}

// Up to one wave of 128 x 128 tiles (at most 256 tiles): the pipelined loop on 128 x 128 tiles with four waves, a
// 64 KiB ring (measured 20-40 % faster than the register-staged tiles at 1024^3 and 2048^3 for every format)
template <int FMT>
static int launch_mid(const void* a, const void* b, void* c, int64_t m, int64_t n, int64_t kbytes, int64_t lda,
                      int64_t ldb, int64_t ldc, const Epilogue& e, hipStream_t stream) {
  if constexpr (FMT == FMT_BF16 || FMT == FMT_F16)
    return launch_pipe<FMT, 128, 128, 2, 2, 4, 64>(a, b, c, m, n, kbytes, lda, ldb, ldc, e, stream);
  else
    return launch_pipe<FMT, 128, 128, 2, 2, 2, 128>(a, b, c, m, n, kbytes, lda, ldb, ldc, e, stream);
}

// 128 x 256 tiles, eight waves (64 x 64 each), for the products between one wave of 128 x 128 tiles and 128 tiles
// of 256 x 256 (bf16/f16 and int8; int8 with three 128-byte stages, 144 KiB: the W8A8 4096 x 14336 x 4096 column
// tail 49.9 -> 45.2 us against two)
template <int FMT>
static int launch_band(const void* a, const void* b, void* c, int64_t m, int64_t n, int64_t kbytes, int64_t lda,
                       int64_t ldb, int64_t ldc, const Epilogue& e, hipStream_t stream) {
  if constexpr (FMT == FMT_BF16 || FMT == FMT_F16)
    return launch_pipe<FMT, 128, 256, 2, 4, 4, 64>(a, b, c, m, n, kbytes, lda, ldb, ldc, e, stream);
  else if constexpr (FMT == FMT_I8)
    return launch_pipe<FMT, 128, 256, 2, 4, 3, 128>(a, b, c, m, n, kbytes, lda, ldb, ldc, e, stream);
  else
    return launch_gemm<FMT, 128, 128, 2, 2>(a, b, c, m, n, kbytes, lda, ldb, ldc, e, stream);
}

static int gemm_dispatch(int fmt, const void* a, const void* b, void* c, int64_t m, int64_t n, int64_t k,
                         int64_t elem, const Epilogue& e, hipStream_t stream) {
  const int64_t kbytes = k * elem, lda = k * elem, ldb = k * elem;
  const int64_t ldc = n;
  // Kernel choice on 256 CUs (measured at 1024^3 .. 8192^3 for every format). With K in whole 128-byte slices and
  // 16-byte aligned rows the pipelined direct-to-LDS loops serve everything but the skinny products:
  //   M <= 128: the skinny kernel (B streamed once, every CU busy);
  //   at least 128 tiles of 256 x 256 (ragged edges included): 256 x 256 tiles; at half the CUs already 20-40 %
  //   faster than smaller tiles, whose operands are re-read from L2 twice as often;
  //   up to 256 tiles of 128 x 128: 128 x 128 tiles, four waves;
  //   between: 128 x 256 tiles, eight waves (fp8: the register-staged 128 x 128 tiles, as fast there).
  // Otherwise (K ragged, unaligned rows) the register-staged, bounds-checked tiles, 256 x 256 when there are at
  // least 256 of them. The 256-row (128-row) operand panels must be addressable by 31-bit buffer offsets.
  const bool vec = kbytes % 16 == 0 && (uintptr_t)a % 16 == 0 && (uintptr_t)b % 16 == 0;
  const int64_t t256 = ((m + 255) / 256) * ((n + 255) / 256), t128 = ((m + 127) / 128) * ((n + 127) / 128);
  const bool piped = vec && kbytes % 128 == 0 && kbytes > 0 && m > 0 && n > 0;
  const bool skinny = piped && m <= 128;
  const bool whole = piped && t256 >= 128 && 256 * lda <= 0x7fffffff;
  const bool mid = piped && t128 <= 256 && 128 * lda <= 0x7fffffff;
  const bool band = piped && fmt != FMT_FP8 && 256 * ldb <= 0x7fffffff;
  const bool large = t256 >= 256 && vec;
  // A last wave of 256 x 256 tiles at most half full (W8A8 4096 x 14336: 896 tiles, 3.5 waves on 256 CUs) would
  // leave half the chip idle for a whole tile time. When the full waves cover whole columns of tiles, those
  // columns run as 256 x 256 tiles and the remaining columns as a second launch of 128 x 256 tiles (twice as many,
  // half the work each), which fills the last wave. The two launches write disjoint columns of C.
  const int64_t full_tiles = (t256 / 256) * 256, tile_rows = (m + 255) / 256;
  const bool split = whole && band && t256 % 256 != 0 && t256 % 256 <= 128 && full_tiles > 0 &&
                     full_tiles % tile_rows == 0;
  const int64_t n_split = split ? full_tiles / tile_rows * 256 : 0;
  Epilogue tail = e;  // the epilogue of the columns from n_split on: column vectors start at that column
  for (int i = 0; i < e.nops; ++i) {
    const int op = e.op[i] & ((1 << VEC_KIND_SHIFT) - 1), kind = e.op[i] >> VEC_KIND_SHIFT;
    if (op == MUL_COL || op == ADD_COL)
      tail.vec[i] = static_cast<const uint8_t*>(e.vec[i]) + n_split * (kind == 0 ? 4 : 2);
  }
  const int out_bytes = (e.out_kind == F32 || e.out_kind == I32) ? 4 : 2;
  const void* b_tail = static_cast<const uint8_t*>(b) + n_split * ldb;
  void* c_tail = static_cast<uint8_t*>(c) + n_split * out_bytes;
#define KRN_GEMM(F)                                                                                    \
  if (skinny) return launch_skinny<F>(a, b, c, m, n, kbytes, lda, ldb, ldc, e, stream);                \
  if (split) {                                                                                         \
    const int rc = launch_whole<F>(a, b, c, m, n_split, kbytes, lda, ldb, ldc, e, stream);             \
    if (rc != 0) return rc;                                                                            \
    return launch_band<F>(a, b_tail, c_tail, m, n - n_split, kbytes, lda, ldb, ldc, tail, stream);     \
  }                                                                                                    \
  if (whole) return launch_whole<F>(a, b, c, m, n, kbytes, lda, ldb, ldc, e, stream);                  \
  if (mid) return launch_mid<F>(a, b, c, m, n, kbytes, lda, ldb, ldc, e, stream);                      \
  if (band) return launch_band<F>(a, b, c, m, n, kbytes, lda, ldb, ldc, e, stream);                    \
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

extern "C" int krn_transpose16(const void* in, void* out, int64_t rows, int64_t cols, void* stream);

// The epilogue chain of a launch, checked: at most four known operations, a vector for every per-row or per-column
// one. `who` prefixes the error message.
static bool epilogue_of(Epilogue& e, int out_kind, int nops, const int* ops, const float* scalars,
                        const void* const* vectors, const char* who) {
  e.out_kind = out_kind;
  if (nops < 0 || nops > 4) {
    krn_set_error("%s: %d epilogue operations, at most 4", who, nops);
    return false;
  }
  e.nops = nops;
  for (int i = 0; i < nops; ++i) {
    e.op[i] = ops[i];
    e.scalar[i] = scalars ? scalars[i] : 0.0f;
    e.vec[i] = vectors ? vectors[i] : nullptr;
    const int op = ops[i] & ((1 << VEC_KIND_SHIFT) - 1), kind = ops[i] >> VEC_KIND_SHIFT;
    if (ops[i] < 0 || op > SILU || kind > 2 || (kind != 0 && (op >= RELU || op % 3 == 0))) {
      krn_set_error("%s: unknown epilogue operation %d", who, ops[i]);
      return false;
    }
    if (op < RELU && op % 3 != 0 && e.vec[i] == nullptr) {
      krn_set_error("%s: epilogue operation %d needs a vector", who, i);
      return false;
    }
  }
  return true;
}

extern "C" {

// See include/krn_amd.h for the contract of each entry point.
int krn_gemm_nt(int in_kind, const void* a, const void* b, void* c, int out_kind, int64_t m, int64_t n, int64_t k,
                int nops, const int* ops, const float* scalars, const void* const* vectors, void* stream) {
  Epilogue e{};
  if (!epilogue_of(e, out_kind, nops, ops, scalars, vectors, "gemm")) return -1;
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

// The NN product `a[rows, ks] @ b[ks, cols]` with B stored K x N: B is transposed into `bt` (N x K, n * k 16-bit
// elements) and the NT kernels run on it. Both launches go on `stream`, in that order.
// The NN products gemm_quad16 takes with B read K-major from LDS (no transposed copy): at least 128 tiles
// of 256 x 256, N a multiple of 256, K of 64 (whole 128-byte slices, at least two), 16-byte aligned operands, and
// panels addressable by 31-bit buffer offsets.
static bool nn_direct(const void* a, const void* b, int64_t m, int64_t n, int64_t k) {
  const int64_t t256 = ((m + 255) / 256) * (n / 256);
  return m > 0 && n > 0 && n % 256 == 0 && k % 64 == 0 && k >= 128 && t256 >= 128 && t256 <= 0x7fffffff &&
         (uintptr_t)a % 16 == 0 &&
         (uintptr_t)b % 16 == 0 && 256 * k * 2 <= 0x7fffffff && (k - 1) * n * 2 + 512 <= 0x7fffffff;
}

static int gemm_nn_through(int in_kind, const void* a, const void* b, void* c, int out_kind, int64_t m, int64_t n,
                           int64_t k, int nops, const int* ops, const float* scalars, const void* const* vectors,
                           void* bt, void* stream) {
  if (in_kind != BF16 && in_kind != F16) {
    krn_set_error("gemm_nn: operand kind %d; the NN product takes bf16 or f16 operands", in_kind);
    return -1;
  }
  if (m < 0 || n < 0 || k < 0) {
    krn_set_error("gemm_nn: negative extent");
    return -1;
  }
  if (nn_direct(a, b, m, n, k)) {
    Epilogue e{};
    if (!epilogue_of(e, out_kind, nops, ops, scalars, vectors, "gemm_nn")) return -1;
    if (out_kind != F32 && out_kind != F16 && out_kind != BF16) {
      krn_set_error("gemm_nn: output kind %d is not stored by the tile GEMM", out_kind);
      return -1;
    }
    const int64_t tiles = ((m + 255) / 256) * (n / 256);
    if (in_kind == BF16)
      hipLaunchKernelGGL((gemm_quad16<FMT_BF16, true>), dim3((unsigned)tiles), dim3(256), 0, (hipStream_t)stream,
                         (const uint8_t*)a, (const uint8_t*)b, c, m, n, k * 2, k * 2, n * 2, n, e);
    else
      hipLaunchKernelGGL((gemm_quad16<FMT_F16, true>), dim3((unsigned)tiles), dim3(256), 0, (hipStream_t)stream,
                         (const uint8_t*)a, (const uint8_t*)b, c, m, n, k * 2, k * 2, n * 2, n, e);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) {
      krn_set_error("gemm_nn launch: %s", hipGetErrorString(err));
      return (int)err;
    }
    return 0;
  }
  if (bt == nullptr && n > 0 && k > 0) {
    krn_set_error("gemm_nn: this product needs the transposed operand's workspace");
    return -1;
  }
  if (n > 0 && k > 0) {
    const int rc = krn_transpose16(b, bt, k, n, stream);
    if (rc) return rc;
  }
  return krn_gemm_nt(in_kind, a, bt, c, out_kind, m, n, k, nops, ops, scalars, vectors, stream);
}

extern "C" int64_t krn_gemm_nn_workspace(int64_t n, int64_t k) { return n < 0 || k < 0 ? 0 : n * k * 2; }

extern "C" int64_t krn_gemm_nn_workspace_for(const void* a, const void* b, int64_t m, int64_t n, int64_t k) {
  return nn_direct(a, b, m, n, k) ? 0 : krn_gemm_nn_workspace(n, k);
}

extern "C" int krn_gemm_nn(int in_kind, const void* a, const void* b, void* c, int out_kind, int64_t m, int64_t n,
                           int64_t k, int nops, const int* ops, const float* scalars, const void* const* vectors,
                           void* workspace, int64_t workspace_bytes, void* stream) {
  const int64_t need = nn_direct(a, b, m, n, k) ? 0 : krn_gemm_nn_workspace(n, k);
  if (need > 0 && (workspace == nullptr || workspace_bytes < need)) {
    krn_set_error("gemm_nn: the workspace holds %lld bytes, the transposed operand needs %lld",
                  (long long)workspace_bytes, (long long)need);
    return -1;
  }
  return gemm_nn_through(in_kind, a, b, c, out_kind, m, n, k, nops, ops, scalars, vectors, workspace, stream);
}

// The scratch of krn_gemm_nn_noalloc: the transposed B operand lives in this file-scope device array instead of a
// caller's workspace or an allocation. Every GPU the library runs on holds its own copy until the process ends. In
// host code `scratch` names a host-side stand-in, not the device memory: the device address comes from
// hipGetSymbolAddress, once per device, and only that address is handed to kernels.
constexpr int64_t KRN_NN_SCRATCH_BYTES = (int64_t)64 << 20;
static __device__ __align__(256) uint8_t scratch[KRN_NN_SCRATCH_BYTES];
constexpr int KRN_MAX_DEVICES = 64;

// Per device: the array's address, and an event recorded after the last eager call that used it. Every call first
// makes its stream wait (hipStreamWaitEvent, on the device) for that event, so two streams never hold the array at
// once (on the previous call's own stream the wait is already satisfied by stream order; it is kept unconditional so
// a stream handle reused after a destroy cannot skip it). The lock covers the look-up, that wait, the enqueue and the new record, so
// host threads are ordered too. A stream under graph capture neither waits nor records (an event of the eager world
// cannot order graph replays): a captured call is ordered only by the graph's and the caller's own dependencies.
struct ScratchUse {
  void* ptr = nullptr;
  hipEvent_t done = nullptr;  // recorded after the last eager call that used the array
  bool used = false;
};
static std::mutex scratch_lock;
static ScratchUse scratch_use[KRN_MAX_DEVICES];

// The device the call runs on: the stream's own device, which must be the current one (the address comes from
// the current device's array). The null stream runs on the current device.
static int scratch_device(hipStream_t stream) {
  int device = -1;
  hipError_t rc = hipGetDevice(&device);
  if (rc != hipSuccess || device < 0 || device >= KRN_MAX_DEVICES) {
    krn_set_error("gemm_nn_noalloc: no usable current device (%s, ordinal %d)", hipGetErrorString(rc), device);
    return -1;
  }
  if (stream != nullptr) {
    int of_stream = -1;
    rc = hipStreamGetDevice(stream, &of_stream);
    if (rc != hipSuccess) {
      krn_set_error("gemm_nn_noalloc: hipStreamGetDevice failed: %s", hipGetErrorString(rc));
      return -1;
    }
    if (of_stream != device) {
      krn_set_error("gemm_nn_noalloc: the stream belongs to device %d but device %d is current; make the stream's "
                    "device current", of_stream, device);
      return -1;
    }
  }
  return device;
}

// Set-up of one device, on its first call, with the lock held: the array's address and the ordering event.
static bool scratch_setup(int device) {
  ScratchUse& use = scratch_use[device];
  if (use.ptr != nullptr) return true;
  void* ptr = nullptr;
  hipError_t rc = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
  if (rc != hipSuccess || ptr == nullptr) {
    krn_set_error("gemm_nn_noalloc: hipGetSymbolAddress of the scratch array failed: %s", hipGetErrorString(rc));
    return false;
  }
  rc = hipEventCreateWithFlags(&use.done, hipEventDisableTiming);
  if (rc != hipSuccess) {
    krn_set_error("gemm_nn_noalloc: hipEventCreateWithFlags failed: %s", hipGetErrorString(rc));
    return false;
  }
  use.ptr = ptr;
  return true;
}

extern "C" int64_t krn_gemm_nn_noalloc_limit(void) { return KRN_NN_SCRATCH_BYTES; }

extern "C" int krn_gemm_nn_noalloc(int in_kind, const void* a, const void* b, void* c, int out_kind, int64_t m,
                                   int64_t n, int64_t k, int nops, const int* ops, const float* scalars,
                                   const void* const* vectors, void* stream) {
  const int64_t need = nn_direct(a, b, m, n, k) ? 0 : krn_gemm_nn_workspace(n, k);
  if (need > KRN_NN_SCRATCH_BYTES) {
    krn_set_error("gemm_nn_noalloc: B of %lld x %lld needs %lld bytes of scratch; the library holds %lld "
                  "(use krn_gemm_nn with a workspace)", (long long)k, (long long)n, (long long)need,
                  (long long)KRN_NN_SCRATCH_BYTES);
    return -1;
  }
  if (need == 0) return gemm_nn_through(in_kind, a, b, c, out_kind, m, n, k, nops, ops, scalars, vectors, nullptr,
                                        stream);
  hipStream_t s = (hipStream_t)stream;
  const int device = scratch_device(s);
  if (device < 0) return -1;
  hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
  hipError_t rc = hipStreamIsCapturing(s, &capture);
  if (rc != hipSuccess) {
    krn_set_error("gemm_nn_noalloc: hipStreamIsCapturing failed: %s", hipGetErrorString(rc));
    return -1;
  }
  const bool eager = capture == hipStreamCaptureStatusNone;
  std::lock_guard<std::mutex> hold(scratch_lock);
  if (!scratch_setup(device)) return -1;
  ScratchUse& use = scratch_use[device];
  if (eager && use.used && (rc = hipStreamWaitEvent(s, use.done, 0)) != hipSuccess) {
    krn_set_error("gemm_nn_noalloc: hipStreamWaitEvent failed: %s", hipGetErrorString(rc));
    return -1;
  }
  const int status = gemm_nn_through(in_kind, a, b, c, out_kind, m, n, k, nops, ops, scalars, vectors, use.ptr, s);
  if (status != 0 || !eager) return status;
  if ((rc = hipEventRecord(use.done, s)) != hipSuccess) {
    krn_set_error("gemm_nn_noalloc: hipEventRecord failed: %s", hipGetErrorString(rc));
    return -1;
  }
  use.used = true;
  return 0;
}

// Whole 128 x 128 tiles (rows and cols multiples of 128, 16-byte aligned): rows land in LDS with 16-byte loads (256
// contiguous bytes per 16 lanes); each thread then reads one 8 x 8 block with eight 16-byte LDS reads, transposes it
// in registers (v_perm_b32 pairs the 16-bit halves of two rows) and writes eight 16-byte pieces of output rows, 256
// contiguous bytes per 16 lanes (8192^2: 70 -> 56 us).
__global__ __launch_bounds__(256) void transpose16_tiles(const uint16_t* __restrict__ in, uint16_t* __restrict__ out,
                                                         int64_t rows, int64_t cols) {
  constexpr int P = 128 + 8;  // LDS row pitch in elements: 16 bytes of padding keep the block reads off one bank
  __shared__ __attribute__((aligned(16))) uint16_t tile[128 * P];
  const int t = threadIdx.x;
  const int64_t r0 = (int64_t)blockIdx.y * 128, c0 = (int64_t)blockIdx.x * 128;
#pragma unroll
  for (int p = 0; p < 8; ++p) {
    const int row = p * 16 + (t >> 4), cb = (t & 15) * 8;
    *reinterpret_cast<u32x4*>(tile + row * P + cb) =
        __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(in + (r0 + row) * cols + c0 + cb));
  }
  __syncthreads();
  const int bi = t & 15, bj = t >> 4;
  u32x4 r[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) r[i] = *reinterpret_cast<const u32x4*>(tile + (bi * 8 + i) * P + bj * 8);
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const uint32_t sel = (j & 1) ? 0x07060302u : 0x05040100u;  // the high or the low halves of two words
    u32x4 o;
#pragma unroll
    for (int w = 0; w < 4; ++w) o[w] = __builtin_amdgcn_perm(r[2 * w + 1][j >> 1], r[2 * w][j >> 1], sel);
    __builtin_nontemporal_store(o, reinterpret_cast<u32x4*>(out + (c0 + bj * 8 + j) * rows + r0 + bi * 8));
  }
}

extern "C" int krn_transpose16(const void* in, void* out, int64_t rows, int64_t cols, void* stream) {
  if (rows < 0 || cols < 0) {
    krn_set_error("transpose: negative extent");
    return -1;
  }
  if (rows == 0 || cols == 0) return 0;
  if (rows % 128 == 0 && cols % 128 == 0 && (uintptr_t)in % 16 == 0 && (uintptr_t)out % 16 == 0 &&
      cols / 128 <= 0x7fffffff && rows / 128 <= 65535) {
    hipLaunchKernelGGL(transpose16_tiles, dim3((unsigned)(cols / 128), (unsigned)(rows / 128)), dim3(256), 0,
                       (hipStream_t)stream, (const uint16_t*)in, (uint16_t*)out, rows, cols);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) {
      krn_set_error("transpose launch: %s", hipGetErrorString(err));
      return (int)err;
    }
    return 0;
  }
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
