// Shared device helpers for the gfx950 tile kernels: vector types, rounding of float32 to the 16-bit storage
// formats, and the error slot of the C ABI.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace krn {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef int i32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Element kinds shared with the host (include/krn_amd.h).
enum Kind : int { F32 = 0, F16 = 1, BF16 = 2, F8E4M3 = 3, I8 = 4, I32 = 5 };

// float32 -> bfloat16 word, ties to even; a NaN keeps its sign and top payload and is made quiet
// (the rounding krn's HIP renderer writes, reference compiler/hip.py:123-130). gfx950's v_cvt_pk_bf16_f32 rounds
// exactly so, denormals and NaN payloads included (checked bit for bit against the integer form
// (u + 0x7fff + ((u >> 16) & 1)) >> 16, NaN -> (u >> 16) | 0x40, over every 7th float32 pattern and every pattern
// of the denormal, largest-finite and NaN ranges), at one instruction per two values instead of a branch per value.
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t f2bf2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, bf16x2{(__bf16)lo, (__bf16)hi});
}
__device__ __forceinline__ uint16_t f2bf(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }

__device__ __forceinline__ float bf2f(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

// float32 -> IEEE half word, round to nearest even (the hardware conversion).
__device__ __forceinline__ uint16_t f2h(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }

__device__ __forceinline__ float h2f(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }

// A buffer resource over `bytes` bytes from `base` (raw 32-bit offsets, no stride, no swizzle; at most 2^31 - 1).
// Loads past the end return zeros instead of touching memory: that is how the whole-tile GEMMs read the ragged
// last rows of an operand.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t panel_rsrc(const void* base, int64_t bytes = 0x7fffffff) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)min(bytes, (int64_t)0x7fffffff),
                                           0x00020000);
}

// 16 bytes per lane from resource offset voff + soff straight into LDS: the wave's 64 lanes fill 1 KiB at `dst`
// (buffer_load_dwordx4 ... lds). A device function so that the host pass never sees the builtin.
__device__ __forceinline__ void buffer_to_lds16(__amdgpu_buffer_rsrc_t r, void* dst, uint32_t voff, int soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)dst, 16, voff, soff, 0, 0);
}

}  // namespace krn

// Host side: the last error message of the calling thread, read through krn_amd_last_error().
void krn_set_error(const char* fmt, ...);
