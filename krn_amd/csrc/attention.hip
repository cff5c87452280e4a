// Flash attention forward for gfx950: O = softmax(scale * Q K^T masked) V, one pass over the keys per query tile.
//
// This is the lowering of krn's flash-attention tile program (reference examples/04_libraries/08_flash_attention.py
// :35-59): `s = (q @ k^T) * scale`, an optional causal `where(k_pos <= q_pos, s, -1e30)`, the running row maximum
// `m`, row sum `total` and output `acc` rescaled by `exp2(m - m_new)`, `acc += p.to(dtype) @ v`, and finally
// `o = (acc / total).to(dtype)`. Keys past the end of the sequence are invalid lanes: they take no part in the
// maximum, the sum or the product.
//
// Layout (MI355X-first). A workgroup owns 128 query rows of one (batch, head); each of its 4 waves owns 32 rows and
// computes the transposed products S^T = K Q^T and O^T += V^T P^T with v_mfma_f32_32x32x16_{bf16,f16}. In that form
// every lane holds one query row (lane & 31) and 16 of the keys of a 32-key block (its half-wave partner holds the
// other 16), so the row maximum and sum are lane-local plus one exchange with lane ^ 32, the rescale of O is
// lane-local, and P feeds the next MFMA straight from registers as its B operand. Q stays in registers for the
// whole pass. K and V tiles of 64 keys stream through LDS in a two-slot ring filled by direct-to-LDS loads
// (global_load_lds_dwordx4) while the previous tile multiplies; both keep the row-major [key][d] layout of global
// memory. K is read as the A operand of S^T with 16-byte reads (chunk c of key row r at slot c ^ (r & 15)); V is
// read as the A operand of O^T with ds_read_b64_tr_b16, which hands each lane four keys of one d column, so V never
// needs a transposing copy (chunk c of key row r at slot c ^ 4 (r & 3)). Two workgroups share a CU, so each SIMD
// interleaves the softmax of one wave with the MFMAs of another.
//
// Shortcuts. Exact: the row maximum of an unmasked tile is taken on the raw scores and scaled once (rounding is
// monotonic, scale > 0); tiles wholly past a wave's last causal row are skipped (their p are exp2(-1e30 - m) = 0 and
// their corr is 1). Equal up to rounding: the exponent argument s * scale - m is one fused multiply-add on unmasked
// tiles, and the running maximum used as the exponent base is refreshed only when it is beaten by more than 8
// (p <= 2^8), which scales p, acc and total by the same power of two and leaves acc / total unchanged.
#include "common.h"

namespace krn {

typedef short v4s __attribute__((ext_vector_type(4)));

template <bool BF>
struct Half;
template <>
struct Half<true> {
  __device__ static uint32_t pack(float lo, float hi) {
    typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, bf2{(__bf16)lo, (__bf16)hi});  // v_cvt_pk_bf16_f32, nearest even
  }
  __device__ static uint16_t from(float x) { return f2bf(x); }
  __device__ static void mma(f32x16& c, u32x4 a, u32x4 b) {
    c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0,
                                                0, 0);
  }
};
template <>
struct Half<false> {
  __device__ static uint32_t pack(float lo, float hi) { return (uint32_t)f2h(lo) | ((uint32_t)f2h(hi) << 16); }
  __device__ static uint16_t from(float x) { return f2h(x); }
  __device__ static void mma(f32x16& c, u32x4 a, u32x4 b) {
    c = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0,
                                               0);
  }
};

constexpr int BQ = 128;   // query rows per workgroup
constexpr int BKEY = 64;  // keys per LDS tile

// LDS swizzles of the [key][d] tiles (64 banks serve 256 bytes per cycle). K: the 16-byte reads of 16 consecutive
// keys must hit 16 distinct positions modulo 256 bytes. V: the transposed 8-byte reads cover 4 consecutive keys x
// 64 bytes per 32 lanes. D = 128 (256-byte rows) and D = 64 (128-byte rows) need different XOR patterns.
template <int D>
__device__ __forceinline__ int k_slot(int key, int chunk) {
  return D == 128 ? chunk ^ (key & 15) : chunk ^ ((key >> 1) & 7);
}
template <int D>
__device__ __forceinline__ int v_slot(int key, int chunk) {
  return D == 128 ? chunk ^ ((key & 3) << 2) : chunk ^ (((key >> 1) & 1) << 2);
}

template <bool BF, int D, bool CAUSAL>
__global__ __launch_bounds__(256, 2) void attention_fwd(const uint16_t* __restrict__ Q, const uint16_t* __restrict__ K,
                                                        const uint16_t* __restrict__ V, uint16_t* __restrict__ O,
                                                        int64_t sq, int64_t sk, float scale, int q_tiles) {
  static_assert(D == 64 || D == 128, "head dimension 64 or 128");
  constexpr int DCH = D / 8;                // 16-byte chunks per key row
  constexpr int TILE_BYTES = BKEY * D * 2;  // one K (or V) tile
  constexpr int ROWS_PER_LOAD = 1024 / (D * 2);
  constexpr int LOADS = BKEY / ROWS_PER_LOAD / 4;  // wave load instructions per tile, per operand
  static_assert(LOADS * ROWS_PER_LOAD * 4 == BKEY, "whole wave loads");
  static_assert(DCH <= 16, "swizzle range");
  __shared__ __attribute__((aligned(1024))) uint8_t lds[2][2 * TILE_BYTES];

  // Heavy (late) query tiles first, so the causal tail is spread over the machine.
  const int head = blockIdx.x / q_tiles;
  const int qt = CAUSAL ? (q_tiles - 1 - (int)(blockIdx.x % q_tiles)) : (int)(blockIdx.x % q_tiles);
  const int64_t q0 = (int64_t)qt * BQ;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6, half = lane >> 5, r32 = lane & 31;
  const uint16_t* q = Q + (int64_t)head * sq * D;
  const uint16_t* k = K + (int64_t)head * sk * D;
  const uint16_t* v = V + (int64_t)head * sk * D;
  uint16_t* o = O + (int64_t)head * sq * D;

  // this lane's query row and its Q fragments (B operand of S^T = K Q^T): 8 contiguous d per MFMA step
  const int64_t qrow = q0 + wave * 32 + r32;
  u32x4 qf[D / 16];
#pragma unroll
  for (int s = 0; s < D / 16; ++s)
    qf[s] = qrow < sq ? *reinterpret_cast<const u32x4*>(q + qrow * D + s * 16 + half * 8) : u32x4{};

  f32x16 acc[D / 32];
#pragma unroll
  for (int i = 0; i < D / 32; ++i) acc[i] = f32x16{};
  float m = -1.0e30f, total = 0.0f;

  const int64_t kend = CAUSAL ? min(sk, q0 + BQ) : sk;
  const int64_t wave_first_q = q0 + wave * 32, wave_last_q = wave_first_q + 31;
  const int ntiles = (int)((kend + BKEY - 1) / BKEY);

  // direct-to-LDS loads: lane -> (row within its 1 KiB block, slot); rows past the sequence read the last row
  // (finite data whose scores are masked to -inf, so their p is 0)
  const int lrow = lane / DCH, lslot = lane % DCH;
#define KRN_FA_ISSUE(tile)                                                                                    \
  do {                                                                                                        \
    uint8_t* st = &lds[(tile) & 1][0];                                                                        \
    _Pragma("unroll") for (int j = 0; j < LOADS; ++j) {                                                       \
      const int row = (wave * LOADS + j) * ROWS_PER_LOAD + lrow;                                              \
      const int64_t key = min((int64_t)(tile) * BKEY + row, sk - 1);                                          \
      __builtin_amdgcn_global_load_lds((const void*)(k + key * D + k_slot<D>(row, lslot) * 8),                    \
                                       (__attribute__((address_space(3))) void*)(st + (wave * LOADS + j) * 1024), \
                                       16, 0, 0);                                                             \
      __builtin_amdgcn_global_load_lds(                                                                       \
          (const void*)(v + key * D + v_slot<D>(row, lslot) * 8),                                                \
          (__attribute__((address_space(3))) void*)(st + TILE_BYTES + (wave * LOADS + j) * 1024), 16, 0, 0);  \
    }                                                                                                         \
  } while (0)
#define KRN_FA_PUBLISH()                                                                                      \
  do {                                                                                                        \
    __builtin_amdgcn_s_waitcnt(0x0070 | 0x0f00);  /* vmcnt(0) */                                             \
    __builtin_amdgcn_s_waitcnt(0xc07f & ~0x0f00); /* lgkmcnt(0) */                                            \
    __builtin_amdgcn_s_barrier();                                                                             \
  } while (0)

  if (ntiles > 0) KRN_FA_ISSUE(0);
  KRN_FA_PUBLISH();

  // V^T fragment address pieces for ds_read_b64_tr_b16: lane group g = lane / 16 reads keys
  // K0 + (lane % 16) / 4 at d columns dblk * 32 + (g % 2) * 16 + 4 * (lane % 4)
  const int g = lane >> 4, a16 = lane & 15;
  const int tr_key = (g >> 1) * 4 + (a16 >> 2);
  const int tr_col = (g & 1) * 16 + 4 * (a16 & 3);

  for (int tile = 0; tile < ntiles; ++tile) {
    const int64_t c0 = (int64_t)tile * BKEY;
    if (tile + 1 < ntiles) KRN_FA_ISSUE(tile + 1);
    const bool active = !CAUSAL || c0 <= wave_last_q;
    if (active) {
      const uint8_t* st = &lds[tile & 1][0];
      const u32x4* kl = reinterpret_cast<const u32x4*>(st);
      // S^T for the two 32-key halves of the tile
      f32x16 s[2];
#pragma unroll
      for (int hb = 0; hb < 2; ++hb) s[hb] = f32x16{};
      // the two halves interleaved, so consecutive MFMAs never wait for each other's result
#pragma unroll
      for (int j = 0; j < D / 16; ++j)
#pragma unroll
        for (int hb = 0; hb < 2; ++hb) {
          const int key = hb * 32 + r32;
          Half<BF>::mma(s[hb], kl[key * DCH + k_slot<D>(key, j * 2 + half)], qf[j]);
        }
      const bool masked = c0 + BKEY > sk || (CAUSAL && c0 + BKEY - 1 > wave_first_q) || !(scale > 0.0f);
      float tmax;
      if (!masked) {
        float raw = s[0][0];
#pragma unroll
        for (int hb = 0; hb < 2; ++hb)
#pragma unroll
          for (int r = 0; r < 16; ++r) raw = fmaxf(raw, s[hb][r]);
        tmax = raw * scale;
      } else {
        tmax = -INFINITY;
        const int key0 = (int)c0 + half * 4, row = (int)qrow, valid = (int)(sk - c0);
#pragma unroll
        for (int hb = 0; hb < 2; ++hb)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int key = key0 + hb * 32 + (r >> 2) * 8 + (r & 3);
            float x = s[hb][r] * scale;
            if (CAUSAL && key > row) x = -1.0e30f;
            if (key - (int)c0 >= valid) x = -INFINITY;  // an invalid lane: no part in the max, sum or product
            s[hb][r] = x;
            tmax = fmaxf(tmax, x);
          }
      }
      tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
      // Lazy rescale: the exponent base m only moves when some row maximum of the wave exceeds it by more than
      // 8 (so every p <= 2^8); acc and total are then rescaled by exp2(m - m_new). Keeping a stale base scales p,
      // acc and total alike, which leaves acc / total unchanged up to rounding.
      if (__builtin_amdgcn_ballot_w64(tmax > m + 8.0f) != 0) {
        const float m_new = fmaxf(m, tmax);
        const float corr = __builtin_amdgcn_exp2f(m - m_new);
        total = total * corr;
#pragma unroll
        for (int i = 0; i < D / 32; ++i)
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[i][r] *= corr;
        m = m_new;
      }
      // p = exp2(s - m) in f32 for the sum, packed to 16 bits as P^T, the B operand: [half block][k16 step]
      float psum = 0.0f;
      u32x4 pf[2][2];
      const float neg_m = -m;
#pragma unroll
      for (int hb = 0; hb < 2; ++hb)
#pragma unroll
        for (int step = 0; step < 2; ++step) {
          uint32_t w[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const float x0 = s[hb][step * 8 + 2 * j], x1 = s[hb][step * 8 + 2 * j + 1];
            const float p0 = __builtin_amdgcn_exp2f(masked ? x0 + neg_m : __builtin_fmaf(x0, scale, neg_m));
            const float p1 = __builtin_amdgcn_exp2f(masked ? x1 + neg_m : __builtin_fmaf(x1, scale, neg_m));
            psum += p0;
            psum += p1;
            w[j] = Half<BF>::pack(p0, p1);
          }
          pf[hb][step] = u32x4{w[0], w[1], w[2], w[3]};
        }
      psum += __shfl_xor(psum, 32);
      total = total + psum;
      // O^T += V^T P^T: A operand lane = d row, the same 8 keys per lane as P (two 4-key transposed reads)
      // (the D / 32 accumulators innermost, so consecutive MFMAs are independent)
#pragma unroll
      for (int hb = 0; hb < 2; ++hb) {
#pragma unroll
        for (int step = 0; step < 2; ++step)
#pragma unroll
          for (int i = 0; i < D / 32; ++i) {
            u32x4 va;
#pragma unroll
            for (int part = 0; part < 2; ++part) {
              const int key = hb * 32 + step * 16 + part * 8 + tr_key;
              const int col = i * 32 + tr_col;  // 4 consecutive d: half a 16-byte chunk
              const int off = key * (D * 2) + v_slot<D>(key, col >> 3) * 16 + (col & 7) * 2;
              const v4s x = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                  (__attribute__((address_space(3))) v4s*)(st + TILE_BYTES + off));
              const u32x2 w = __builtin_bit_cast(u32x2, x);
              va[part * 2] = w[0];
              va[part * 2 + 1] = w[1];
            }
            Half<BF>::mma(acc[i], va, pf[hb][step]);
          }
      }
    }
    KRN_FA_PUBLISH();
  }
#undef KRN_FA_ISSUE
#undef KRN_FA_PUBLISH

  if (qrow < sq) {
#pragma unroll
    for (int i = 0; i < D / 32; ++i)
#pragma unroll
      for (int gq = 0; gq < 4; ++gq) {
        const int d = i * 32 + gq * 8 + half * 4;
        const uint32_t lo = Half<BF>::pack(acc[i][gq * 4 + 0] / total, acc[i][gq * 4 + 1] / total);
        const uint32_t hi = Half<BF>::pack(acc[i][gq * 4 + 2] / total, acc[i][gq * 4 + 3] / total);
        *reinterpret_cast<uint2*>(o + qrow * D + d) = uint2{lo, hi};
      }
  }
}

}  // namespace krn

using namespace krn;

template <bool BF, int D, bool CAUSAL>
static void launch_attention(const void* q, const void* k, const void* v, void* o, int64_t bh, int64_t sq,
                             int64_t sk, float scale, hipStream_t stream) {
  const int q_tiles = (int)((sq + BQ - 1) / BQ);
  dim3 grid((unsigned)(bh * q_tiles)), block(256);
  hipLaunchKernelGGL((attention_fwd<BF, D, CAUSAL>), grid, block, 0, stream, (const uint16_t*)q, (const uint16_t*)k,
                     (const uint16_t*)v, (uint16_t*)o, sq, sk, scale, q_tiles);
}

extern "C" int krn_attention_fwd(int kind, const void* q, const void* k, const void* v, void* o, int64_t bh,
                                 int64_t sq, int64_t sk, int64_t d, float scale, int causal, void* stream) {
  if (kind != BF16 && kind != F16) {
    krn_set_error("attention: element kind %d; bf16 or f16 tensors only", kind);
    return -1;
  }
  if (d != 64 && d != 128) {
    krn_set_error("attention: head dimension %lld; 64 or 128 only", (long long)d);
    return -1;
  }
  if (bh < 0 || sq < 0 || sk < 0) {
    krn_set_error("attention: negative extent");
    return -1;
  }
  if ((uintptr_t)q % 16 || (uintptr_t)k % 16 || (uintptr_t)v % 16 || (uintptr_t)o % 16) {
    krn_set_error("attention: tensors must be 16-byte aligned");
    return -1;
  }
  const int64_t blocks = bh * ((sq + BQ - 1) / BQ);
  if (blocks == 0) return 0;
  if (blocks > 0x7fffffff) {
    krn_set_error("attention: %lld workgroups exceed the grid limit", (long long)blocks);
    return -1;
  }
  if (sk == 0) {
    // no keys: the tile program divides 0 by 0
    krn_set_error("attention: an empty key sequence has no softmax");
    return -1;
  }
  hipStream_t s = (hipStream_t)stream;
  const bool bf = kind == BF16;
#define KRN_FA(BFV, DV)                                                       \
  (causal ? launch_attention<BFV, DV, true>(q, k, v, o, bh, sq, sk, scale, s) \
          : launch_attention<BFV, DV, false>(q, k, v, o, bh, sq, sk, scale, s))
  if (bf && d == 128) KRN_FA(true, 128);
  else if (bf) KRN_FA(true, 64);
  else if (d == 128) KRN_FA(false, 128);
  else KRN_FA(false, 64);
#undef KRN_FA
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    krn_set_error("attention launch: %s", hipGetErrorString(err));
    return (int)err;
  }
  return 0;
}
