// Flash attention forward for gfx950: O = softmax(scale * Q K^T masked) V, one pass over the keys per query tile.
//
// This is the lowering of krn's flash-attention tile program (reference examples/04_libraries/08_flash_attention.py
// :35-59): `s = (q @ k^T) * scale`, an optional causal `where(k_pos <= q_pos, s, -1e30)`, the running row maximum
// `m`, row sum `total` and output `acc` rescaled by `exp2(m - m_new)`, `acc += p.to(dtype) @ v`, and finally
// `o = (acc / total).to(dtype)`. Keys past the end of the sequence are invalid lanes: they take no part in the
// maximum, the sum or the product.
//
// Layout (MI355X-first): a workgroup owns 128 query rows of one (batch, head); each of its 4 waves owns 32 rows and
// computes the transposed products S^T = K Q^T and O^T += V^T P^T with v_mfma_f32_32x32x16_{bf16,f16}. In that form
// every lane holds one query row (lane & 31) and 16 of the keys of a 32-key block (its half-wave partner holds the
// other 16), so the row maximum and sum are lane-local plus one exchange with lane ^ 32, the rescale of O is
// lane-local, and P feeds the next MFMA straight from registers as its B operand. K and V^T tiles of 64 keys are
// staged in LDS, double buffered; K rows are 16-byte-chunk swizzled by (key & 7) and V^T rows 8-byte-unit swizzled
// by f(d) = (d ^ (d >> 3)) & 15, which keeps both the transposing writes and the fragment reads conflict-free.
#include "common.h"

namespace krn {

template <bool BF>
struct Half;
template <>
struct Half<true> {
  __device__ static uint16_t from(float x) { return f2bf(x); }
  __device__ static void mma(f32x16& c, u32x4 a, u32x4 b) {
    c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0,
                                                0, 0);
  }
};
template <>
struct Half<false> {
  __device__ static uint16_t from(float x) { return f2h(x); }
  __device__ static void mma(f32x16& c, u32x4 a, u32x4 b) {
    c = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0,
                                               0);
  }
};

constexpr int BQ = 128;  // query rows per workgroup
constexpr int BKEY = 64;  // keys per LDS tile

__device__ __forceinline__ int vt_unit(int d, int unit) { return unit ^ ((d ^ (d >> 3)) & 15); }

template <bool BF, int D, bool CAUSAL>
__global__ __launch_bounds__(256, 1) void attention_fwd(const uint16_t* __restrict__ Q, const uint16_t* __restrict__ K,
                                                        const uint16_t* __restrict__ V, uint16_t* __restrict__ O,
                                                        int64_t sq, int64_t sk, float scale, int q_tiles) {
  static_assert(D == 64 || D == 128, "head dimension 64 or 128");
  constexpr int DCH = D / 8;                         // 16-byte chunks per K row
  constexpr int KT_BYTES = BKEY * D * 2;             // one K tile
  constexpr int VT_BYTES = D * BKEY * 2;             // one V^T tile
  __shared__ __attribute__((aligned(16))) uint8_t lds[2][KT_BYTES + VT_BYTES];

  // Heavy (late) query tiles first, so the causal tail is spread over the machine.
  const int tile_linear = blockIdx.x;
  const int head = tile_linear / q_tiles;
  const int qt = CAUSAL ? (q_tiles - 1 - tile_linear % q_tiles) : tile_linear % q_tiles;
  const int64_t q0 = (int64_t)qt * BQ;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6, half = lane >> 5, r32 = lane & 31;
  const uint16_t* q = Q + (int64_t)head * sq * D;
  const uint16_t* k = K + (int64_t)head * sk * D;
  const uint16_t* v = V + (int64_t)head * sk * D;
  uint16_t* o = O + (int64_t)head * sq * D;

  // This lane's query row and its Q fragments (B operand of S^T = K Q^T): 8 contiguous d per MFMA step.
  const int64_t qrow = q0 + wave * 32 + r32;
  u32x4 qf[D / 16];
#pragma unroll
  for (int s = 0; s < D / 16; ++s)
    qf[s] = qrow < sq ? *reinterpret_cast<const u32x4*>(q + qrow * D + s * 16 + half * 8) : u32x4{};

  f32x16 acc[D / 32];
#pragma unroll
  for (int i = 0; i < D / 32; ++i) acc[i] = f32x16{};
  float m = -1.0e30f, total = 0.0f;

  // key range of this workgroup and of this wave
  int64_t kend = sk;
  if (CAUSAL) kend = min(sk, q0 + BQ);
  const int64_t wave_last_q = q0 + wave * 32 + 31;
  const int ntiles = (int)((kend + BKEY - 1) / BKEY);

  // staging: K tile = 64 rows x DCH chunks; V tile = 16 groups of 4 keys x DCH chunks (4 rows per thread)
  constexpr int KLOADS = BKEY * DCH / 256;           // 16-byte K chunks per thread
  constexpr int VGROUPS = BKEY / 4 * DCH;            // (4-key, 8-d) blocks per tile
  constexpr int VLOADS = (VGROUPS + 255) / 256;      // blocks per thread (the last round may be partial)
  static_assert(KLOADS >= 1 && BKEY * DCH % 256 == 0, "K tile splits evenly over the workgroup");
  u32x4 kr[KLOADS], vr[VLOADS][4];

#define KRN_FA_LOAD(tile)                                                                                      \
  do {                                                                                                         \
    const int64_t c0 = (int64_t)(tile) * BKEY;                                                                 \
    _Pragma("unroll") for (int i = 0; i < KLOADS; ++i) {                                                       \
      const int id = t + 256 * i, key = id / DCH, ch = id % DCH;                                               \
      kr[i] = c0 + key < sk ? *reinterpret_cast<const u32x4*>(k + (c0 + key) * D + ch * 8) : u32x4{};          \
    }                                                                                                          \
    _Pragma("unroll") for (int i = 0; i < VLOADS; ++i) {                                                       \
      const int id = t + 256 * i, group = id / DCH, ch = id % DCH;                                             \
      _Pragma("unroll") for (int r = 0; r < 4; ++r) {                                                          \
        const int64_t key = c0 + group * 4 + r;                                                                \
        vr[i][r] = (id < VGROUPS && key < sk) ? *reinterpret_cast<const u32x4*>(v + key * D + ch * 8) : u32x4{}; \
      }                                                                                                        \
    }                                                                                                          \
  } while (0)

#define KRN_FA_STORE(buf)                                                                                      \
  do {                                                                                                         \
    u32x4* kl = reinterpret_cast<u32x4*>(&lds[buf][0]);                                                        \
    _Pragma("unroll") for (int i = 0; i < KLOADS; ++i) {                                                       \
      const int id = t + 256 * i, key = id / DCH, ch = id % DCH;                                               \
      kl[key * DCH + (ch ^ (key & 7))] = kr[i];                                                                \
    }                                                                                                          \
    uint2* vl = reinterpret_cast<uint2*>(&lds[buf][KT_BYTES]);                                                 \
    _Pragma("unroll") for (int i = 0; i < VLOADS; ++i) {                                                       \
      const int id = t + 256 * i, group = id / DCH, ch = id % DCH;                                             \
      if (id < VGROUPS) _Pragma("unroll") for (int e = 0; e < 8; ++e) {                                       \
        const int d = ch * 8 + e;                                                                              \
        const uint32_t w = e >> 1, sh = (e & 1) * 16;                                                          \
        uint32_t k0 = (vr[i][0][w] >> sh) & 0xffffu, k1 = (vr[i][1][w] >> sh) & 0xffffu;                       \
        uint32_t k2 = (vr[i][2][w] >> sh) & 0xffffu, k3 = (vr[i][3][w] >> sh) & 0xffffu;                       \
        vl[d * (BKEY / 4) + vt_unit(d, group)] = uint2{k0 | (k1 << 16), k2 | (k3 << 16)};                      \
      }                                                                                                        \
    }                                                                                                          \
  } while (0)

  if (ntiles > 0) {
    KRN_FA_LOAD(0);
    KRN_FA_STORE(0);
  }
  __syncthreads();

  for (int tile = 0; tile < ntiles; ++tile) {
    const int buf = tile & 1;
    const int64_t c0 = (int64_t)tile * BKEY;
    if (tile + 1 < ntiles) KRN_FA_LOAD(tile + 1);

    const bool active = !CAUSAL || c0 <= wave_last_q;
    if (active) {
      const u32x4* kl = reinterpret_cast<const u32x4*>(&lds[buf][0]);
      const uint2* vl = reinterpret_cast<const uint2*>(&lds[buf][KT_BYTES]);
      // S^T for the two 32-key halves of the tile
      f32x16 st[2];
#pragma unroll
      for (int hb = 0; hb < 2; ++hb) {
        st[hb] = f32x16{};
        const int key = hb * 32 + r32;
#pragma unroll
        for (int s = 0; s < D / 16; ++s) {
          const int ch = s * 2 + half;
          Half<BF>::mma(st[hb], kl[key * DCH + (ch ^ (key & 7))], qf[s]);
        }
      }
      // scale, mask, running maximum (lane-local over 32 values, then with the partner lane)
      float tmax = -INFINITY;
#pragma unroll
      for (int hb = 0; hb < 2; ++hb)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int64_t key = c0 + hb * 32 + (r >> 2) * 8 + half * 4 + (r & 3);
          float x = st[hb][r] * scale;
          if (CAUSAL && key > qrow) x = -1.0e30f;
          if (key >= sk) x = -INFINITY;  // an invalid lane: no part in the max, the sum or the product
          st[hb][r] = x;
          tmax = fmaxf(tmax, x);
        }
      tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
      const float m_new = fmaxf(m, tmax);
      const float corr = exp2f(m - m_new);
      float psum = 0.0f;
      u32x4 pf[2][2];  // P^T as the B operand: [half block][k16 step], 8 keys per lane
#pragma unroll
      for (int hb = 0; hb < 2; ++hb)
#pragma unroll
        for (int step = 0; step < 2; ++step) {
          uint32_t w[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const float p0 = exp2f(st[hb][step * 8 + 2 * j] - m_new);
            const float p1 = exp2f(st[hb][step * 8 + 2 * j + 1] - m_new);
            psum += p0 + p1;
            w[j] = (uint32_t)Half<BF>::from(p0) | ((uint32_t)Half<BF>::from(p1) << 16);
          }
          pf[hb][step] = u32x4{w[0], w[1], w[2], w[3]};
        }
      psum += __shfl_xor(psum, 32);
      total = total * corr + psum;
      m = m_new;
#pragma unroll
      for (int i = 0; i < D / 32; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][r] *= corr;
      // O^T += V^T P^T: A operand lane = d row, the same 8 keys per lane as P (two 4-key units)
#pragma unroll
      for (int i = 0; i < D / 32; ++i) {
        const int d = i * 32 + r32;
#pragma unroll
        for (int hb = 0; hb < 2; ++hb)
#pragma unroll
          for (int step = 0; step < 2; ++step) {
            const int u0 = hb * 8 + step * 4 + half, u1 = u0 + 2;
            const uint2 lo = vl[d * (BKEY / 4) + vt_unit(d, u0)];
            const uint2 hi = vl[d * (BKEY / 4) + vt_unit(d, u1)];
            Half<BF>::mma(acc[i], u32x4{lo.x, lo.y, hi.x, hi.y}, pf[hb][step]);
          }
      }
    }
    if (tile + 1 < ntiles) KRN_FA_STORE(buf ^ 1);
    __syncthreads();
  }
#undef KRN_FA_LOAD
#undef KRN_FA_STORE

  if (qrow < sq) {
    const float inv_total = 1.0f;  // acc / total is a division per element, as the tile program writes it
    (void)inv_total;
#pragma unroll
    for (int i = 0; i < D / 32; ++i)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d = i * 32 + g * 8 + half * 4;
        uint32_t lo = (uint32_t)Half<BF>::from(acc[i][g * 4 + 0] / total) |
                      ((uint32_t)Half<BF>::from(acc[i][g * 4 + 1] / total) << 16);
        uint32_t hi = (uint32_t)Half<BF>::from(acc[i][g * 4 + 2] / total) |
                      ((uint32_t)Half<BF>::from(acc[i][g * 4 + 3] / total) << 16);
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
