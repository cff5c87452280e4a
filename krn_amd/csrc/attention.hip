// Flash attention forward for gfx950: O = softmax(scale * Q K^T masked) V, one pass over the keys per query tile.
//
// This is the lowering of krn's flash-attention tile program (reference examples/04_libraries/08_flash_attention.py
// :35-59): `s = (q @ k^T) * scale`, an optional causal `where(k_pos <= q_pos, s, -1e30)`, the running row maximum
// `m`, row sum `total` and output `acc` rescaled by `exp2(m - m_new)`, `acc += p.to(dtype) @ v`, and finally
// `o = (acc / total).to(dtype)`. Keys past the end of the sequence are invalid lanes: they take no part in the
// maximum, the sum or the product.
//
// Layout (MI355X-first). A workgroup owns 256 query rows of one (batch, head); each of its 8 waves owns 32 rows and
// computes the transposed products S^T = K Q^T and O^T += V^T P^T with v_mfma_f32_32x32x16_{bf16,f16}. In that form
// every lane holds one query row (lane & 31) and 16 of the keys of a 32-key block (its half-wave partner holds the
// other 16), so the row maximum and sum are lane-local plus one exchange with lane ^ 32, the rescale of O is
// lane-local, and P feeds the next MFMA straight from registers as its B operand. The row maximum is exchanged with
// v_permlane32_swap; each lane keeps its own part of the row sum, and the two parts are added once at the end (the
// lazy rescale multiplies both by the same factor). Q stays in registers for the whole pass. K and V tiles of 64
// keys stream through LDS (a ring of three K tiles and two V tiles) filled by direct-to-LDS loads
// (global_load_lds_dwordx4); both keep the row-major [key][d] layout of global memory. K is read
// as the A operand of S^T with 16-byte reads (chunk c of key row r at slot c ^ (r & 15)); V is read as the A
// operand of O^T with ds_read_b64_tr_b16, which hands each lane four keys of one d column, so V never needs a
// transposing copy (chunk c of key row r at slot c ^ 4 (r & 3)). The key loop is software-pipelined in 32-key
// halves: the score MFMAs of half h + 1 are issued before the exp2 / sum / pack of half h, so the matrix core and
// the vector ALU of one wave work at the same time. Each SIMD interleaves two waves of the workgroup, and every K
// and V tile loaded into LDS serves all 256 query rows (half the L2 traffic of 128-row workgroups). Large launches
// give each workgroup two query tiles of one head, a late (long) one and an early (short) one, so a causal launch
// has no tail of short workgroups.
//
// Shortcuts. Exact: the row maximum of an unmasked half is taken on the raw scores and scaled once (rounding is
// monotonic, scale > 0); halves wholly past a wave's last causal row are skipped (their p are exp2(-1e30 - m) = 0
// and their corr is 1). Equal up to rounding: the exponent argument s * scale - m is one fused multiply-add on
// unmasked halves, and the running maximum used as the exponent base is refreshed only when it is beaten by more
// than 8 (p <= 2^8), which scales p, acc and total by the same power of two and leaves acc / total unchanged; the
// output is acc times the correctly rounded reciprocal of the row sum (at most one float32 rounding more than
// acc / total, before the rounding to 16 bits).
#include "common.h"

#ifndef KRN_FA_WAVES_DEFAULT
#define KRN_FA_WAVES_DEFAULT 8
#endif

namespace krn {

typedef short v4s __attribute__((ext_vector_type(4)));

template <bool BF>
struct Half;
template <>
struct Half<true> {
  __device__ static uint32_t pack(float lo, float hi) {
    return f2bf2(lo, hi);  // v_cvt_pk_bf16_f32, nearest even
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

constexpr int FA_WAVES = KRN_FA_WAVES_DEFAULT;  // waves per workgroup, 32 query rows each
constexpr int BQ = 32 * FA_WAVES;               // query rows per workgroup
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

// max(x, x of lane ^ 32): the two lanes that hold one query row (v_permlane32_swap, no LDS round trip). One
// v_max_f32 (written as assembly: as fmaxf the compiler first quiets both operands, two more VALU instructions; the
// instruction quiets a signaling NaN itself, and these operands are arithmetic results or swaps of them).
__device__ __forceinline__ float pair_max(float x) {
  const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  float y;
  asm("v_max_f32 %0, %1, %2" : "=v"(y) : "v"(__uint_as_float(sw[0])), "v"(__uint_as_float(sw[1])));
  return y;
}

// One query tile `qt` (BQ rows) of head `head`: the whole key pass and the store of its rows. `lds` is the
// workgroup's ring of K and V tiles. `qf` holds this lane's Q fragments: loaded here unless `preloaded`, in which
// case the previous tile of the same head has already loaded them and issued this tile's first K and V loads.
// `next_qt` (or -1) is the query tile this workgroup takes next in the same head: once the key loop's last
// barrier has passed (every wave is done with the ring), its first K and V tiles and its Q fragments are loaded
// before this tile's epilogue, so their latency runs under the epilogue instead of at the next tile's start.
// `causal` is a run-time argument rather than a template parameter: both variants then get the same code and
// register allocation, and a non-causal launch only sees its limits at +infinity.
template <bool BF, int D>
__device__ __forceinline__ void attention_tile(const uint16_t* __restrict__ Q, const uint16_t* __restrict__ K,
                                               const uint16_t* __restrict__ V, uint16_t* __restrict__ O, int64_t sq,
                                               int64_t sk, float scale, int causal, int qt, int head, uint8_t* lds,
                                               u32x4 (&qf)[D / 16], bool preloaded, int next_qt) {
  static_assert(D == 64 || D == 128, "head dimension 64 or 128");
  constexpr int DCH = D / 8;                // 16-byte chunks per key row
  constexpr int TILE_BYTES = BKEY * D * 2;  // one K (or V) tile
  constexpr int ROWS_PER_LOAD = 1024 / (D * 2);
  constexpr int LOADS = BKEY / ROWS_PER_LOAD / FA_WAVES;  // wave load instructions per tile, per operand
  static_assert(LOADS * ROWS_PER_LOAD * FA_WAVES == BKEY, "whole wave loads");
  static_assert(DCH <= 16, "swizzle range");

  const int64_t q0 = (int64_t)qt * BQ;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6, half = lane >> 5, r32 = lane & 31;
  const uint16_t* q = Q + (int64_t)head * sq * D;
  const uint16_t* k = K + (int64_t)head * sk * D;
  const uint16_t* v = V + (int64_t)head * sk * D;
  uint16_t* o = O + (int64_t)head * sq * D;

  // this lane's query row and its Q fragments (B operand of S^T = K Q^T): 8 contiguous d per MFMA step
  const int64_t qrow = q0 + wave * 32 + r32;
  if (!preloaded) {
#pragma unroll
    for (int s = 0; s < D / 16; ++s)
      qf[s] = qrow < sq ? *reinterpret_cast<const u32x4*>(q + qrow * D + s * 16 + half * 8) : u32x4{};
  }
  // Q is complete here: the loop's MFMAs read registers that no load is still writing, so the compiler waits for
  // no load inside the loop (it would otherwise re-check the Q loads before the first score MFMA of every half)
#pragma unroll
  for (int s = 0; s < D / 16; ++s) asm volatile("" : "+v"(qf[s]));

  f32x16 acc[D / 32];
#pragma unroll
  for (int i = 0; i < D / 32; ++i) acc[i] = f32x16{};
  // m: the exponent base of this lane's row (shared with lane ^ 32); total: this lane's part of the row sum
  float m = -1.0e30f, total = 0.0f;

  const int64_t kend = causal ? min(sk, q0 + BQ) : sk;
  // the causal limits of this wave's rows (no limit without a causal mask)
  const int64_t NONE = (int64_t)1 << 62;
  const int64_t wave_first_q = causal ? q0 + wave * 32 : NONE, wave_last_q = causal ? q0 + wave * 32 + 31 : NONE;
  const int row_limit = causal ? (int)qrow : 0x7fffffff;  // keys beyond it are masked
  const int ntiles = (int)((kend + BKEY - 1) / BKEY);
  const int nhalves = (int)((kend + 31) / 32);

  // LDS: a ring of three K tiles, then two V tiles. The loop is software-pipelined in 32-key halves: while half h
  // turns its scores into P (VALU), the scores of half h + 1 multiply (MFMA); then O += V P for half h runs beside
  // the row maximum of half h + 1. So the K tile of the next half is read before this tile's V: tile iteration t
  // reads K(t) and K(t + 1), and V(t). It loads K(t + 2) into the slot K(t - 1) left and V(t + 1) into the slot
  // V(t - 1) left (both free once every wave has passed the barrier that ended tile t - 1); one barrier per tile
  // publishes both.
  // Direct-to-LDS loads through buffer resources over this head's K and V (base in SGPRs; the host keeps a head's
  // rows under 2^31 bytes): lane -> (row within its 1 KiB block, slot).
  // Each lane's element offsets inside a tile are fixed: computed once here; a load adds the tile's base (uniform)
  const int lrow = lane / DCH, lslot = lane % DCH;
  const int wave_s = __builtin_amdgcn_readfirstlane(wave);
  const __amdgpu_buffer_rsrc_t k_rsrc = panel_rsrc(k), v_rsrc = panel_rsrc(v);
  uint32_t koff[LOADS], voff[LOADS];  // byte offsets within a tile
#pragma unroll
  for (int j = 0; j < LOADS; ++j) {
    const int row = (wave * LOADS + j) * ROWS_PER_LOAD + lrow;
    koff[j] = (uint32_t)(row * D + k_slot<D>(row, lslot) * 8) * 2;
    voff[j] = (uint32_t)(row * D + v_slot<D>(row, lslot) * 8) * 2;
  }
#define KRN_FA_LOAD(rsrc, tile, base, OFF)                                                                    \
  do {                                                                                                        \
    const int64_t t0 = (int64_t)(tile) * BKEY;                                                                \
    if (t0 + BKEY <= sk) {                                                                                    \
      const int soff = (int)(t0 * D * 2);                                                                     \
      _Pragma("unroll") for (int j = 0; j < LOADS; ++j)                                                       \
          buffer_to_lds16(rsrc, lds + (base) + (wave_s * LOADS + j) * 1024, OFF[j], soff);                    \
    } else { /* the ragged last tile: rows past the sequence read the last row (masked, so their p is 0) */   \
      _Pragma("unroll") for (int j = 0; j < LOADS; ++j) {                                                     \
        const int row = (wave * LOADS + j) * ROWS_PER_LOAD + lrow;                                            \
        const int64_t key = min(t0 + row, sk - 1);                                                            \
        buffer_to_lds16(rsrc, lds + (base) + (wave_s * LOADS + j) * 1024,                                       \
                        (uint32_t)(key * D * 2) + (OFF[j] - (uint32_t)(row * D * 2)), 0);                     \
      }                                                                                                       \
    }                                                                                                         \
  } while (0)
#define KRN_FA_PUBLISH()                                                                                      \
  do {                                                                                                        \
    __builtin_amdgcn_s_waitcnt(0x0070 | 0x0f00);  /* vmcnt(0) */                                             \
    __builtin_amdgcn_s_waitcnt(0xc07f & ~0x0f00); /* lgkmcnt(0) */                                            \
    __builtin_amdgcn_s_barrier();                                                                             \
  } while (0)
  // S^T of the 32-key half `hb` of the K tile at LDS offset `kb`
#define KRN_FA_SCORES(S, kb, hb)                                                                              \
  do {                                                                                                        \
    const u32x4* kl = reinterpret_cast<const u32x4*>(lds + (kb));                                            \
    const int key = (hb) * 32 + r32;                                                                          \
    S = f32x16{};                                                                                             \
    _Pragma("unroll") for (int j = 0; j < D / 16; ++j) Half<BF>::mma(S, kl[key * DCH + k_slot<D>(key, j * 2 + half)], qf[j]); \
  } while (0)
  // the scaled row maximum of an unmasked half, from the raw scores (rounding is monotonic and scale > 0)
#define KRN_FA_RAWMAX(S, out)                                                                                 \
  do {                                                                                                        \
    float raw = S[0];                                                                                         \
    _Pragma("unroll") for (int r = 1; r < 16; ++r) raw = fmaxf(raw, S[r]);                                    \
    raw *= scale;                                                                                             \
    out = pair_max(raw);                                                                                      \
  } while (0)
  // p = exp2(s * sc - m) in f32 for the row sum, packed to 16 bits as P^T, the B operand of two k16 steps
#define KRN_FA_EXP(S, sc)                                                                                     \
  do {                                                                                                        \
    const float neg_m = -m;                                                                                   \
    _Pragma("unroll") for (int step = 0; step < 2; ++step) {                                                  \
      uint32_t w[4];                                                                                          \
      _Pragma("unroll") for (int j = 0; j < 4; ++j) {                                                         \
        const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(S[step * 8 + 2 * j], sc, neg_m));              \
        const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(S[step * 8 + 2 * j + 1], sc, neg_m));          \
        psum[step] = j == 0 ? p0 + p1 : psum[step] + (p0 + p1); /* no 0 + x: -0 keeps it from folding */     \
        w[j] = Half<BF>::pack(p0, p1);                                                                        \
      }                                                                                                       \
      pf[step] = u32x4{w[0], w[1], w[2], w[3]};                                                               \
    }                                                                                                         \
  } while (0)
  // O^T += V^T P^T for the keys of half `hb` of the V tile at `vb`: A operand lane = d row, the same 8 keys per
  // lane as P (two 4-key transposed reads); the D / 32 accumulators innermost, so consecutive MFMAs are independent
#define KRN_FA_PV(vb, hb)                                                                                     \
  do {                                                                                                        \
    _Pragma("unroll") for (int step = 0; step < 2; ++step) _Pragma("unroll") for (int i = 0; i < D / 32; ++i) { \
      u32x4 va;                                                                                               \
      _Pragma("unroll") for (int part = 0; part < 2; ++part) {                                                \
        const int key = (hb) * 32 + step * 16 + part * 8 + tr_key;                                            \
        const int col = i * 32 + tr_col;                                                                      \
        const int off = key * (D * 2) + v_slot<D>(key, col >> 3) * 16 + (col & 7) * 2;                       \
        const v4s x = __builtin_amdgcn_ds_read_tr16_b64_v4i16(                                                \
            (__attribute__((address_space(3))) v4s*)(lds + (vb) + off));                                      \
        const u32x2 w = __builtin_bit_cast(u32x2, x);                                                         \
        va[part * 2] = w[0];                                                                                  \
        va[part * 2 + 1] = w[1];                                                                              \
      }                                                                                                       \
      Half<BF>::mma(acc[i], va, pf[step]);                                                                    \
    }                                                                                                         \
  } while (0)

  // V^T fragment address pieces for ds_read_b64_tr_b16: lane group g = lane / 16 reads keys
  // K0 + (lane % 16) / 4 at d columns dblk * 32 + (g % 2) * 16 + 4 * (lane % 4)
  const int g = lane >> 4, a16 = lane & 15;
  const int tr_key = (g >> 1) * 4 + (a16 >> 2);
  const int tr_col = (g & 1) * 16 + 4 * (a16 & 3);
  const bool positive = scale > 0.0f;
  constexpr int V_BASE = 3 * TILE_BYTES;

  f32x16 sa, sb;
  float tmax_next = -INFINITY;  // the scaled row maximum of the next half's raw scores
  if (ntiles > 0) {
    if (!preloaded) {
      KRN_FA_LOAD(k_rsrc, 0, 0, koff);
      KRN_FA_LOAD(v_rsrc, 0, V_BASE, voff);
      if (ntiles > 1) KRN_FA_LOAD(k_rsrc, 1, TILE_BYTES, koff);
    }
    if (preloaded) {
      // the last vector memory operations issued are the previous tile's D / 16 output stores (every wave issues
      // all of them): everything before them, this tile's first K and V tiles included, has landed at vmcnt(D / 16)
      __builtin_amdgcn_s_waitcnt(0x0070 | 0x0f00 | (D / 16));
      __builtin_amdgcn_s_waitcnt(0xc07f & ~0x0f00); /* lgkmcnt(0) */
      __builtin_amdgcn_s_barrier();
    } else {
      KRN_FA_PUBLISH();
    }
    KRN_FA_SCORES(sa, 0, 0);  // the first half is active for every wave
    KRN_FA_RAWMAX(sa, tmax_next);
  }

  // One pipeline step over half `hb` of tile `t` (K slot `kcur`, the next tile's K slot `knext`): SC holds its
  // scores, SN receives those of the following half.
#define KRN_FA_HALF(t, hb, SC, SN, kcur, knext)                                                               \
  do {                                                                                                        \
    const int h = 2 * (t) + (hb);                                                                             \
    const int64_t c0 = (int64_t)h * 32;                                                                       \
    const bool active = h < nhalves && c0 <= wave_last_q;                                                                                             \
    const bool next = h + 1 < nhalves && c0 + 32 <= wave_last_q;                                                                               \
    if (active) {                                                                                             \
      const bool masked = c0 + 32 > sk || c0 + 31 > wave_first_q || !positive;                                                  \
      float tmax = tmax_next;                                                                                 \
      if (masked) {                                                                                           \
        float mx = -INFINITY;                                                                                 \
        const int key0 = (int)c0 + half * 4, valid = (int)(sk - c0);                                                                   \
        _Pragma("unroll") for (int r = 0; r < 16; ++r) {                                                      \
          const int key = key0 + (r >> 2) * 8 + (r & 3);                                                      \
          float x = SC[r] * scale;                                                                            \
          if (key > row_limit) x = -1.0e30f;                                                                  \
          if (key - (int)c0 >= valid) x = -INFINITY; /* an invalid lane: no part in max, sum or product */    \
          SC[r] = x;                                                                                          \
          mx = fmaxf(mx, x);                                                                                  \
        }                                                                                                     \
        tmax = pair_max(mx);                                                                                  \
      }                                                                                                       \
      /* Lazy rescale: the exponent base m only moves when some row maximum of the wave exceeds it by more    \
         than 8 (so every p <= 2^8); acc and total are then rescaled by exp2(m - m_new). A stale base scales  \
         p, acc and total alike, which leaves acc / total unchanged up to rounding. */                        \
      if (__builtin_amdgcn_ballot_w64(tmax > m + 8.0f) != 0) {                                                \
        const float m_new = fmaxf(m, tmax);                                                                   \
        const float corr = __builtin_amdgcn_exp2f(m - m_new);                                                 \
        total = total * corr;                                                                                 \
        _Pragma("unroll") for (int i = 0; i < D / 32; ++i) _Pragma("unroll") for (int r = 0; r < 16; ++r)     \
            acc[i][r] *= corr;                                                                                \
        m = m_new;                                                                                            \
      }                                                                                                       \
      /* masked halves already hold scaled scores: one fused multiply-add serves both (x * 1 - m is exact) */ \
      const float sc = masked ? 1.0f : scale;                                                                 \
      float psum[2];                                                                                          \
      u32x4 pf[2];                                                                                            \
      if (next) {                                                                                             \
        if ((hb) == 0) KRN_FA_SCORES(SN, kcur, 1);                                                            \
        else KRN_FA_SCORES(SN, knext, 0);                                                                     \
        KRN_FA_EXP(SC, sc);                                                                                   \
        KRN_FA_PV(V_BASE + ((t) & 1) * TILE_BYTES, hb);                                                       \
        KRN_FA_RAWMAX(SN, tmax_next);                                                                         \
      } else {                                                                                                \
        KRN_FA_EXP(SC, sc);                                                                                   \
        KRN_FA_PV(V_BASE + ((t) & 1) * TILE_BYTES, hb);                                                       \
      }                                                                                                       \
      total += psum[0] + psum[1];                                                                             \
    }                                                                                                         \
  } while (0)

  int kcur = 0;  // LDS offset of K(t); K(t + 1) and K(t + 2) follow around the ring
  for (int t = 0; t < ntiles; ++t) {
    const int knext = kcur == 2 * TILE_BYTES ? 0 : kcur + TILE_BYTES;
    const int kfree = knext == 2 * TILE_BYTES ? 0 : knext + TILE_BYTES;
    // the K loads of a tile go out before its first half and the V loads between the halves, so the workgroup's
    // loads reach the texture unit in two groups rather than one burst (causal B4 H32 S4096 D128 +3 %)
    if (t + 2 < ntiles) KRN_FA_LOAD(k_rsrc, t + 2, kfree, koff);
    KRN_FA_HALF(t, 0, sa, sb, kcur, knext);
    if (t + 1 < ntiles) KRN_FA_LOAD(v_rsrc, t + 1, V_BASE + ((t + 1) & 1) * TILE_BYTES, voff);
    KRN_FA_HALF(t, 1, sb, sa, kcur, knext);
    KRN_FA_PUBLISH();
    kcur = knext;
  }
  if (next_qt >= 0) {
    // the ring is free (every wave has passed the loop's last barrier): the next tile's first K and V tiles and
    // its Q fragments (this tile's are dead) go out now
    const int64_t next_q0 = (int64_t)next_qt * BQ;
    const int64_t next_kend = causal ? min(sk, next_q0 + BQ) : sk;
    KRN_FA_LOAD(k_rsrc, 0, 0, koff);
    KRN_FA_LOAD(v_rsrc, 0, V_BASE, voff);
    if (next_kend > BKEY) KRN_FA_LOAD(k_rsrc, 1, TILE_BYTES, koff);
    const int64_t next_row = next_q0 + wave * 32 + r32;
#pragma unroll
    for (int s = 0; s < D / 16; ++s)
      qf[s] = next_row < sq ? *reinterpret_cast<const u32x4*>(q + next_row * D + s * 16 + half * 8) : u32x4{};
  }
#undef KRN_FA_LOAD
#undef KRN_FA_PUBLISH
#undef KRN_FA_SCORES
#undef KRN_FA_RAWMAX
#undef KRN_FA_EXP
#undef KRN_FA_PV
#undef KRN_FA_HALF

  // the row sum: this lane's 16 keys of every half plus those of its partner lane ^ 32
  {
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(total), __float_as_uint(total), false, false);
    total = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
  }
  // the head's rows of O as a buffer resource: stores of rows past sq fall outside it and are dropped, so every
  // wave issues the same D / 16 stores whatever its rows (the next tile's first barrier counts on it)
  const __amdgpu_buffer_rsrc_t o_rsrc = panel_rsrc(o, sq * D * 2);
  const float inv = 1.0f / total;  // one division per row instead of 64 per lane (causal B4 H32 S4096 D128 +2 %)
  // Lane (r32, half) holds columns i * 32 + gq * 8 + half * 4 .. + 3 of its row; its partner lane ^ 32 the other
  // four of each group of eight. One v_permlane32_swap per word pairs them, so that the lower lane owns the eight
  // columns of the even groups and the upper lane those of the odd ones: every store is 16 bytes, and one store
  // instruction writes 32 contiguous bytes of each of 32 rows (8 stores per lane instead of 16 of 8 bytes).
#pragma unroll
  for (int i = 0; i < D / 32; ++i)
#pragma unroll
    for (int gp = 0; gp < 2; ++gp) {
      uint32_t w[2][2];  // [group gq = 2 gp + e][word]: this lane's four columns of each of the two groups
#pragma unroll
      for (int e2 = 0; e2 < 2; ++e2) {
        const int gq = 2 * gp + e2;
        w[e2][0] = Half<BF>::pack(acc[i][gq * 4 + 0] * inv, acc[i][gq * 4 + 1] * inv);
        w[e2][1] = Half<BF>::pack(acc[i][gq * 4 + 2] * inv, acc[i][gq * 4 + 3] * inv);
      }
      // the lower lane gives away its odd group, the upper lane its even group
      uint32_t got[2];
#pragma unroll
      for (int word = 0; word < 2; ++word) {
        const auto sw = __builtin_amdgcn_permlane32_swap(w[0][word], w[1][word], false, false);
        got[word] = half ? sw[0] : sw[1];
      }
      const int e2 = half;  // the group this lane stores
      const uint4 piece = half ? uint4{got[0], got[1], w[1][0], w[1][1]} : uint4{w[0][0], w[0][1], got[0], got[1]};
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, piece), o_rsrc,
                                             (int)((qrow * D + i * 32 + (2 * gp + e2) * 8) * 2), 0, 0);
    }
}

// The grid. Unpaired: one query tile per workgroup; causal launches run the late (long) tiles of every head first,
// so the short ones fill the tail. Paired (large launches): workgroup j of a head takes its query tiles
// q_tiles - 1 - j and then j, so under a causal mask every workgroup has the same number of keys to visit
// (q_tiles + 1 key tiles of BQ) and the launch has no tail of short workgroups; the middle tile of an odd count
// runs alone, after all the pairs.
template <bool BF, int D>
__global__ __launch_bounds__(64 * FA_WAVES, 512 / (64 * FA_WAVES)) void attention_fwd(
    const uint16_t* __restrict__ Q, const uint16_t* __restrict__ K, const uint16_t* __restrict__ V,
    uint16_t* __restrict__ O, int64_t sq, int64_t sk, float scale, int q_tiles, int causal, int paired) {
  __shared__ __attribute__((aligned(1024))) uint8_t lds[5 * BKEY * D * 2];  // three K and two V tiles
  if (paired) {
    const int per_head = (q_tiles + 1) / 2;
    const int heads = (int)(gridDim.x / per_head);
    const int j = (int)(blockIdx.x / heads), head = (int)(blockIdx.x % heads);
    const int first = q_tiles - 1 - j;
    u32x4 qf[D / 16];
    attention_tile<BF, D>(Q, K, V, O, sq, sk, scale, causal, first, head, lds, qf, false, j < first ? j : -1);
    if (j < first) attention_tile<BF, D>(Q, K, V, O, sq, sk, scale, causal, j, head, lds, qf, true, -1);
    return;
  }
  const int heads = (int)(gridDim.x / q_tiles);
  const int head = causal ? (int)(blockIdx.x % heads) : (int)(blockIdx.x / q_tiles);
  const int qt = causal ? (q_tiles - 1 - (int)(blockIdx.x / heads)) : (int)(blockIdx.x % q_tiles);
  u32x4 qf[D / 16];
  attention_tile<BF, D>(Q, K, V, O, sq, sk, scale, causal, qt, head, lds, qf, false, -1);
}

}  // namespace krn

using namespace krn;

template <bool BF, int D>
static void launch_attention(const void* q, const void* k, const void* v, void* o, int64_t bh, int64_t sq,
                             int64_t sk, float scale, int causal, hipStream_t stream) {
  const int q_tiles = (int)((sq + BQ - 1) / BQ);
  // pairs when the launch fills the chip twice over even with half the workgroups (256 CUs)
  const bool paired = q_tiles > 1 && bh * q_tiles >= 2 * 2 * 256;
  const int64_t blocks = paired ? bh * ((q_tiles + 1) / 2) : bh * q_tiles;
  dim3 grid((unsigned)blocks), block(64 * FA_WAVES);
  hipLaunchKernelGGL((attention_fwd<BF, D>), grid, block, 0, stream, (const uint16_t*)q, (const uint16_t*)k,
                     (const uint16_t*)v, (uint16_t*)o, sq, sk, scale, q_tiles, causal, (int)paired);
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
  if (sk * d * 2 > 0x7fffffff) {  // K and V tiles are addressed by 31-bit offsets within a head
    krn_set_error("attention: %lld keys of %lld elements exceed 2 GiB per head", (long long)sk, (long long)d);
    return -1;
  }
  if ((sq + BQ) * d * 2 > 0x7fffffff) {  // so are the output rows, those of a last partial query tile included
    krn_set_error("attention: %lld queries of %lld elements exceed 2 GiB per head", (long long)sq, (long long)d);
    return -1;
  }
  hipStream_t s = (hipStream_t)stream;
  const bool bf = kind == BF16;
#define KRN_FA(BFV, DV) \
  launch_attention<BFV, DV>(q, k, v, o, bh, sq, sk, scale, causal != 0, s)
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
