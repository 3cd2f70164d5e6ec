// Tile-level building blocks shared by the backward kernels (gfx950).
//
// A "tile" is ROWS x D elements in LDS, each row CPR = D*sizeof(T)/16 chunks
// of 16 bytes, logical chunk c of row r stored at position c ^ swz(r, CPR).
// Lanes are (g, p) = (lane / 16, lane % 16). Two products cover every
// contraction of the attention backward:
//
//   mm_rows_frag : acc[m][r]  = sum_d tile[16m + 4g + r][d] * frag_p[d]
//                  (tile rows as the MFMA A operand, one 16-row register
//                  fragment as B: S = Q K^T, dP = dO V^T and transposes)
//   mm_tr_acc    : acc[t][r] += sum_k tile[k][16t + 4g + r] * x_p[k]
//                  (tile^T as A through transposing LDS reads, x given as
//                  per-lane values x[m][r] at k = 16m + 4g + r: dQ = dS K,
//                  dK = dS^T Q, dV = P^T dO)
#pragma once
#include "fbsa_common.h"

namespace fbsa {

// Row fragment: lane (g, p) holds row p's elements k = 32ks + 8g + e (16-bit
// types) or k = 4ks + g (fp32).
template <typename T, int D> struct RowFrag {
  static constexpr bool F32 = sizeof(T) == 4;
  static constexpr int N = F32 ? D / 4 : D / 32;
  s16x8 h[F32 ? 1 : N];
  float f[F32 ? N : 1];
  __device__ __forceinline__ void load(const T *row, int g) {
    if constexpr (F32) {
#pragma unroll
      for (int ks = 0; ks < N; ++ks) f[ks] = ((const float *)row)[4 * ks + g];
    } else {
#pragma unroll
      for (int ks = 0; ks < N; ++ks) h[ks] = *(const s16x8 *)(row + 32 * ks + 8 * g);
    }
  }
};

// W > 0 (16-bit types): the tile reads are issued as asm in a sliding window of
// W outstanding reads, each MFMA waiting only for its own (LDS reads complete
// in order); W = 0 leaves the schedule to the compiler.
// TOFF (both products): a compile-time byte offset of the tile from `tile`,
// carried in the LDS instructions' offset fields (a loop over ring stages
// unrolled by the stage count passes the ring base, so the per-lane bases stay
// loop-invariant and no per-chunk address arithmetic remains).
// acc0 (optional): the accumulators' initial values instead of zeros (a
// rank-1 term such as -delta enters the product at no VALU cost).
template <typename T, int D, int NM, int W = 0, int TOFF = 0>
__device__ __forceinline__ void mm_rows_frag(const char *tile, const RowFrag<T, D> &fr, f32x4 *acc, int g, int p,
                                             const f32x4 *acc0 = nullptr) {
  constexpr int CPR = D * (int)sizeof(T) / 16;
  if constexpr (sizeof(T) == 2) {
    // read (m, ks) at lane base kb[ks % 4] + (ks / 4) * 256 + m * 256 * CPR
    constexpr int KS = D / 32, NK = NM * KS, KL = KS < 4 ? KS : 4;
    if constexpr (W > 0) {
      unsigned kb[KL];
#pragma unroll
      for (int l = 0; l < KL; ++l) kb[l] = (unsigned)(uintptr_t)tile + tile_kbase(l, g, p, CPR);
      s16x8 x[NK];
      auto rd = [&](auto K) {
        constexpr int k = decltype(K)::value, m = k / KS, ks = k % KS;
        x[k] = lds_read_b128_at<TOFF + (ks / 4) * 256 + m * 256 * CPR>(kb[ks % 4]);
      };
      static_for<(W < NK ? W : NK)>(rd);
      static_for<NK>([&](auto K) {
        constexpr int k = decltype(K)::value;
        constexpr int last = k + W - 1 < NK - 1 ? k + W - 1 : NK - 1;  // last read issued so far
        lds_wait_le<(last - k < 15 ? last - k : 15)>();
        lds_ready(x[k]);
        if constexpr (k % KS == 0) acc[k / KS] = acc0 ? acc0[k / KS] : f32x4{0.f, 0.f, 0.f, 0.f};
        acc[k / KS] = Mfma16<T>::run(x[k], fr.h[k % KS], acc[k / KS]);
        if constexpr (k + W < NK) rd(std::integral_constant<int, k + W>{});
      });
    } else {
      const char *kb[KL];
#pragma unroll
      for (int l = 0; l < KL; ++l) kb[l] = tile + tile_kbase(l, g, p, CPR);
#pragma unroll
      for (int m = 0; m < NM; ++m) {
        acc[m] = acc0 ? acc0[m] : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          const s16x8 x = *(const s16x8 *)(kb[ks % 4] + TOFF + (ks / 4) * 256 + m * 256 * CPR);
          acc[m] = Mfma16<T>::run(x, fr.h[ks], acc[m]);
        }
      }
    }
    return;
  }
#pragma unroll
  for (int m = 0; m < NM; ++m) {
    acc[m] = acc0 ? acc0[m] : f32x4{0.f, 0.f, 0.f, 0.f};
    const int row = 16 * m + p;
#pragma unroll
    for (int ks = 0; ks < D / 4; ++ks) {
      const float x = *(const float *)(tile + TOFF + (row * CPR + (ks ^ swz(row, CPR))) * 16 + g * 4);
      acc[m] = mfma_f32_16x16x4(x, fr.f[ks], acc[m]);
      if constexpr (D >= 256) if (ks % 16 == 15) asm volatile("" ::: "memory");  // at most 16 loads ahead
    }
    // keeps the next row tile's loads from being hoisted above these MFMAs
    // (at d >= 128 the hoisted loads of every tile exhaust the registers)
    if constexpr (D >= 128) asm volatile("" ::: "memory");
  }
}

// TW > 0 (16-bit types, KC >= 32): the transposed reads go out in a sliding
// window of TW output tiles, each tile's MFMAs waiting only for its own reads.
// SPLIT (16-bit types): x enters the product as a hi/lo operand pair
// (pack8_split), two MFMAs per read, so the product carries x to ~2^-17
// relative instead of one 16-bit rounding. NX = 2: a second operand x2
// (plain 16-bit rounding) is accumulated into acc2 from the same tile reads.
template <typename T, int D, int KC, int TW = 0, bool SPLIT = false, int NX = 1, int TOFF = 0>
__device__ __forceinline__ void mm_tr_acc(const char *tile, const float (&x)[KC / 16][4], f32x4 *acc, int g, int p,
                                          const float (*x2)[4] = nullptr, f32x4 *acc2 = nullptr) {
  constexpr int CPR = D * (int)sizeof(T) / 16;
  constexpr bool SP = SPLIT && sizeof(T) == 2;
  if constexpr (sizeof(T) == 2 && KC >= 32) {
    s16x8 pk[KC / 32], pkl[SP ? KC / 32 : 1], pk2[NX == 2 ? KC / 32 : 1];
#pragma unroll
    for (int k2 = 0; k2 < KC / 32; ++k2) {
      float y[8];
#pragma unroll
      for (int r = 0; r < 4; ++r) { y[r] = x[2 * k2][r]; y[4 + r] = x[2 * k2 + 1][r]; }
      if constexpr (SP) pack8_split<T>(y, pk[k2], pkl[k2]);
      else pk[k2] = pack8<T>(y);
      if constexpr (NX == 2) {
#pragma unroll
        for (int r = 0; r < 4; ++r) { y[r] = x2[2 * k2][r]; y[4 + r] = x2[2 * k2 + 1][r]; }
        pk2[k2] = pack8<T>(y);
      }
    }
    // an output tile's A operands from its transposed reads; its hi products
    // (and the second operand's); its lo products, issued one tile later so
    // that they do not wait on the hi products of the same accumulator
    auto tile_av = [&](s16x8 (&av)[KC / 32], s16x4 (&lo)[KC / 32], s16x4 (&hi)[KC / 32]) {
#pragma unroll
      for (int k2 = 0; k2 < KC / 32; ++k2) {
        lds_ready(lo[k2]);
        lds_ready(hi[k2]);
        const s16x4 a = lo[k2], b = hi[k2];
        av[k2] = s16x8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
      }
    };
    auto tile_hi = [&](const s16x8 (&av)[KC / 32], f32x4 &at, f32x4 &a2t) {
#pragma unroll
      for (int k2 = 0; k2 < KC / 32; ++k2) at = Mfma16<T>::run(av[k2], pk[k2], at);
      if constexpr (NX == 2) {
#pragma unroll
        for (int k2 = 0; k2 < KC / 32; ++k2) a2t = Mfma16<T>::run(av[k2], pk2[k2], a2t);
      }
    };
    auto tile_lo = [&](const s16x8 (&av)[KC / 32], f32x4 &at) {
      if constexpr (SP) {
#pragma unroll
        for (int k2 = 0; k2 < KC / 32; ++k2) at = Mfma16<T>::run(av[k2], pkl[k2], at);
      }
    };
    constexpr int NTL = D / 16;
    if constexpr (TW > 0) {
      constexpr int RPT = 2 * (KC / 32);  // reads per tile
      constexpr int W = TW < NTL ? TW : NTL, VL = NTL < 8 ? NTL : 8;
      s16x4 lo[NTL][KC / 32], hi[NTL][KC / 32];
      s16x8 avp[KC / 32];  // the previous tile's operands (its lo products are pending)
      // tile t, rows 32 k2 + 4g + p/4 (+16): lane base vb[t % 8] plus a constant
      unsigned vb[VL];
#pragma unroll
      for (int l = 0; l < VL; ++l) vb[l] = (unsigned)(uintptr_t)tile + tile_vbase(l, g, p, CPR);
      auto rd = [&](auto TT) {
        constexpr int t = decltype(TT)::value;
        static_for<KC / 32>([&](auto K2) {
          constexpr int k2 = decltype(K2)::value, off = (t / 8) * 256 + k2 * 512 * CPR;
          lo[t][k2] = lds_read_tr16_at<TOFF + off>(vb[t % 8]);
          hi[t][k2] = lds_read_tr16_at<TOFF + off + 256 * CPR>(vb[t % 8]);
        });
      };
      static_for<W>(rd);
      static_for<NTL>([&](auto TT) {
        constexpr int t = decltype(TT)::value;
        constexpr int last = t + W - 1 < NTL - 1 ? t + W - 1 : NTL - 1;  // last tile requested so far
        constexpr int n = (last - t) * RPT;
        lds_wait_le<(n < 15 ? n : 15)>();
        s16x8 av[KC / 32];
        tile_av(av, lo[t], hi[t]);
        tile_hi(av, acc[t], NX == 2 ? acc2[t] : acc[t]);
        if constexpr (t > 0) tile_lo(avp, acc[t - 1]);
        if constexpr (SP) {
#pragma unroll
          for (int k2 = 0; k2 < KC / 32; ++k2) avp[k2] = av[k2];
        }
        if constexpr (t + W < NTL) rd(std::integral_constant<int, t + W>{});
      });
      tile_lo(avp, acc[NTL - 1]);
    } else {
      // the transposed reads go out in batches of up to 8 output tiles (all of
      // them for d <= 128), each batch waited for once, so d = 256 does not hold
      // every tile's operands in registers at the same time
      constexpr int TB = NTL < 8 ? NTL : 8, VL = TB;
      unsigned vb[VL];
#pragma unroll
      for (int l = 0; l < VL; ++l) vb[l] = (unsigned)(uintptr_t)tile + tile_vbase(l, g, p, CPR);
#pragma unroll
      for (int t0 = 0; t0 < NTL; t0 += TB) {
        s16x4 lo[TB][KC / 32], hi[TB][KC / 32];
        static_for<TB>([&](auto TT) {
          constexpr int tt = decltype(TT)::value;
          static_for<KC / 32>([&](auto K2) {
            constexpr int k2 = decltype(K2)::value, off = k2 * 512 * CPR;
            // tile t0 + tt: lane base vb[tt] (t0 is a multiple of 8) plus (t0 / 8) * 256
            lo[tt][k2] = lds_read_tr16_at<TOFF + off>(vb[tt] + (t0 / 8) * 256);
            hi[tt][k2] = lds_read_tr16_at<TOFF + off + 256 * CPR>(vb[tt] + (t0 / 8) * 256);
          });
        });
        lds_wait_all();
        if constexpr (SP) {
          // every tile's hi products, then every tile's lo products
          s16x8 av[TB][KC / 32];
#pragma unroll
          for (int tt = 0; tt < TB; ++tt) {
            tile_av(av[tt], lo[tt], hi[tt]);
            tile_hi(av[tt], acc[t0 + tt], NX == 2 ? acc2[t0 + tt] : acc[t0 + tt]);
          }
#pragma unroll
          for (int tt = 0; tt < TB; ++tt) tile_lo(av[tt], acc[t0 + tt]);
        } else {
#pragma unroll
          for (int tt = 0; tt < TB; ++tt) {
            s16x8 av[KC / 32];
            tile_av(av, lo[tt], hi[tt]);
            tile_hi(av, acc[t0 + tt], NX == 2 ? acc2[t0 + tt] : acc[t0 + tt]);
          }
        }
      }
    }
    return;
  }
  if constexpr (sizeof(T) == 4) {
#pragma unroll
    for (int t = 0; t < D / 16; ++t) {
#pragma unroll
      for (int m = 0; m < KC / 16; ++m)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = 16 * m + 4 * g + r;
          const float a = *(const float *)(tile + TOFF + (row * CPR + ((4 * t + (p >> 2)) ^ swz(row, CPR))) * 16 + (p & 3) * 4);
          acc[t] = mfma_f32_16x16x4(a, x[m][r], acc[t]);
          if constexpr (NX == 2) acc2[t] = mfma_f32_16x16x4(a, x2[m][r], acc2[t]);
        }
      // keeps the next tile's loads from being hoisted above these MFMAs (at
      // d >= 128 the hoisted loads of every tile exhaust the registers)
      if constexpr (D >= 128) asm volatile("" ::: "memory");
    }
  } else {
    // KC == 16: one 16x16x16 MFMA per d tile (and per split part / operand)
    s16x4 pk, pkl, pk2;
    if constexpr (SP) pack4_split<T>(x[0], pk, pkl);
    else {
#pragma unroll
      for (int r = 0; r < 4; ++r) pk[r] = bits16<T>((T)x[0][r]);
    }
    if constexpr (NX == 2) {
#pragma unroll
      for (int r = 0; r < 4; ++r) pk2[r] = bits16<T>((T)x2[0][r]);
    }
    s16x4 a[D / 16];
#pragma unroll
    for (int t = 0; t < D / 16; ++t) {
      const int cb = 2 * t + ((p & 3) >> 1);
      const int ra = 4 * g + (p >> 2);
      a[t] = lds_read_tr16(tile + TOFF + (ra * CPR + (cb ^ swz(ra, CPR))) * 16 + (p & 1) * 8);
    }
    lds_wait_all();
#pragma unroll
    for (int t = 0; t < D / 16; ++t) {
      lds_ready(a[t]);
      acc[t] = Mfma16<T>::run16(a[t], pk, acc[t]);
      if constexpr (NX == 2) acc2[t] = Mfma16<T>::run16(a[t], pk2, acc2[t]);
    }
    if constexpr (SP) {
#pragma unroll
      for (int t = 0; t < D / 16; ++t) acc[t] = Mfma16<T>::run16(a[t], pkl, acc[t]);
    }
  }
}

// Per-thread plan of the direct-to-LDS copy of a KC-row tile pair (two
// swizzled tiles back to back in one LDS stage, 16-byte loads, LPT per
// thread): load n reads byte off[n] of source part[n]'s first row (part[n] is
// uniform across a wave). Computed once; each issue then needs only the two
// sources' row-0 addresses.
template <typename T, int KC, int D, int NW, int LPT> struct TilePairPlan {
  uint32_t off[LPT];
  bool part[LPT];
  __device__ __forceinline__ void init(int64_t stride0, int64_t stride1, int w, int lane) {
    constexpr int CPR = D * (int)sizeof(T) / 16;
#pragma unroll
    for (int n = 0; n < LPT; ++n) {
      const int u = (n * NW + w) * 64 + lane;
      const int pt = u / (KC * CPR);
      const int rem = u - pt * (KC * CPR);
      const int row = rem / CPR, pos = rem % CPR;
      part[n] = (n * NW + w) * 64 >= KC * CPR;  // == (pt != 0), uniform across the wave
      off[n] = (uint32_t)(((int64_t)row * (pt ? stride1 : stride0) + (pos ^ swz(row, CPR)) * (16 / (int)sizeof(T))) *
                          (int64_t)sizeof(T));
    }
  }
  // src0 / src1: the first rows of the chunk (wave-uniform)
  template <bool TRACKED>
  __device__ __forceinline__ void issue(char *st, const char *src0, const char *src1, int w) const {
#pragma unroll
    for (int n = 0; n < LPT; ++n) {
      const char *base = part[n] ? src1 : src0;
      if constexpr (TRACKED) g2lds16_tracked(base + off[n], st + (n * NW + w) * 1024);
      else g2lds16_s(base, off[n], st + (n * NW + w) * 1024);
    }
  }
};

}  // namespace fbsa
