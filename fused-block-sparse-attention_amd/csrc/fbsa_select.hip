// Block pooling and streaming block-pair selection for gfx950.
//
// Pooling (fbsa_pool): one workgroup per output block (b, output head, block
// i); threads own 16-byte d-chunks of a token row, sums are exact float64
// (bf16/fp16 sums of a block are exact in fp64; fp32 sums are exact for the
// magnitudes seen here), then divided and rounded to fp32 and the dtype at the
// same points as torch's mean (fp32 accumulate, round once).
//
// Selection (fbsa_select): one workgroup per (b, h, tile of R query rows).
// The 4 waves split the candidate key blocks (interleaved by 64) and compute
// the pooled scores with float64 FMA in the fixed order d = 0..D-1 (products
// of bf16/fp32 values are exact in fp64), round them like torch, and keep a
// per-row top-k list distributed over the 64 lanes (lane l holds the l-th
// best (score, index) as one orderable 64-bit key). Candidates below the
// current k-th key are rejected with one compare; survivors are inserted by
// ballot + shift. The four per-wave lists are merged in LDS at the end. The
// nblk x nblk score matrix never exists in memory.
#include <math.h>
#include <type_traits>

#include "fbsa_common.h"
#include "fbsa_internal.h"
#include "fbsa_round.h"

namespace fbsa {

// ---------------------------------------------------------------- pooling
// x / n for a mean: a multiplication when n is a power of two (the reciprocal
// is exact, so the quotient is identical), an IEEE division otherwise.
__device__ __forceinline__ double mean_div(double x, int64_t n) {
  if ((n & (n - 1)) == 0) return x * (1.0 / (double)n);
  return x / (double)n;
}

struct PoolArgs {
  const void *x;
  void *out, *out2;
  int64_t B, H, L, D, bs, nblk, grp, l_valid, Ho;
  int64_t sx[3];
  int op;
  // optional (mean ops of pool_wave_kernel): the selection's row norm of every
  // pooled row, at norm[(b * Ho + ho) * norm_pitch + block]; norm_key: rounded
  // up to bf16 (candidate side) instead of fp32 (query side)
  float *norm;
  int64_t norm_pitch;
  int norm_key;
};

// bf16 bit pattern of the smallest bf16 value >= x (x >= 0, +inf or NaN).
__device__ __forceinline__ uint32_t bf16_up_bits(float x) {
  uint32_t u = __float_as_uint(x);
  if (u & 0xFFFFu) u = (u + 0x10000u) & 0xFFFF0000u;
  return u >> 16;
}

// Row norm for the bracketed MFMA selection from an exact sum of squares:
// rounded up (a bound must not shrink); norms outside [2^-40, 1e18] become
// +inf, so every pair they touch has no usable bound (inf or NaN) and takes the
// exact path, which keeps the MFMA accumulation away from fp32 overflow and
// underflow. Candidate-side norms are rounded up to bf16, the precision of the
// rank-1 MFMA term.
__device__ __forceinline__ float sel_row_norm(double ss, bool key) {
  float n;
  if (ss == 0.0) {
    n = 0.f;
  } else {
    const double nrm = sqrt(ss) * (1.0 + 1e-6);
    n = nrm >= 0x1p-40 && nrm <= 1e18 ? (float)nrm : INFINITY;
  }
  return key ? __uint_as_float(bf16_up_bits(n) << 16) : n;
}

// Raw 8-element row chunk (kept undecoded until used, to keep registers low).
template <typename T> struct Raw8 {
  uint4 w[sizeof(T) == 4 ? 2 : 1];
};
template <typename T> __device__ __forceinline__ Raw8<T> load_raw8(const T *p) {
  Raw8<T> r;
  r.w[0] = *(const uint4 *)p;
  if constexpr (sizeof(T) == 4) r.w[1] = *(const uint4 *)(p + 4);
  return r;
}
template <typename T> __device__ __forceinline__ void decode8(const Raw8<T> &r, double *v) {
  const uint32_t w[4] = {r.w[0].x, r.w[0].y, r.w[0].z, r.w[0].w};
  if constexpr (sizeof(T) == 4) {
    const uint32_t w2[4] = {r.w[1].x, r.w[1].y, r.w[1].z, r.w[1].w};
#pragma unroll
    for (int e = 0; e < 4; ++e) { v[e] = (double)__uint_as_float(w[e]); v[4 + e] = (double)__uint_as_float(w2[e]); }
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[2 * e] = (double)half_bits_to_f32<T>(w[e] & 0xFFFFu);
      v[2 * e + 1] = (double)half_bits_to_f32<T>(w[e] >> 16);
    }
  }
}

template <typename T>
__global__ __launch_bounds__(256) void pool_kernel(PoolArgs a) {
  __shared__ double red[256 * 8];   // per-thread partial results (8 d values)
  const int tid = threadIdx.x;
  const int64_t blk = blockIdx.x;
  const int64_t i = blk % a.nblk;
  const int64_t ho = (blk / a.nblk) % a.Ho;
  const int64_t b = blk / (a.nblk * a.Ho);
  const int DC = (int)(a.D / 8);          // 16-byte chunks per row
  const int TL = 256 / DC;                // token lanes
  const int dc = tid % DC, tl = tid / DC;
  const bool active = tl < TL;
  const int op = a.op;
  const bool is_mean = op == FBSA_POOL_MEAN_TOK_THEN_GRP || op == FBSA_POOL_MEAN_GRP_THEN_TOK;

  double acc[8], acc2[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) { acc[e] = is_mean ? 0.0 : INFINITY; acc2[e] = -INFINITY; }

  auto rowptr = [&](int64_t h, int64_t t) {
    return (const T *)a.x + b * a.sx[0] + h * a.sx[1] + t * a.sx[2] + 8 * dc;
  };

  if (op == FBSA_POOL_MEAN_TOK_THEN_GRP) {
    // per head: exact token sum -> rnd(sum/bs); then rnd(sum over heads / grp)
    double hsum[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) hsum[e] = 0.0;
    for (int64_t hh = 0; hh < a.grp; ++hh) {
      const int64_t h = ho * a.grp + hh;
      double s[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) s[e] = 0.0;
      if (active)
        for (int64_t t = tl; t < a.bs; t += TL) {
          const int64_t pos = i * a.bs + t;
          if (pos >= a.l_valid) break;
          double v[8];
          load8<T>(rowptr(h, pos), v);
#pragma unroll
          for (int e = 0; e < 8; ++e) s[e] += v[e];
        }
#pragma unroll
      for (int e = 0; e < 8; ++e) red[tid * 8 + e] = s[e];
      __syncthreads();
      if (tid < DC) {
        for (int e = 0; e < 8; ++e) {
          double tot = 0.0;
          for (int l = 0; l < TL; ++l) tot += red[(l * DC + tid) * 8 + e];
          hsum[e] += (double)round_dt<T>(mean_div(tot, a.bs));
        }
      }
      __syncthreads();
    }
    if (tid < DC) {
      T *o = (T *)a.out + ((b * a.Ho + ho) * a.nblk + i) * a.D + 8 * tid;
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = (T)round_dt<T>(mean_div(hsum[e], a.grp));
    }
    return;
  }

  if (op == FBSA_POOL_MEAN_GRP_THEN_TOK) {
    // per token: rnd(sum over group / grp); then rnd(sum over tokens / bs)
    if (active)
      for (int64_t t = tl; t < a.bs; t += TL) {
        const int64_t pos = i * a.bs + t;
        double g[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) g[e] = 0.0;
        if (pos < a.l_valid)
          for (int64_t hh = 0; hh < a.grp; ++hh) {
            double v[8];
            load8<T>(rowptr(ho * a.grp + hh, pos), v);
#pragma unroll
            for (int e = 0; e < 8; ++e) g[e] += v[e];
          }
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] += (double)round_dt<T>(mean_div(g[e], a.grp));
      }
  } else {
    // MAX / MIN / MINMAX over tokens (padding tokens count as 0)
    if (active)
      for (int64_t t = tl; t < a.bs; t += TL) {
        const int64_t pos = i * a.bs + t;
        double v[8];
        if (pos < a.l_valid) load8<T>(rowptr(ho, pos), v);
        else {
#pragma unroll
          for (int e = 0; e < 8; ++e) v[e] = 0.0;
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          acc[e] = fmin(acc[e], v[e]);
          acc2[e] = fmax(acc2[e], v[e]);
        }
      }
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) red[tid * 8 + e] = acc[e];
  __syncthreads();
  double res[8], res2[8];
  if (tid < DC) {
    for (int e = 0; e < 8; ++e) {
      double tot = is_mean ? 0.0 : INFINITY;
      for (int l = 0; l < TL; ++l) {
        const double x = red[(l * DC + tid) * 8 + e];
        tot = is_mean ? tot + x : fmin(tot, x);
      }
      res[e] = tot;
    }
  }
  __syncthreads();
  if (!is_mean) {
#pragma unroll
    for (int e = 0; e < 8; ++e) red[tid * 8 + e] = acc2[e];
    __syncthreads();
    if (tid < DC)
      for (int e = 0; e < 8; ++e) {
        double tot = -INFINITY;
        for (int l = 0; l < TL; ++l) tot = fmax(tot, red[(l * DC + tid) * 8 + e]);
        res2[e] = tot;
      }
  }
  if (tid < DC) {
    const int64_t off = ((b * a.Ho + ho) * a.nblk + i) * a.D + 8 * tid;
    T *o = (T *)a.out + off;
    if (op == FBSA_POOL_MEAN_GRP_THEN_TOK) {
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = (T)round_dt<T>(mean_div(res[e], a.bs));
    } else if (op == FBSA_POOL_MAX) {
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = (T)(float)res2[e];
    } else if (op == FBSA_POOL_MIN) {
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = (T)(float)res[e];
    } else {
      T *o2 = (T *)a.out2 + off;
#pragma unroll
      for (int e = 0; e < 8; ++e) { o[e] = (T)(float)res[e]; o2[e] = (T)(float)res2[e]; }
    }
  }
}

// Wave-organised pooling for a block of BS tokens and D/8 = DC a power of two
// <= 64: a wave covers whole rows (DC lanes per row, 64/DC rows at a time),
// every lane keeps eight exact fp64 sums, and row partials meet by in-wave
// xor-shuffles; only the four wave partials go through LDS. Each lane's loads
// are issued back to back (fixed trip count; rows past l_valid are read at a
// clamped address and contribute 0). MEAN_TOK_THEN_GRP gives each wave whole
// heads; the other ops split the block's tokens over the waves.
// Workgroups [0, nwg0) pool a0, the rest pool a1 (two tensors in one launch).
template <typename T, int DC, int BS, int OP>
__global__ __launch_bounds__(256) void pool_wave_kernel(PoolArgs a0, PoolArgs a1, int64_t nwg0) {
  constexpr int NW = 4, TLW = 64 / DC;
  constexpr int RPH = BS >= TLW ? BS / TLW : 1;            // rows per lane per head (whole block in one wave)
  constexpr int RPW = BS >= NW * TLW ? BS / (NW * TLW) : 1;  // rows per lane when the waves split the block
  __shared__ double red[2][NW][DC][8];
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, c = lane % DC, tl = lane / DC;
  const bool second = (int64_t)blockIdx.x >= nwg0;
  const PoolArgs a = second ? a1 : a0;
  const int64_t blk = second ? (int64_t)blockIdx.x - nwg0 : (int64_t)blockIdx.x;
  const int64_t i = blk % a.nblk;
  const int64_t ho = (blk / a.nblk) % a.Ho;
  const int64_t b = blk / (a.nblk * a.Ho);
  constexpr int op = OP;
  // valid tokens in the block; 0 for a block wholly past l_valid (never block
  // 0, as l_valid >= 1), whose rows then all read row i * BS - 1 and count as 0
  const int64_t rem = a.l_valid - i * BS;
  const int nval = rem < BS ? (rem > 0 ? (int)rem : 0) : BS;
  auto rowptr = [&](int64_t h, int t) {
    const int tc = t < nval ? t : nval - 1;
    return (const T *)a.x + b * a.sx[0] + h * a.sx[1] + (i * BS + tc) * a.sx[2] + 8 * c;
  };
  auto xor_sum = [&](double *v) {
#pragma unroll
    for (int off = DC; off < 64; off <<= 1)
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] += __shfl_xor(v[e], off, 64);
  };

  double r0[8], r1[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) { r0[e] = 0.0; r1[e] = 0.0; }
  if constexpr (op == FBSA_POOL_MEAN_TOK_THEN_GRP) {
    // wave w: heads w, w + 4, ...; per head an exact token sum and its rounded mean
    for (int64_t hh = w; hh < a.grp; hh += NW) {
      double acc[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] = 0.0;
      constexpr int NB = RPH < 8 ? RPH : 8;  // rows loaded back to back per batch
      for (int n0 = 0; n0 < RPH; n0 += NB) {
        Raw8<T> raw[NB];
#pragma unroll
        for (int n = 0; n < NB; ++n) raw[n] = load_raw8<T>(rowptr(ho * a.grp + hh, tl + (n0 + n) * TLW));
#pragma unroll
        for (int n = 0; n < NB; ++n) {
          const int t = tl + (n0 + n) * TLW;
          const bool ok = t < nval && t < BS;
          double v[8];
          decode8<T>(raw[n], v);
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[e] += ok ? v[e] : 0.0;
        }
      }
      xor_sum(acc);
#pragma unroll
      for (int e = 0; e < 8; ++e) r0[e] += (double)round_dt<T>(acc[e] / (double)BS);
    }
  } else if constexpr (op == FBSA_POOL_MEAN_GRP_THEN_TOK) {
    // tokens split over waves and lanes; per token an exact group sum, rounded mean
    for (int n = 0; n < RPW; ++n) {
      const int t = (w + n * NW) * TLW + tl;
      double g[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) g[e] = 0.0;
#pragma unroll 8
      for (int64_t hh = 0; hh < a.grp; ++hh) {
        double v[8];
        load8<T>(rowptr(ho * a.grp + hh, t), v);
#pragma unroll
        for (int e = 0; e < 8; ++e) g[e] += v[e];
      }
      const bool ok = t < nval && t < BS;
#pragma unroll
      for (int e = 0; e < 8; ++e) r0[e] += ok ? (double)round_dt<T>(mean_div(g[e], a.grp)) : 0.0;
    }
    xor_sum(r0);
  } else {
    // per-block min / max over tokens; padding tokens count as 0
#pragma unroll
    for (int e = 0; e < 8; ++e) { r0[e] = INFINITY; r1[e] = -INFINITY; }
    constexpr int NB = RPW < 8 ? RPW : 8;
    for (int n0 = 0; n0 < RPW; n0 += NB) {
      Raw8<T> raw[NB];
#pragma unroll
      for (int n = 0; n < NB; ++n) raw[n] = load_raw8<T>(rowptr(ho, (w + (n0 + n) * NW) * TLW + tl));
#pragma unroll
      for (int n = 0; n < NB; ++n) {
        const int t = (w + (n0 + n) * NW) * TLW + tl;
        if (t >= BS) continue;
        const bool ok = t < nval;
        double v[8];
        decode8<T>(raw[n], v);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const double x = ok ? v[e] : 0.0;
          r0[e] = fmin(r0[e], x);
          r1[e] = fmax(r1[e], x);
        }
      }
    }
#pragma unroll
    for (int off = DC; off < 64; off <<= 1)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        r0[e] = fmin(r0[e], __shfl_xor(r0[e], off, 64));
        r1[e] = fmax(r1[e], __shfl_xor(r1[e], off, 64));
      }
  }
  if (tl == 0) {
#pragma unroll
    for (int e = 0; e < 8; ++e) { red[0][w][c][e] = r0[e]; red[1][w][c][e] = r1[e]; }
  }
  __syncthreads();
  if (tid < DC * 8) {
    const int cc = tid >> 3, e = tid & 7;
    const int64_t off = ((b * a.Ho + ho) * a.nblk + i) * a.D + 8 * cc + e;
    if (op == FBSA_POOL_MEAN_TOK_THEN_GRP || op == FBSA_POOL_MEAN_GRP_THEN_TOK) {
      double tot = 0.0;
#pragma unroll
      for (int ww = 0; ww < NW; ++ww) tot += red[0][ww][cc][e];
      const T y = (T)round_dt<T>(mean_div(tot, op == FBSA_POOL_MEAN_TOK_THEN_GRP ? a.grp : (int64_t)BS));
      ((T *)a.out)[off] = y;
      red[1][0][cc][e] = (double)(float)y;  // element 8 cc + e of the pooled row (red[1] is free here)
    } else {
      double mn = red[0][0][cc][e], mx = red[1][0][cc][e];
#pragma unroll
      for (int ww = 1; ww < NW; ++ww) { mn = fmin(mn, red[0][ww][cc][e]); mx = fmax(mx, red[1][ww][cc][e]); }
      if (a.op == FBSA_POOL_MAX) ((T *)a.out)[off] = (T)(float)mx;
      else if (a.op == FBSA_POOL_MIN) ((T *)a.out)[off] = (T)(float)mn;
      else { ((T *)a.out)[off] = (T)(float)mn; ((T *)a.out2)[off] = (T)(float)mx; }
    }
  }
  if constexpr (op == FBSA_POOL_MEAN_TOK_THEN_GRP || op == FBSA_POOL_MEAN_GRP_THEN_TOK) {
    if (a.norm) {
      // the pooled row's sum of squares over d = 0, 1, ... in order (the sum
      // sel_norms_kernel forms from the stored row)
      __syncthreads();
      if (tid == 0) {
        const double *row = &red[1][0][0][0];
        double ss = 0.0;
        for (int d = 0; d < DC * 8; ++d) ss += row[d] * row[d];
        a.norm[(b * a.Ho + ho) * a.norm_pitch + i] = sel_row_norm(ss, a.norm_key != 0);
      }
    }
  }
}

// Token mean of a block with one input head per output head (mean pooling
// with grp == 1): one block per wave, four per workgroup. DC lanes cover a row
// (8 elements each), 64 / DC rows at a time; a lane's BS / (64 / DC) row loads
// are issued back to back, its exact fp64 sums meet by in-wave xor-shuffles,
// and no LDS or workgroup barrier is involved (the workgroup-per-block kernel
// leaves three of its four waves idle in this case). The result is the one
// pool_wave_kernel writes: the block sum rounded once after the exact division
// by BS, and, when norm is set, the pooled row's sum of squares over
// d = 0, 1, ... in order. Waves [0, nb0) pool a0, waves [nb0, nbt) pool a1.
template <typename T, int DC, int BS>
__global__ __launch_bounds__(256) void pool_mean1_kernel(PoolArgs a0, PoolArgs a1, int64_t nb0, int64_t nbt) {
  constexpr int TLW = 64 / DC;
  constexpr int RPL = BS >= TLW ? BS / TLW : 1;  // rows per lane
  const int lane = threadIdx.x & 63, c = lane % DC, tl = lane / DC;
  const int64_t wv = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (wv >= nbt) return;  // wave-uniform
  const bool second = wv >= nb0;
  const PoolArgs a = second ? a1 : a0;
  const int64_t blk = second ? wv - nb0 : wv;
  const int64_t i = blk % a.nblk;
  const int64_t ho = (blk / a.nblk) % a.Ho;
  const int64_t b = blk / (a.nblk * a.Ho);
  // valid tokens in the block; 0 for a block wholly past l_valid (never block
  // 0, as l_valid >= 1), whose rows then all read row i * BS - 1 and count as 0
  const int64_t rem = a.l_valid - i * BS;
  const int nval = rem < BS ? (rem > 0 ? (int)rem : 0) : BS;
  const T *base = (const T *)a.x + b * a.sx[0] + ho * a.sx[1] + i * BS * a.sx[2] + 8 * c;
  Raw8<T> raw[RPL];
#pragma unroll
  for (int n = 0; n < RPL; ++n) {
    const int t = tl + n * TLW;
    const int tc = t < nval ? t : nval - 1;  // rows past l_valid: a clamped address, counted as 0
    raw[n] = load_raw8<T>(base + tc * a.sx[2]);
  }
  double acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = 0.0;
#pragma unroll
  for (int n = 0; n < RPL; ++n) {
    const int t = tl + n * TLW;
    const bool ok = t < nval && t < BS;
    double v[8];
    decode8<T>(raw[n], v);
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] += ok ? v[e] : 0.0;
  }
#pragma unroll
  for (int off = DC; off < 64; off <<= 1)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] += __shfl_xor(acc[e], off, 64);
  float yf[8];
  T y[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    yf[e] = round_dt<T>(acc[e] * (1.0 / (double)BS));  // BS is a power of two: the product is the quotient
    y[e] = (T)yf[e];
  }
  if (tl == 0) {
    T *o = (T *)a.out + ((b * a.Ho + ho) * a.nblk + i) * a.D + 8 * c;
    if (((uintptr_t)o & 15) == 0) {
      uint4 u[sizeof(T) / 2];
      __builtin_memcpy(u, y, sizeof(y));
#pragma unroll
      for (int q = 0; q < (int)(sizeof(T) / 2); ++q) ((uint4 *)o)[q] = u[q];
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = y[e];
    }
  }
  if (a.norm) {
    // element 8 cc + e of the pooled row is yf[e] of lane cc; every lane forms
    // the same ordered sum and lane 0 writes it
    double ss = 0.0;
#pragma unroll
    for (int cc = 0; cc < DC; ++cc)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const double v = (double)__int_as_float(__builtin_amdgcn_readlane(__float_as_int(yf[e]), cc));
        ss += v * v;
      }
    if (lane == 0) a.norm[(b * a.Ho + ho) * a.norm_pitch + i] = sel_row_norm(ss, a.norm_key != 0);
  }
}

// Per-token group mean (bs = 1, MEAN_GRP_THEN_TOK): one thread per 8-element
// chunk of an output row, the exact fp64 group sum rounded once as in the
// block kernels (the mean over one token is the identity), coalesced 16-byte
// loads and stores.
template <typename T>
__global__ __launch_bounds__(256) void pool_grp_kernel(PoolArgs a, int64_t n) {
  const int64_t g = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (g >= n) return;
  const int64_t DC = a.D / 8;
  const int64_t c = g % DC;
  const int64_t t = (g / DC) % a.nblk;
  const int64_t ho = (g / (DC * a.nblk)) % a.Ho;
  const int64_t b = g / (DC * a.nblk * a.Ho);
  double s[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) s[e] = 0.0;
  const T *base = (const T *)a.x + b * a.sx[0] + ho * a.grp * a.sx[1] + t * a.sx[2] + 8 * c;
  if (t < a.l_valid)
    for (int64_t h0 = 0; h0 < a.grp; h0 += 8) {
      // up to eight heads' loads in flight before any is summed
      Raw8<T> raw[8];
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if (h0 + u < a.grp) raw[u] = load_raw8<T>(base + (h0 + u) * a.sx[1]);
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if (h0 + u < a.grp) {
          double v[8];
          decode8<T>(raw[u], v);
#pragma unroll
          for (int e = 0; e < 8; ++e) s[e] += v[e];
        }
    }
  T r[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) r[e] = (T)round_dt<T>(mean_div(s[e], a.grp));
  T *o = (T *)a.out + ((b * a.Ho + ho) * a.nblk + t) * a.D + 8 * c;
  if (((uintptr_t)o & 15) == 0) {
    uint4 u[sizeof(T) / 2];
    __builtin_memcpy(u, r, sizeof(r));
#pragma unroll
    for (int q = 0; q < (int)(sizeof(T) / 2); ++q) ((uint4 *)o)[q] = u[q];
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = r[e];
  }
}

template <typename T, int DC, int BS> static void launch_pool_op(const PoolArgs &a, int64_t nwg, hipStream_t s) {
  switch (a.op) {
    case FBSA_POOL_MEAN_TOK_THEN_GRP:
      if (a.grp == 1) {
        hipLaunchKernelGGL((pool_mean1_kernel<T, DC, BS>), dim3((unsigned)((nwg + 3) / 4)), dim3(256), 0, s, a, a, nwg, nwg);
        return;
      }
      hipLaunchKernelGGL((pool_wave_kernel<T, DC, BS, FBSA_POOL_MEAN_TOK_THEN_GRP>), dim3((unsigned)nwg), dim3(256), 0, s, a,
                         a, nwg);
      return;
    case FBSA_POOL_MEAN_GRP_THEN_TOK:
      hipLaunchKernelGGL((pool_wave_kernel<T, DC, BS, FBSA_POOL_MEAN_GRP_THEN_TOK>), dim3((unsigned)nwg), dim3(256), 0, s, a,
                         a, nwg);
      return;
    default:  // MAX / MIN / MINMAX share one instantiation (the op picks the outputs)
      hipLaunchKernelGGL((pool_wave_kernel<T, DC, BS, FBSA_POOL_MINMAX>), dim3((unsigned)nwg), dim3(256), 0, s, a, a, nwg);
      return;
  }
}

template <typename T, int DC> static bool launch_pool_bs(const PoolArgs &a, int64_t nwg, hipStream_t s) {
  switch (a.bs) {
    case 16: launch_pool_op<T, DC, 16>(a, nwg, s); return true;
    case 32: launch_pool_op<T, DC, 32>(a, nwg, s); return true;
    case 64: launch_pool_op<T, DC, 64>(a, nwg, s); return true;
    case 128: launch_pool_op<T, DC, 128>(a, nwg, s); return true;
  }
  return false;
}

template <typename T> static void launch_pool(const PoolArgs &a, int64_t nwg, hipStream_t s) {
  bool done = false;
  switch (a.D / 8) {
    case 2: done = a.D == 16 && launch_pool_bs<T, 2>(a, nwg, s); break;
    case 4: done = a.D == 32 && launch_pool_bs<T, 4>(a, nwg, s); break;
    case 8: done = a.D == 64 && launch_pool_bs<T, 8>(a, nwg, s); break;
    case 16: done = a.D == 128 && launch_pool_bs<T, 16>(a, nwg, s); break;
    case 32: done = a.D == 256 && launch_pool_bs<T, 32>(a, nwg, s); break;
  }
  if (!done) hipLaunchKernelGGL(pool_kernel<T>, dim3((unsigned)nwg), dim3(256), 0, s, a);
}

static PoolArgs pool_args(const fbsa_pool_desc *d, const void *x, void *out, void *out2) {
  PoolArgs a;
  a.x = x; a.out = out; a.out2 = out2;
  a.B = d->B; a.H = d->H; a.L = d->L; a.D = d->D; a.bs = d->bs; a.nblk = d->nblk; a.grp = d->grp;
  a.l_valid = d->l_valid; a.Ho = d->H / d->grp; a.op = d->op;
  for (int k = 0; k < 3; ++k) a.sx[k] = d->sx[k];
  a.norm = nullptr; a.norm_pitch = 0; a.norm_key = 0;
  return a;
}

int run_pool(const fbsa_pool_desc *d, const void *x, void *out, void *out2, hipStream_t s) {
  const PoolArgs a = pool_args(d, x, out, out2);
  const int64_t nwg = a.B * a.Ho * a.nblk;
  if (a.bs == 1 && a.op == FBSA_POOL_MEAN_GRP_THEN_TOK) {
    const int64_t n = nwg * (a.D / 8);
    const dim3 grid((unsigned)((n + 255) / 256));
    switch (d->dtype) {
      case FBSA_BF16: hipLaunchKernelGGL(pool_grp_kernel<bf16>, grid, dim3(256), 0, s, a, n); break;
      case FBSA_F16: hipLaunchKernelGGL(pool_grp_kernel<f16>, grid, dim3(256), 0, s, a, n); break;
      default: hipLaunchKernelGGL(pool_grp_kernel<float>, grid, dim3(256), 0, s, a, n); break;
    }
    return hip_check(hipGetLastError(), "pool_grp_kernel launch");
  }
  switch (d->dtype) {
    case FBSA_BF16: launch_pool<bf16>(a, nwg, s); break;
    case FBSA_F16: launch_pool<f16>(a, nwg, s); break;
    default: launch_pool<float>(a, nwg, s); break;
  }
  return hip_check(hipGetLastError(), "pool_kernel launch");
}

// ---------------------------------------------------------------- selection
struct SelArgs {
  const void *a, *b1, *b2;
  int32_t *sel;
  float *sel_score;
  const float *an1, *an2, *bn1, *bn2;  // row norms (MFMA path): query-side parts and key-side operands
  int norms_ready;                      // the workspace's norm arrays are already filled (by the pooling)
  uint64_t *part;                      // MFMA path: per-(row, candidate chunk) top-k keys
  int64_t B, H, nblk, D, topk, kk;
  int64_t ct, nch;                     // MFMA path: candidate tiles per chunk, chunks per row block
  int64_t row0, row1;                  // query blocks (rows) selected by this launch
  int conv, causal, sink, score;
};

// Orderable key: larger = better. Score bits mapped monotonically (NaN above
// +inf, -0 == +0), then the complemented index so ties favour the lower index.
__device__ __forceinline__ uint64_t make_key(float s, int j) {
  if (s == 0.f) s = 0.f;
  uint32_t u = __float_as_uint(s);
  if (s != s) u = 0xFFFFFFFFu;
  else u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((uint64_t)u << 32) | (uint32_t)(~(uint32_t)j);
}
__device__ __forceinline__ float key_score(uint64_t k) {
  const uint32_t u = (uint32_t)(k >> 32);
  if (u == 0xFFFFFFFFu) return __uint_as_float(0x7FC00000u);
  return __uint_as_float((u & 0x80000000u) ? (u & 0x7FFFFFFFu) : ~u);
}
__device__ __forceinline__ int key_index(uint64_t k) { return (int)(~(uint32_t)k); }

// Wave-uniform lane read (src is the same for every lane): v_readlane, no LDS.
__device__ __forceinline__ uint64_t readlane_u64(uint64_t v, int src) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, src);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), src);
  return ((uint64_t)hi << 32) | lo;
}
// Lane l receives lane l-1's value (lane 0 keeps its own): DPP wave_shr:1.
__device__ __forceinline__ uint64_t wave_shr1_u64(uint64_t v) {
  const int lo = (int)(uint32_t)v, hi = (int)(uint32_t)(v >> 32);
  const uint32_t slo = (uint32_t)__builtin_amdgcn_update_dpp(lo, lo, 0x138, 0xF, 0xF, false);
  const uint32_t shi = (uint32_t)__builtin_amdgcn_update_dpp(hi, hi, 0x138, 0xF, 0xF, false);
  return ((uint64_t)shi << 32) | slo;
}

// Insert key c (wave-uniform) into the distributed descending list (lane l
// holds entry l; 0 = empty). K = capacity (<= 64). Keys are unique (the index
// is part of them).
__device__ __forceinline__ void list_insert(uint64_t &mine, uint64_t c, int lane, int K) {
  const uint64_t better = __ballot(mine > c);  // empties (0) are never better
  const int pos = __popcll(better);
  if (pos >= K) return;
  const uint64_t prev = wave_shr1_u64(mine);
  if (lane > pos && lane < K) mine = prev;
  if (lane == pos) mine = c;
}

template <typename T, int D, int R, int MODE>
__global__ __launch_bounds__(256) void select_kernel(SelArgs a) {
  __shared__ double sa[2][R][D];       // query-side operands (fp64; QUEST: relu and neg parts)
  __shared__ uint64_t lists[4][R][64];  // per-wave lists for the final merge
  __shared__ float diag[R], sinks[R];
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int64_t ntile = (a.row1 - a.row0 + R - 1) / R;
  // heavy (late) row tiles first: blockIdx 0 gets the last tile
  const int64_t t = ntile - 1 - (int64_t)blockIdx.x % ntile;
  const int64_t bh = blockIdx.x / ntile;  // b * H + h
  const int64_t i0 = a.row0 + t * R;
  const T *A = (const T *)a.a + bh * a.nblk * D;
  const T *B1 = (const T *)a.b1 + bh * a.nblk * D;
  const T *B2 = MODE != FBSA_SCORE_DOT ? (const T *)a.b2 + bh * a.nblk * D : nullptr;

  for (int x = tid; x < R * D; x += 256) {
    const int r = x / D, dd = x % D;
    const int64_t i = i0 + r;
    const double v = i < a.nblk ? (double)(float)A[i * D + dd] : 0.0;
    if (MODE == FBSA_SCORE_QUEST) { sa[0][r][dd] = v > 0.0 ? v : 0.0; sa[1][r][dd] = v < 0.0 ? v : 0.0; }
    else sa[0][r][dd] = v;
  }
  __syncthreads();

  const bool convA = a.conv == FBSA_SEL_OWN_FIRST;
  const int K = (int)(convA ? (a.topk < a.nblk - 1 ? a.topk : a.nblk - 1) : (a.topk < a.nblk ? a.topk : a.nblk));
  const int64_t last_row = (i0 + R - 1 < a.nblk - 1) ? i0 + R - 1 : a.nblk - 1;
  const int64_t jmax = (a.causal || !convA) ? last_row : a.nblk - 1;

  uint64_t lst[R];
#pragma unroll
  for (int r = 0; r < R; ++r) lst[r] = 0;

  for (int64_t jb = (int64_t)w * 64; jb <= jmax; jb += 256) {
    const int64_t j = jb + lane;
    const bool jin = j <= jmax;
    double acc[R], acc2[R];
#pragma unroll
    for (int r = 0; r < R; ++r) { acc[r] = 0.0; acc2[r] = 0.0; }
    if (jin) {
#pragma unroll 2
      for (int d0 = 0; d0 < D; d0 += 8) {
        double bv[8], bv2[8];
        load8<T>(B1 + j * D + d0, bv);
        if (MODE != FBSA_SCORE_DOT) load8<T>(B2 + j * D + d0, bv2);
#pragma unroll
        for (int e = 0; e < 8; ++e)
#pragma unroll
          for (int r = 0; r < R; ++r) {
            if (MODE == FBSA_SCORE_QUEST) {
              acc[r] = __builtin_fma(sa[0][r][d0 + e], bv[e], acc[r]);
              acc2[r] = __builtin_fma(sa[1][r][d0 + e], bv2[e], acc2[r]);
            } else {
              acc[r] = __builtin_fma(sa[0][r][d0 + e], bv[e], acc[r]);
              if (MODE == FBSA_SCORE_MAX2) acc2[r] = __builtin_fma(sa[0][r][d0 + e], bv2[e], acc2[r]);
            }
          }
      }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int64_t i = i0 + r;
      float sc;
      if (MODE == FBSA_SCORE_DOT) sc = round_dt<T>(acc[r]);
      else if (MODE == FBSA_SCORE_MAX2) sc = fmaxf(round_dt<T>(acc[r]), round_dt<T>(acc2[r]));
      else sc = round_dt_f<T>(round_dt<T>(acc[r]) + round_dt<T>(acc2[r]));  // bf16+bf16 is exact in fp32
      if (jin && j == i) diag[r] = sc;
      if (jin && j == 0) sinks[r] = sc;
      bool cand = jin && i < a.nblk && K > 0;
      if (convA) cand = cand && (a.causal ? j < i : j != i);
      else cand = cand && j <= i;
      const uint64_t key = make_key(sc, (int)j);
      // reject against the current K-th key (list entry K-1)
      const uint64_t kth = readlane_u64(lst[r], K > 0 ? K - 1 : 0);
      uint64_t surv = __ballot(cand && key > kth);
      while (surv) {
        const int src = __ffsll((unsigned long long)surv) - 1;
        surv &= surv - 1;
        const uint64_t c = readlane_u64(key, src);
        list_insert(lst[r], c, lane, K);
      }
    }
  }

  // merge the 4 per-wave lists of each row in wave 0..3 (row r -> wave r % 4)
#pragma unroll
  for (int r = 0; r < R; ++r) lists[w][r][lane] = lst[r];
  __syncthreads();
  for (int r = w; r < R; r += 4) {
    const int64_t i = i0 + r;
    if (i >= a.row1) continue;
    uint64_t mine = lists[0][r][lane];
    for (int ww = 1; ww < 4; ++ww)
      for (int l = 0; l < K; ++l) {
        const uint64_t c = lists[ww][r][l];
        if (c == 0) break;
        list_insert(mine, c, lane, K);
      }
    const float dsc = diag[r];
    int32_t *srow = a.sel + (bh * a.nblk + i) * a.kk;
    float *scrow = a.sel_score ? a.sel_score + (bh * a.nblk + i) * a.kk : nullptr;
    if (convA) {
      // slot 0 = own block; slots 1..K = list order; missing picks -> own
      const uint64_t prev = wave_shr1_u64(mine);
      if (lane < a.kk) {
        int idx = (int)i;
        float sc = dsc;
        if (lane >= 1 && prev != 0) { idx = key_index(prev); sc = key_score(prev); }
        srow[lane] = idx;
        if (scrow) scrow[lane] = sc;
      }
    } else {
      // _finish: K picks (non-finite or missing -> own), own, sink; sorted ascending
      int idx = (int)i;
      float sc = dsc;
      if (lane < K) {
        if (mine != 0) {
          const float v = key_score(mine);
          if (isfinite(v)) { idx = key_index(mine); sc = v; }
        }
      } else if (lane == K + 1 && a.sink) { idx = 0; sc = sinks[r]; }
      const int n = (int)a.kk;
      int rank = 0;
      for (int m = 0; m < n; ++m) {
        const int om = __builtin_amdgcn_readlane(idx, m);
        rank += (om < idx) || (om == idx && m < lane);
      }
      if (lane < n) {
        srow[rank] = idx;
        if (scrow) scrow[rank] = sc;
      }
    }
  }
}

// ------------------------------------------------ wide top-k (K > 62)
//
// Budgets past one wave-wide list: one workgroup per (batch, head, query row).
// Candidates are scored exactly as in select_kernel (fp64 dot products in
// dimension order, rounded where torch rounds) in tiles of KP, where KP is a
// power of two >= max(K, 256). LDS holds the row's best keys so far (sorted,
// descending; 0 = empty) followed by the tile; a tile with no key above the
// current K-th is skipped, otherwise the 2 KP keys are sorted (bitonic network)
// and the first KP kept. Keys order as in the other kernels (score, then the
// lower block index), so the chosen blocks are the same.
__device__ __forceinline__ void bitonic_desc_u64(uint64_t *v, int n, int tid) {
  for (int k = 2; k <= n; k <<= 1)
    for (int jj = k >> 1; jj > 0; jj >>= 1) {
      for (int x = tid; x < n; x += 256) {
        const int y = x ^ jj;
        if (y > x) {
          const uint64_t p = v[x], q = v[y];
          const bool desc = (x & k) == 0;
          if (desc ? p < q : p > q) { v[x] = q; v[y] = p; }
        }
      }
      __syncthreads();
    }
}

template <typename T, int D, int MODE>
__global__ __launch_bounds__(256) void select_wide_kernel(SelArgs a, int KP) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  uint64_t *buf = (uint64_t *)smem;                     // [2 KP] best keys | tile
  double *qa = (double *)(buf + 2 * KP);                // [2][D] query operand (QUEST: relu / negative parts)
  float *osc = (float *)(qa + 2 * D);                   // [KP + 2] scores of the output slots
  __shared__ float s_diag, s_sink;
  const int tid = threadIdx.x;
  const int64_t nrows = a.row1 - a.row0;
  const int64_t bh = blockIdx.x / nrows;
  const int64_t i = a.row1 - 1 - (int64_t)blockIdx.x % nrows;  // later (longer) rows first
  const T *A = (const T *)a.a + bh * a.nblk * D;
  const T *B1 = (const T *)a.b1 + bh * a.nblk * D;
  const T *B2 = MODE != FBSA_SCORE_DOT ? (const T *)a.b2 + bh * a.nblk * D : nullptr;
  for (int d = tid; d < D; d += 256) {
    const double v = (double)(float)A[i * D + d];
    if (MODE == FBSA_SCORE_QUEST) { qa[d] = v > 0.0 ? v : 0.0; qa[D + d] = v < 0.0 ? v : 0.0; }
    else qa[d] = v;
  }
  for (int x = tid; x < KP; x += 256) buf[x] = 0;
  __syncthreads();
  auto score = [&](int64_t j) {
    double acc = 0.0, acc2 = 0.0;
    for (int d0 = 0; d0 < D; d0 += 8) {
      double bv[8], bv2[8];
      load8<T>(B1 + j * D + d0, bv);
      if (MODE != FBSA_SCORE_DOT) load8<T>(B2 + j * D + d0, bv2);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        if (MODE == FBSA_SCORE_QUEST) {
          acc = __builtin_fma(qa[d0 + e], bv[e], acc);
          acc2 = __builtin_fma(qa[D + d0 + e], bv2[e], acc2);
        } else {
          acc = __builtin_fma(qa[d0 + e], bv[e], acc);
          if (MODE == FBSA_SCORE_MAX2) acc2 = __builtin_fma(qa[d0 + e], bv2[e], acc2);
        }
      }
    }
    if (MODE == FBSA_SCORE_DOT) return round_dt<T>(acc);
    if (MODE == FBSA_SCORE_MAX2) return fmaxf(round_dt<T>(acc), round_dt<T>(acc2));
    return round_dt_f<T>(round_dt<T>(acc) + round_dt<T>(acc2));
  };
  if (tid == 0) s_diag = score(i);
  if (tid == 64) s_sink = score(0);
  const bool convA = a.conv == FBSA_SEL_OWN_FIRST;
  const int K = (int)(convA ? (a.topk < a.nblk - 1 ? a.topk : a.nblk - 1) : (a.topk < a.nblk ? a.topk : a.nblk));
  const int64_t jmax = (a.causal || !convA) ? i : a.nblk - 1;
  for (int64_t t0 = 0; t0 <= jmax; t0 += KP) {
    const uint64_t kth = buf[K - 1];  // stable: the previous tile ended with a barrier
    int any = 0;
    for (int x = tid; x < KP; x += 256) {
      const int64_t j = t0 + x;
      uint64_t key = 0;
      if (j <= jmax && (convA ? (a.causal ? j < i : j != i) : true)) {
        key = make_key(score(j), (int)j);
        if (key <= kth) key = 0;
      }
      buf[KP + x] = key;
      any |= key != 0;
    }
    if (!__syncthreads_or(any)) continue;
    bitonic_desc_u64(buf, 2 * KP, tid);
  }
  __syncthreads();
  int32_t *srow = a.sel + (bh * a.nblk + i) * a.kk;
  float *scrow = a.sel_score ? a.sel_score + (bh * a.nblk + i) * a.kk : nullptr;
  const float dsc = s_diag;
  if (convA) {
    // slot 0 = own block, slots 1..K in score order; missing picks -> own
    for (int s = tid; s < a.kk; s += 256) {
      int idx = (int)i;
      float sc = dsc;
      if (s >= 1 && buf[s - 1] != 0) { idx = key_index(buf[s - 1]); sc = key_score(buf[s - 1]); }
      srow[s] = idx;
      if (scrow) scrow[s] = sc;
    }
    return;
  }
  // _finish: K picks (non-finite or missing -> own), own, sink; sorted ascending
  // (by block, then slot: keys block << 32 | slot into the free tile half)
  const int n = (int)a.kk;
  for (int s = tid; s < n; s += 256) {
    int idx = (int)i;
    float sc = dsc;
    if (s < K) {
      const uint64_t kv = buf[s];
      if (kv != 0 && isfinite(key_score(kv))) { idx = key_index(kv); sc = key_score(kv); }
    } else if (s == K + 1) {
      idx = 0;
      sc = s_sink;
    }
    osc[s] = sc;
    buf[KP + s] = ((uint64_t)(uint32_t)idx << 32) | (uint32_t)s;
  }
  int np = 1;
  while (np < n) np <<= 1;
  for (int s = n + tid; s < np; s += 256) buf[KP + s] = 0;  // empties sort last in descending order
  __syncthreads();
  bitonic_desc_u64(buf + KP, np, tid);
  for (int s = tid; s < n; s += 256) {
    const uint64_t kv = buf[KP + n - 1 - s];  // ascending
    srow[s] = (int32_t)(kv >> 32);
    if (scrow) scrow[s] = osc[(uint32_t)kv];
  }
}

// ------------------------------------------------ MFMA selection (16-bit operands)
//
// Scores come from bf16/fp16 MFMA (fp32 accumulate). With exact 16-bit
// products, the fp32 result differs from the exact dot product by at most
// beta = 4 (D + 4) 2^-24 |a| |b| (any summation order, round-to-nearest or
// toward zero, plus the final fp32 rounding), so rounding r - beta and
// r + beta to the score dtype brackets the exactly rounded score (rounding is
// monotone):
//   * a candidate whose upper end lies below the row's reject boundary (the
//     rounding midpoint under its current k-th score) cannot enter the row's
//     top-k and is dropped with one compare -- almost every candidate once the
//     row has a k-th score;
//   * a survivor whose bracket collapses has its exact score; otherwise the
//     score is recomputed exactly in fp64 from the 16-bit operands (rare).
// Survivors are appended to a per-row buffer; a full buffer is compacted to
// its top k by a wave-wide bitonic sort of (score, complemented index) keys,
// which also raises the reject boundary. Keys order exactly as in the fp64
// kernel, so the selected blocks and their tie-break are identical.
//
// Work split: a workgroup takes 64 query rows (16 per wave, one MFMA tile
// each) and one chunk of candidate tiles (64 candidates), streamed through a
// two-stage direct-to-LDS ring shared by the waves. Rows with more than one
// chunk leave per-chunk top-k keys that select_merge_kernel combines.

// max(m, x) ignoring a NaN x (IEEE maxNum); one instruction.
__device__ __forceinline__ float vmax(float m, float x) {
  float r;
  asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(m), "v"(x));
  return r;
}

// Norm arrays hold nbp = nblk rounded up to 64 entries per (batch, head), so a
// 64-candidate tile of norms is one aligned run; the padding is never used.
__host__ __device__ static inline int64_t sel_norm_pitch(int64_t nblk) { return (nblk + 63) & ~(int64_t)63; }

template <typename T, int D, int MODE>
__global__ __launch_bounds__(256) void sel_norms_kernel(SelArgs a, int64_t nneed, float *an1, float *an2,
                                                        float *bn1, float *bn2) {
  // rows [0, nneed) of every (batch, head)
  const int64_t r = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (r >= a.B * a.H * nneed) return;
  const int64_t row = r / nneed * a.nblk + r % nneed;
  const int64_t nrow = r / nneed * sel_norm_pitch(a.nblk) + r % nneed;
  const T *A = (const T *)a.a + row * D;
  const T *B1 = (const T *)a.b1 + row * D;
  const T *B2 = MODE != FBSA_SCORE_DOT ? (const T *)a.b2 + row * D : nullptr;
  double sa1 = 0.0, sa2 = 0.0, sb1 = 0.0, sb2 = 0.0;
  for (int d0 = 0; d0 < D; d0 += 8) {
    double v[8], w1[8], w2[8];
    load8<T>(A + d0, v);
    load8<T>(B1 + d0, w1);
    if (MODE != FBSA_SCORE_DOT) load8<T>(B2 + d0, w2);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      if (MODE == FBSA_SCORE_QUEST) {
        if (v[e] > 0.0) sa1 += v[e] * v[e];
        else sa2 += v[e] * v[e];
      } else {
        sa1 += v[e] * v[e];
      }
      sb1 += w1[e] * w1[e];
      if (MODE != FBSA_SCORE_DOT) sb2 += w2[e] * w2[e];
    }
  }
  an1[nrow] = sel_row_norm(sa1, false);
  an2[nrow] = sel_row_norm(sa2, false);
  bn1[nrow] = sel_row_norm(sb1, true);
  bn2[nrow] = sel_row_norm(sb2, true);
}

// Wave-wide bitonic sort of 64 keys (one per lane), descending.
__device__ __forceinline__ uint64_t wave_sort_desc(uint64_t v, int lane) {
#pragma unroll
  for (int k = 2; k <= 64; k <<= 1)
#pragma unroll
    for (int j = k >> 1; j > 0; j >>= 1) {
      const uint32_t lo = (uint32_t)__shfl_xor((int)(uint32_t)v, j, 64);
      const uint32_t hi = (uint32_t)__shfl_xor((int)(uint32_t)(v >> 32), j, 64);
      const uint64_t pv = ((uint64_t)hi << 32) | lo;
      const bool desc = (lane & k) == 0;    // this lane's run is sorted descending
      const bool lower = (lane & j) == 0;   // this lane holds the first element of the pair
      const bool keep_max = lower == desc;
      v = keep_max ? (v > pv ? v : pv) : (v < pv ? v : pv);
    }
  return v;
}

// Largest fp32 value below which every value rounds (in T) to less than s:
// the midpoint between s and the next smaller T value.
template <typename T> __device__ __forceinline__ float reject_boundary(float s) {
  if (!(s > -INFINITY)) return -INFINITY;  // -inf or NaN: nothing can be rejected
  if (s == INFINITY) return s;
  if constexpr (__is_same(T, bf16)) {
    uint32_t u = __float_as_uint(s);
    // next smaller bf16: step the 16-bit pattern down (toward -inf)
    uint32_t prev;
    if (s == 0.f) prev = 0x80010000u;  // -smallest subnormal bf16
    else if (u & 0x80000000u) prev = u + 0x10000u;
    else prev = u - 0x10000u;
    return (float)(((double)s + (double)__uint_as_float(prev)) * 0.5);
  } else {
    const _Float16 h = (_Float16)s;
    unsigned short b;
    __builtin_memcpy(&b, &h, 2);
    unsigned short pb;
    if (s == 0.f) pb = 0x8001;
    else if (b & 0x8000) pb = (unsigned short)(b + 1);
    else pb = (unsigned short)(b - 1);
    _Float16 ph;
    __builtin_memcpy(&ph, &pb, 2);
    return (float)(((double)s + (double)(float)ph) * 0.5);
  }
}

// Exact score of (query row i, candidate j), rounded like torch, from the
// operands in global memory (fp64 products and sum).
template <typename T, int D, int MODE>
__device__ float exact_score_global(const SelArgs &a, int64_t bh, int64_t i, int64_t j) {
  const T *A = (const T *)a.a + (bh * a.nblk + i) * D;
  float part[2] = {0.f, 0.f};
  const int nop = MODE == FBSA_SCORE_DOT ? 1 : 2;
  for (int op = 0; op < nop; ++op) {
    const T *Bj = (const T *)(op ? a.b2 : a.b1) + (bh * a.nblk + j) * D;
    double acc = 0.0;
    for (int d0 = 0; d0 < D; d0 += 8) {
      double av[8], bv[8];
      load8<T>(A + d0, av);
      load8<T>(Bj + d0, bv);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        double x = av[e];
        if (MODE == FBSA_SCORE_QUEST) x = op == 0 ? (x > 0.0 ? x : 0.0) : (x < 0.0 ? x : 0.0);
        acc = __builtin_fma(x, bv[e], acc);
      }
    }
    part[op] = round_dt<T>(acc);
  }
  if (MODE == FBSA_SCORE_DOT) return part[0];
  if (MODE == FBSA_SCORE_MAX2) return fmaxf(part[0], part[1]);
  return round_dt_f<T>(part[0] + part[1]);
}

// Writes a row's selection from its top-K keys (lane l holds the l-th best;
// 0 = none): own-first (convention A) or _finish (convention B).
template <typename T, int D, int MODE>
__device__ void emit_row(const SelArgs &a, int64_t bh, int64_t i, uint64_t mine, int lane, int K) {
  const bool convA = a.conv == FBSA_SEL_OWN_FIRST;
  int32_t *srow = a.sel + (bh * a.nblk + i) * a.kk;
  float *scrow = a.sel_score ? a.sel_score + (bh * a.nblk + i) * a.kk : nullptr;
  float dsc = 0.f, ssc = 0.f;
  if (scrow) {
    dsc = exact_score_global<T, D, MODE>(a, bh, i, i);
    if (!convA && a.sink) ssc = exact_score_global<T, D, MODE>(a, bh, i, 0);
  }
  if (convA) {
    const uint64_t prev = wave_shr1_u64(mine);
    if (lane < a.kk) {
      int idx = (int)i;
      float sc = dsc;
      if (lane >= 1 && prev != 0) { idx = key_index(prev); sc = key_score(prev); }
      srow[lane] = idx;
      if (scrow) scrow[lane] = sc;
    }
  } else {
    int idx = (int)i;
    float sc = dsc;
    if (lane < K) {
      if (mine != 0) {
        const float v = key_score(mine);
        if (isfinite(v)) { idx = key_index(mine); sc = v; }
      }
    } else if (lane == K + 1 && a.sink) { idx = 0; sc = ssc; }
    const int n = (int)a.kk;
    int rank = 0;
    for (int m = 0; m < n; ++m) {
      const int om = __builtin_amdgcn_readlane(idx, m);
      rank += (om < idx) || (om == idx && m < lane);
    }
    if (lane < n) {
      srow[rank] = idx;
      if (scrow) scrow[rank] = sc;
    }
  }
}

// ring depth of the tiled selection for 16-bit d <= 64 dot scores: two stages
// (about 50 KB of LDS, three workgroups per CU) measured faster than four (74 KB,
// two per CU): 3.01 against 3.92 ms over 65536 blocks, 60 against 61 us over 4096
#ifndef FBSA_SELT_NST
#define FBSA_SELT_NST 2
#endif
template <typename T, int D, int MODE> struct SelTCfg {
  static constexpr int KS = D / 32;
  static constexpr int NOP = MODE == FBSA_SCORE_DOT ? 1 : 2;
  static constexpr int CPR = D * 2 / 16;         // 16-byte chunks per candidate row
  static constexpr int OPB = 64 * D * 2;         // one operand tile (64 candidates)
  static constexpr int NRMB = NOP * 64 * 4;      // the tile's candidate norms
  static constexpr int STB = NOP * OPB + NRMB;   // one ring stage
  static constexpr int LPT = NOP * OPB / (256 * 16);
  static constexpr int CAP = 64;                 // per-row key buffer
  static constexpr int NST = NOP * OPB <= 8192 ? FBSA_SELT_NST : 2;  // ring depth
  static constexpr int OFF_BUF = NST * STB;
  static constexpr int OFF_ROWN = OFF_BUF + 64 * (CAP + 1) * 8;
  static constexpr int OFF_CNT = OFF_ROWN + 2 * 64 * 4;
  static constexpr int LDS = OFF_CNT + 64 * 4;
  static_assert(LPT * 256 * 16 == NOP * OPB, "stage must split evenly over threads");
};

// LDS fetch-and-add, returning the old value. Inline asm: the compiler's
// atomic waits for every outstanding direct-to-LDS load first.
__device__ __forceinline__ int lds_fetch_add(int *p, int v) {
  int r;
  asm volatile("ds_add_rtn_u32 %0, %1, %2\n\ts_waitcnt lgkmcnt(0)"
               : "=v"(r)
               : "v"((unsigned)(uintptr_t)p), "v"(v)
               : "memory");
  return r;
}

// Register grids indexed by per-lane values: a binary tree of selects on the
// index bits (a chain of compares against 1, 2, 3 gets turned into indexed
// scratch memory).
__device__ __forceinline__ float pick4(float v0, float v1, float v2, float v3, int i) {
  const float lo = (i & 1) ? v1 : v0, hi = (i & 1) ? v3 : v2;
  return (i & 2) ? hi : lo;
}
__device__ __forceinline__ float pick4(const float (&v)[4], int i) { return pick4(v[0], v[1], v[2], v[3], i); }
__device__ __forceinline__ int pick4i(const int (&v)[4], int i) {
  const int lo = (i & 1) ? v[1] : v[0], hi = (i & 1) ? v[3] : v[2];
  return (i & 2) ? hi : lo;
}
__device__ __forceinline__ float pick16(const f32x4 (&v)[4], int t, int r) {
  return pick4(pick4(v[0][0], v[1][0], v[2][0], v[3][0], t), pick4(v[0][1], v[1][1], v[2][1], v[3][1], t),
               pick4(v[0][2], v[1][2], v[2][2], v[3][2], t), pick4(v[0][3], v[1][3], v[2][3], v[3][3], t), r);
}

// Sorts, descending, four independent sets of 64 values (index r), each held
// by a 16-lane group of the wave: element 4 p + i of set r is v[r][i] of lane
// p of the group. The four sorts run interleaved so the lane exchanges overlap.
__device__ __forceinline__ void group_sort64x4_desc(float (&v)[4][4], int p) {
#pragma unroll
  for (int k = 2; k <= 64; k <<= 1)
#pragma unroll
    for (int j = k >> 1; j > 0; j >>= 1) {
      if (j >= 4) {
        const int lx = j >> 2;  // partner lane p ^ lx, same register
        const bool lower = (p & lx) == 0;
        float o[4][4];
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
          for (int i = 0; i < 4; ++i) o[r][i] = __shfl_xor(v[r][i], lx, 64);
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const bool desc = ((4 * p + i) & k) == 0;
            v[r][i] = lower == desc ? fmaxf(v[r][i], o[r][i]) : fminf(v[r][i], o[r][i]);
          }
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            if (i & j) continue;
            const bool desc = ((4 * p + i) & k) == 0;
            const float x = v[r][i], y = v[r][i | j];
            v[r][i] = desc ? fmaxf(x, y) : fminf(x, y);
            v[r][i | j] = desc ? fminf(x, y) : fmaxf(x, y);
          }
      }
    }
}

// Two passes over a workgroup's candidate tiles, on MFMA bounds:
//  * each score is formed by MFMA together with a rank-1 term +-beta(i, j),
//    beta = bf16_up(CB |a_i|) * bf16_up(|b_j|) with CB = 4 (D+8) 2^-24 (1.01):
//    that covers the accumulation error of the D products and of the term
//    itself, so lo(i, j) <= exact score <= hi(i, j) comes straight out of
//    the matrix core (the norm arrays hold bf16-rounded-up values);
//  1. per row, the maximum of lo over each of 64 candidate streams (stream =
//     position in the tile). The K-th largest stream maximum tau is the lower
//     end of K distinct candidates, so rnd(tau) <= the row's K-th best score,
//     and a candidate whose hi lies below the rounding midpoint under rnd(tau)
//     has K candidates strictly above it: it cannot be selected.
//  2. candidates at or above that boundary get exact keys (the bracket
//     [hi - 2.02 beta, hi] rounded, or fp64 when that is ambiguous) and go to
//     the row's key buffer; a buffer near capacity is cut to its top K, which
//     also raises the boundary to the midpoint under its K-th score.
// Pass 2 keeps about K candidates per row, so the exact work and the
// bookkeeping stay small next to the MFMA and the reject compare.

template <typename T, int D, int MODE>
__global__ __launch_bounds__(256) void select_tiled_kernel(SelArgs a) {
  using C = SelTCfg<T, D, MODE>;
  constexpr int NST = C::NST;
  constexpr int NA = MODE == FBSA_SCORE_QUEST ? 2 : 1;  // query-side operand parts
  constexpr float CB = 4.f * (float)(D + 8) * 5.9604645e-8f * 1.01f;
  // All LDS is one dynamic block (C::LDS bytes): accesses to statically
  // declared LDS get a wait for every outstanding direct-to-LDS load inserted
  // before them, which would drain the prefetch ring.
  extern __shared__ __attribute__((aligned(16))) char smem[];
  char *ring = smem;                                             // NST stages
  auto buf = (uint64_t(*)[C::CAP + 1])(smem + C::OFF_BUF);     // per-row entry buffers (padded pitch)
  auto rown = (float(*)[64])(smem + C::OFF_ROWN);              // bf16_up(CB |a-part|) per row
  int *cnt = (int *)(smem + C::OFF_CNT);                       // key buffer fill

  const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63, g = lane >> 4, p = lane & 15;
  // row blocks [rb0, rb1) cover this launch's rows [row0, row1)
  const int64_t rb0 = a.row0 / 64, rb1 = (a.row1 + 63) / 64, nrr = rb1 - rb0;
  // consecutive work items (same head) on one XCD, so its L2 holds that head's candidates
  int64_t x = xcd_remap(blockIdx.x, gridDim.x);
  const int64_t ch = x % a.nch; x /= a.nch;
  // tile and block indices fit 32 bits (the host rejects nblk >= 2^31 - 64)
  const int rb = (int)(rb1 - 1 - x % nrr);  // heavy (late) row blocks first
  const int64_t bh = x / nrr;
  const int r0 = rb * 64;
  const bool convA = a.conv == FBSA_SEL_OWN_FIRST;
  const int nb = (int)a.nblk, ct = (int)a.ct;
  const int last_row = r0 + 63 < nb - 1 ? r0 + 63 : nb - 1;
  const int jmax = (a.causal || !convA) ? last_row : nb - 1;
  const int ntiles = jmax / 64 + 1;
  const int nchunks = (ntiles + ct - 1) / ct;
  const int t0 = (int)ch * ct, t1 = t0 + ct < ntiles ? t0 + ct : ntiles;
  if (t0 >= t1) return;  // uniform: this chunk is past the row block's candidates
  const int nt = (int)(t1 - t0);
  const int K = (int)(convA ? (a.topk < a.nblk - 1 ? a.topk : a.nblk - 1) : (a.topk < a.nblk ? a.topk : a.nblk));

  const T *A = (const T *)a.a + bh * a.nblk * D;
  const char *Bop[2] = {(const char *)((const T *)a.b1 + bh * a.nblk * D),
                        (const char *)((const T *)(MODE != FBSA_SCORE_DOT ? a.b2 : a.b1) + bh * a.nblk * D)};
  const int64_t nbp = sel_norm_pitch(a.nblk);
  const char *Nop[2] = {(const char *)(a.bn1 + bh * nbp), (const char *)(a.bn2 + bh * nbp)};
  const float *Anrm[2] = {a.an1 + bh * nbp, a.an2 + bh * nbp};

  // per-row beta factors and counters; MFMA A fragments of this wave's 16
  // rows (lane p <-> row r0 + 16w + p) and the rank-1 fragments (k = 0 held
  // by lanes g == 0)
  if (tid < 64) cnt[tid] = 0;
  if (tid < 64 * NA) {
    const int r = tid & 63;
    const int64_t i = r0 + r < a.nblk ? r0 + r : a.nblk - 1;
    rown[tid >> 6][r] = __uint_as_float(bf16_up_bits(CB * (tid < 64 ? Anrm[0] : Anrm[1])[i]) << 16);
  }
  s16x8 af[NA][C::KS];
  s16x8 alo[NA], ahi[NA];
  {
    const int64_t ip = r0 + 16 * w + p < a.nblk ? r0 + 16 * w + p : a.nblk - 1;
#pragma unroll
    for (int ks = 0; ks < C::KS; ++ks) {
      const s16x8 v = *(const s16x8 *)(A + ip * D + 32 * ks + 8 * g);
      if constexpr (MODE == FBSA_SCORE_QUEST) {
        s16x8 pos, neg;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const bool negative = v[e] < 0;  // sign bit of the 16-bit pattern
          pos[e] = negative ? (short)0 : v[e];
          neg[e] = negative ? v[e] : (short)0;
        }
        af[0][ks] = pos;
        af[1][ks] = neg;
      } else {
        af[0][ks] = v;
      }
    }
#pragma unroll
    for (int oa = 0; oa < NA; ++oa) {
      const uint32_t bb = bf16_up_bits(CB * Anrm[oa][ip]);
      ahi[oa] = s16x8{g == 0 ? (short)bb : (short)0, 0, 0, 0, 0, 0, 0, 0};
      alo[oa] = s16x8{g == 0 ? (short)(bb | 0x8000u) : (short)0, 0, 0, 0, 0, 0, 0, 0};
    }
  }

  // ring: LPT 16-byte loads of the operand tiles per thread plus one norm
  // load per wave. Thread chunk n of a stage: operand (4n + w) / CPR (uniform),
  // candidate row drow[n], byte offset doff[n] within the operand tile.
  uint32_t doff[C::LPT];
  int drow[C::LPT];
#pragma unroll
  for (int n = 0; n < C::LPT; ++n) {
    const int u = (n * 4 + w) * 64 + lane;
    const int rem = u % (64 * C::CPR);
    const int row = rem / C::CPR, pos = rem % C::CPR;
    drow[n] = row;
    doff[n] = (uint32_t)((row * D + (pos ^ swz(row, C::CPR)) * 8) * 2);
  }
  auto issue = [&](int tile, int stg) {
    char *st = ring + stg * C::STB;
    const int j0 = tile * 64;
    const int lim = nb - 1 - j0 < 63 ? nb - 1 - j0 : 63;  // last real candidate row
#pragma unroll
    for (int n = 0; n < C::LPT; ++n) {
      const int op = (n * 4 + w) / C::CPR;
      const char *tb = Bop[op] + j0 * D * 2;
      const int over = drow[n] - lim;  // ragged tile: repeat the last real row
      const uint32_t off = doff[n] - (uint32_t)(over > 0 ? over * D * 2 : 0);
      g2lds16(tb + off, st + (n * 4 + w) * 1024);
    }
    // norms: wave w copies candidates 16w..16w+15 of every operand; lane l
    // lands at byte 16 l of the wave's run, so float (w NOP + op) 16 + c
    // holds candidate 16 w + c of operand op (the per-head arrays are padded
    // to whole tiles)
    if (lane < 4 * C::NOP) {
      const int op = lane >> 2, part = lane & 3;
      g2lds16(Nop[op] + (j0 + 16 * w + 4 * part) * 4, st + C::NOP * C::OPB + w * C::NOP * 64);
    }
  };

  // A buffered entry is either an exact key (make_key: low word ~j, bit 31
  // set) or a pending candidate: low word j + 1 (nonzero, bit 31 clear), high
  // word the bits of its MFMA upper bound (DOT, MAX2). resolve() turns a pending entry of row
  // q into its exact key: the rounded bracket [hi - 2.02 beta, hi] when it
  // pins the score, else the fp64 dot product from global memory.
  auto resolve = [&](uint64_t e, int q) -> uint64_t {
    if (e == 0 || ((uint32_t)e & 0x80000000u)) return e;
    const int j = (int)(uint32_t)e - 1;
    float sc = 0.f;
    bool done = false;
    if constexpr (MODE != FBSA_SCORE_QUEST) {
      const float hi = __uint_as_float((uint32_t)(e >> 32));
      float bj = a.bn1[bh * nbp + j];
      if constexpr (MODE == FBSA_SCORE_MAX2) bj = fmaxf(bj, a.bn2[bh * nbp + j]);
      const float beta = rown[0][q] * bj;
      const float rl = round_dt_f<T>(hi - 2.02f * beta), rh = round_dt_f<T>(hi);
      if (rl == rh && isfinite(rh)) {
        sc = rh;
        done = true;
      }
    }
    if (!done) sc = exact_score_global<T, D, MODE>(a, bh, r0 + q, j);
    return make_key(sc, j);
  };

  // Cuts row 16w + qq (wave-uniform) of the entry buffer to its top K exact
  // keys, in descending order, and raises the row's reject boundary.
  float rej[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
  auto compact = [&](int qq, int n) -> int {
    const int q = 16 * w + qq;
    const uint64_t key = lane < n ? resolve(buf[q][lane], q) : 0;
    // rank = number of larger keys (keys are distinct), from lane reads: no LDS round trips
    int rank = 0;
    for (int m = 0; m < n; ++m) rank += readlane_u64(key, m) > key ? 1 : 0;
    if (lane < n && rank < K) buf[q][rank] = key;
    if (n >= K) {
      const uint64_t bal = __ballot(lane < n && rank == K - 1);
      const uint64_t kth = readlane_u64(key, (int)__builtin_ctzll(bal));
      const float nb = reject_boundary<T>(key_score(kth));
      if (g == (qq >> 2)) {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (r == (qq & 3)) rej[r] = fmaxf(rej[r], nb);
      }
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);
    return n < K ? n : K;
  };

  // validity of (row 4g + r, candidate 16t + p) on a diagonal or ragged tile: bit 4t + r
  const int ilim = nb - r0 < 64 ? nb - r0 : 64;
  uint32_t rowmask = 0;  // rows of this lane that exist (the last row block may be ragged)
#pragma unroll
  for (int r = 0; r < 4; ++r)
    if (16 * w + 4 * g + r < ilim) rowmask |= 0x1111u << r;
  auto valid_mask = [&](int tl) {
    const int jlim = nb - tl * 64 < 64 ? nb - tl * 64 : 64;
    const bool diag = tl == rb;
    const int dm = !diag ? 0 : convA ? (a.causal ? 1 : 2) : 3;  // none, j < i, j != i, j <= i
    uint32_t vm = 0;
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int il = 16 * w + 4 * g + r, jl = 16 * t + p, dd = il - jl;
        bool v = il < ilim && jl < jlim;
        v = v && (dm == 0 || (dm == 1 && dd > 0) || (dm == 2 && dd != 0) || (dm == 3 && dd >= 0));
        vm |= v ? 1u << (4 * t + r) : 0u;
      }
    return vm;
  };

  float smax[4][4];  // [t][r]: stream maxima of the lower ends
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) smax[t][r] = -INFINITY;
  int rcl[4] = {0, 0, 0, 0};  // entries buffered for rows 16w + 4g + r (same in all lanes of a group)

  // Tile order within each pass: the full off-diagonal tiles first, then the
  // (at most two) diagonal / ragged tiles, so those get loop bodies of their own.
  const int big = INT32_MAX / 4;
  int m1 = rb >= t0 && rb < t1 ? rb : big;                          // diagonal
  int m2 = (nb & 63) && t1 == (nb + 63) / 64 ? t1 - 1 : big;  // ragged last tile
  if (m2 == m1) m2 = big;
  if (m2 < m1) { const int tmp = m1; m1 = m2; m2 = tmp; }
  const int nm = (m1 != big) + (m2 != big);
  const int nu = nt - nm;
  auto tile_of = [&](int k) -> int {  // stage k: tile of pass k / nt
    const int kk = k < nt ? k : k - nt;
    if (kk >= nu) return kk == nu ? m1 : m2;
    int u = t0 + kk;
    if (u >= m1) ++u;
    if (u >= m2) ++u;
    return u;
  };

#pragma unroll
  for (int k = 0; k < NST - 1; ++k)
    if (k < 2 * nt) issue(tile_of(k), k);
  // the register-operand loads above and the first stages have landed (issued
  // together, so their latencies overlap): the compiler then waits for nothing
  // inside the ring loop, where its own waits would also drain the prefetch
  wait_vmcnt<0>();


  // one ring step: wait for stage it, refill, score its tile (lo in pass 1, hi in pass 2)
  auto step = [&](int it, auto masked_c, auto collect_c) {
    constexpr bool MASKED = decltype(masked_c)::value, COLLECT = decltype(collect_c)::value;
    const int stg = it % NST;
    const int tl = tile_of(it);
    // this wave's loads of stage it have landed (LPT + 1 per stage; later stages may be in flight)
    const int ahead = 2 * nt - 1 - it < NST - 2 ? 2 * nt - 1 - it : NST - 2;
    wait_ring<C::LPT + 1>(ahead);
    lds_barrier();  // every wave's part has landed; the stage refilled next is no longer read
    if (it + NST - 1 < 2 * nt) issue(tile_of(it + NST - 1), (it + NST - 1) % NST);
    const char *st = ring + stg * C::STB;
    const float *nrm = (const float *)(st + C::NOP * C::OPB);
    const int j0 = tl * 64;

    s16x8 bfr[C::NOP][4][C::KS];
    s16x8 bp[C::NOP][4];
#pragma unroll
    for (int op = 0; op < C::NOP; ++op)
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int row = 16 * t + p;
        const uint32_t nb = __float_as_uint(nrm[(t * C::NOP + op) * 16 + p]) >> 16;  // already bf16
        bp[op][t] = s16x8{g == 0 ? (short)nb : (short)0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
        for (int ks = 0; ks < C::KS; ++ks)
          bfr[op][t][ks] = *(const s16x8 *)(st + op * C::OPB + (row * C::CPR + ((4 * ks + g) ^ swz(row, C::CPR))) * 16);
      }
    f32x4 acc[C::NOP][4];
#pragma unroll
    for (int op = 0; op < C::NOP; ++op) {
      const int oa = MODE == FBSA_SCORE_QUEST ? op : 0;
      const s16x8 ar = COLLECT ? ahi[oa] : alo[oa];
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        // rank-1 term (k = 0 of an extra bf16 k-block). For bf16 operands it
        // heads the same-opcode accumulation chain; for fp16 it is a separate
        // product added afterwards (a chain mixing MFMA opcodes through the
        // accumulator reads it before the first product has landed)
        const f32x4 r1 = Mfma16<bf16>::run(ar, bp[op][t], f32x4{0.f, 0.f, 0.f, 0.f});
        acc[op][t] = __is_same(T, bf16) ? r1 : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < C::KS; ++ks) acc[op][t] = Mfma16<T>::run(af[oa][ks], bfr[op][t][ks], acc[op][t]);
        if constexpr (!__is_same(T, bf16)) acc[op][t] += r1;
      }
    }
    const uint32_t vm = MASKED ? valid_mask(tl) : rowmask;

    if constexpr (!COLLECT) {
      // pass 1: stream maxima of the lower ends (a NaN end is ignored)
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          float lo0 = acc[0][t][r], lo1 = -INFINITY;
          if constexpr (MODE == FBSA_SCORE_QUEST) lo0 = round_dt_f<T>(acc[0][t][r]) + round_dt_f<T>(acc[1][t][r]);
          if constexpr (MODE == FBSA_SCORE_MAX2) lo1 = acc[1][t][r];
          if (MASKED && !((vm >> (4 * t + r)) & 1u)) lo0 = lo1 = -INFINITY;
          smax[t][r] = vmax(smax[t][r], lo0);
          if constexpr (MODE == FBSA_SCORE_MAX2) smax[t][r] = vmax(smax[t][r], lo1);
        }
      return;
    } else {
      // pass 2: reject against the row's boundary (NaN survives)
      bool sr[4][4];
      uint64_t any = 0;
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          if constexpr (MODE == FBSA_SCORE_QUEST) {
            sr[t][r] = !(round_dt_f<T>(acc[0][t][r]) + round_dt_f<T>(acc[1][t][r]) < rej[r]);
          } else {
            sr[t][r] = !(acc[0][t][r] < rej[r]);
            if constexpr (MODE == FBSA_SCORE_MAX2) sr[t][r] = sr[t][r] || !(acc[1][t][r] < rej[r]);
          }
          any |= __ballot(sr[t][r]);
        }
      if (!any) return;
      uint32_t sv = 0;  // bit 4t + r: candidate 16t + p survives for row 4g + r
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) sv |= sr[t][r] ? 1u << (4 * t + r) : 0u;
      sv &= vm;

      // survivors, one per lane per round, appended as pending entries; the
      // slots come from ballots (rows of a group only receive entries from
      // that group's 16 lanes), the counts live in registers
      const uint64_t gm = 0xFFFFull << (16 * g);
      while (__ballot(sv != 0)) {
        {  // a round adds at most 16 entries to a row
          const bool near = rcl[0] > C::CAP - 16 || rcl[1] > C::CAP - 16 || rcl[2] > C::CAP - 16 || rcl[3] > C::CAP - 16;
          uint64_t ov = __ballot(near && p == 0);
          while (ov) {
            const int gg = (int)__builtin_ctzll(ov) >> 4;
            ov &= ov - 1;
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) {
              const int n = __builtin_amdgcn_readlane(rcl[rr], 16 * gg);
              if (n > C::CAP - 16) {
                const int nn = compact(4 * gg + rr, n);
                if (g == gg) rcl[rr] = nn;
              }
            }
          }
        }
        const bool has = sv != 0;
        const int b = has ? __builtin_ctz(sv) : 0;
        sv &= sv - 1;
        const int t = b >> 2, r = b & 3;
        uint64_t mr[4];
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) mr[rr] = __ballot(has && r == rr);
        if (has) {
          const uint64_t mine = (r == 0 ? mr[0] : r == 1 ? mr[1] : r == 2 ? mr[2] : mr[3]) & gm;
          const int off = (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(mine >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)mine, 0u));
          uint32_t hb = 0;
          if constexpr (MODE == FBSA_SCORE_DOT) {
            hb = __float_as_uint(pick16(acc[0], t, r));
          } else if constexpr (MODE == FBSA_SCORE_MAX2) {
            const float h0 = pick16(acc[0], t, r), h1 = pick16(acc[1], t, r);
            hb = __float_as_uint(h0 != h0 || h1 != h1 ? __builtin_nanf("") : fmaxf(h0, h1));
          }
          buf[16 * w + 4 * g + r][pick4i(rcl, r) + off] = ((uint64_t)hb << 32) | (uint32_t)(j0 + 16 * t + p + 1);
        }
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) rcl[rr] += __popcll(mr[rr] & gm);
      }
    }
  };

  using F = std::integral_constant<bool, false>;
  using Tr = std::integral_constant<bool, true>;
  for (int it = 0; it < nu; ++it) step(it, F{}, F{});
  for (int it = nu; it < nt; ++it) step(it, Tr{}, F{});
  {
    // pass-1 bound: K-th largest of the row's 64 stream maxima
    float v[4][4];
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int t = 0; t < 4; ++t) v[r][t] = smax[t][r];
    group_sort64x4_desc(v, p);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float tau = __shfl(pick4(v[r], (K - 1) & 3), 16 * g + ((K - 1) >> 2), 64);
      rej[r] = reject_boundary<T>(round_dt_f<T>(tau));
    }
  }
  for (int it = nt; it < nt + nu; ++it) step(it, F{}, Tr{});
  for (int it = nt + nu; it < 2 * nt; ++it) step(it, Tr{}, Tr{});
  __builtin_amdgcn_s_waitcnt(0xC07F);
  if (p == 0) {
#pragma unroll
    for (int r = 0; r < 4; ++r) cnt[16 * w + 4 * g + r] = rcl[r];
  }
  __builtin_amdgcn_s_waitcnt(0xC07F);

  // Pending entries -> exact keys, in place, for all 16 rows of the wave at
  // once: lane p holds entries p, p + 16, p + 32, p + 48 of rows 16w + 4qb + g.
  // The candidate norms of every pending entry are fetched together (one
  // memory round trip instead of one per entry), the rounded bracket settles
  // almost all of them, and the rest take the fp64 dot product.
  {
    uint32_t amb = 0;  // bit 4qb + e: entry left for the fp64 path
    if constexpr (MODE != FBSA_SCORE_QUEST) {
      uint64_t ke[4][4];
      float bj[4][4];
#pragma unroll
      for (int qb = 0; qb < 4; ++qb) {
        const int q = 16 * w + 4 * qb + g, n = cnt[q];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          ke[qb][e] = p + 16 * e < n ? buf[q][p + 16 * e] : 0;
          bj[qb][e] = 0.f;
          if (ke[qb][e] != 0 && !((uint32_t)ke[qb][e] & 0x80000000u)) {
            const int64_t j = (int64_t)(uint32_t)ke[qb][e] - 1;
            bj[qb][e] = a.bn1[bh * nbp + j];
            if constexpr (MODE == FBSA_SCORE_MAX2) bj[qb][e] = fmaxf(bj[qb][e], a.bn2[bh * nbp + j]);
          }
        }
      }
#pragma unroll
      for (int qb = 0; qb < 4; ++qb)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint64_t en = ke[qb][e];
          if (en == 0 || ((uint32_t)en & 0x80000000u)) continue;
          const int q = 16 * w + 4 * qb + g;
          const float hi = __uint_as_float((uint32_t)(en >> 32));
          const float beta = rown[0][q] * bj[qb][e];
          const float rl = round_dt_f<T>(hi - 2.02f * beta), rh = round_dt_f<T>(hi);
          if (rl == rh && isfinite(rh)) buf[q][p + 16 * e] = make_key(rh, (int)(uint32_t)en - 1);
          else amb |= 1u << (4 * qb + e);
        }
    } else {
#pragma unroll
      for (int qb = 0; qb < 4; ++qb) {
        const int q = 16 * w + 4 * qb + g, n = cnt[q];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint64_t en = p + 16 * e < n ? buf[q][p + 16 * e] : 0;
          if (en != 0 && !((uint32_t)en & 0x80000000u)) amb |= 1u << (4 * qb + e);
        }
      }
    }
    // one exact_score_global() instance: the loop stays rolled
#pragma unroll 1
    while (amb) {
      const int b = __builtin_ctz(amb);
      amb &= amb - 1;
      const int q = 16 * w + 4 * (b >> 2) + g, slot = p + 16 * (b & 3);
      const int j = (int)(uint32_t)buf[q][slot] - 1;
      buf[q][slot] = make_key(exact_score_global<T, D, MODE>(a, bh, r0 + q, j), j);
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);
  }

  // this chunk's top K of each row, 4 rows at a time (one per lane group):
  // lane p ranks keys p, p + 16, p + 32, p + 48 of its row against the row's
  // buffer. A single chunk stores them in descending order for emit_row();
  // otherwise they go straight to the row's partial list (zeros past the
  // row's entries), which the merge kernel combines.
  const bool single = nchunks == 1;
#pragma unroll 1
  for (int qb = 0; qb < 4; ++qb) {
    const int q = 16 * w + 4 * qb + g;
    const int n = cnt[q];
    const int nmax = __builtin_amdgcn_readfirstlane(
        max(max(__builtin_amdgcn_readlane(n, 0), __builtin_amdgcn_readlane(n, 16)),
            max(__builtin_amdgcn_readlane(n, 32), __builtin_amdgcn_readlane(n, 48))));
    uint64_t k[4];
    int rk[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      k[e] = p + 16 * e < n ? buf[q][p + 16 * e] : 0;
      rk[e] = 0;
    }
    for (int m = 0; m < nmax; m += 4) {
      uint64_t km[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) km[u] = m + u < n ? buf[q][m + u] : 0;
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int e = 0; e < 4; ++e) rk[e] += km[u] > k[e] ? 1 : 0;
    }
    if (single) {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (k[e] != 0 && rk[e] < K) buf[q][rk[e]] = k[e];
      if (p == 0) cnt[q] = n < K ? n : K;
      __builtin_amdgcn_s_waitcnt(0xC07F);
    } else {
      const int64_t i = r0 + q;
      if (i >= a.row0 && i < a.row1) {
        uint64_t *dst = a.part + ((bh * a.nblk + i) * a.nch + ch) * K;
        const int nk = n < K ? n : K;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if (k[e] != 0 && rk[e] < K) dst[rk[e]] = k[e];
          if (p + 16 * e >= nk && p + 16 * e < K) dst[p + 16 * e] = 0;
        }
      }
    }
  }
  if (!single) return;
  for (int qq = 0; qq < 16; ++qq) {
    const int q = 16 * w + qq;
    const int64_t i = r0 + q;
    if (i >= a.row1) break;
    if (i < a.row0) continue;
    const int n = __builtin_amdgcn_readfirstlane(cnt[q]);
    const uint64_t v = lane < n ? buf[q][lane] : 0;
    emit_row<T, D, MODE>(a, bh, i, v, lane, K);
  }
}

// Rows whose candidates span several chunks: merge the chunks' top-k keys.
template <typename T, int D, int MODE>
__global__ __launch_bounds__(256) void select_merge_kernel(SelArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t nr = a.row1 - a.row0;
  const int64_t rr = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);  // (bh, i - row0)
  if (rr >= a.B * a.H * nr) return;
  const int64_t i = a.row0 + rr % nr, bh = rr / nr;
  const int64_t row = bh * a.nblk + i;
  const bool convA = a.conv == FBSA_SEL_OWN_FIRST;
  const int64_t jmax = (a.causal || !convA) ? ((i / 64) * 64 + 63 < a.nblk - 1 ? (i / 64) * 64 + 63 : a.nblk - 1)
                                            : a.nblk - 1;
  const int64_t ntiles = jmax / 64 + 1;
  const int64_t nchunks = (ntiles + a.ct - 1) / a.ct;
  if (nchunks <= 1) return;
  const int K = (int)(convA ? (a.topk < a.nblk - 1 ? a.topk : a.nblk - 1) : (a.topk < a.nblk ? a.topk : a.nblk));
  const uint64_t *src = a.part + row * a.nch * K;
  const int64_t total = nchunks * K;
  uint64_t v = lane < K ? src[lane] : 0;  // chunk 0 (already sorted)
  for (int64_t off = K; off < total; off += 64 - K) {
    const int64_t e = off + (lane - K);
    if (lane >= K) v = e < total ? src[e] : 0;
    v = wave_sort_desc(v, lane);
  }
  if (lane >= K) v = 0;
  emit_row<T, D, MODE>(a, bh, i, v, lane, K);
}

// Candidate tiles per workgroup (chunk). Every chunk pays a fixed cost (its
// pass-1 bound, the cut of its buffers, its partial list, a merge), and a short
// chunk keeps more candidates (its bound comes from fewer tiles), so rows are
// cut into chunks only when the row blocks alone would leave the GPU idle:
// about two workgroups per CU (512 on MI355X's 256 CUs) at one workgroup of 64
// rows per resident slot, chunks of at least 8 tiles, and no chunk longer than
// half an even share of all tiles over those slots (the longest chunk sets the
// kernel's tail). `tri`: row block r has r + 1 candidate tiles (causal or
// convention B), else every row block has all of them. A nonzero override
// (descriptor flags) wins.
static void sel_chunking(int64_t B, int64_t H, int64_t nblk, bool tri, int64_t override_ct, int64_t *ct,
                         int64_t *nch) {
  const int64_t ntiles = (nblk + 63) / 64;
  const int64_t rbs = B * H * ntiles;
  int64_t c = override_ct;
  if (c <= 0) {
    const int64_t slots = 512;
    const int64_t want = (slots + rbs - 1) / rbs;  // chunks per row block
    c = (ntiles + want - 1) / want;
    const int64_t total = tri ? B * H * (ntiles * (ntiles + 1) / 2) : rbs * ntiles;
    int64_t cap = (total + 2 * slots - 1) / (2 * slots);
    if (cap < 64) cap = 64;  // rows of up to 64 tiles stay whole when the row blocks fill the GPU
    if (c > cap) c = cap;
    if (c < 8) c = 8;
  }
  *ct = c;
  *nch = (ntiles + c - 1) / c;
}

// Budgets up to 32: past that the pass-1 bound (the K-th of 64 stream maxima)
// lets most candidates through and the row buffers are cut over and over
// (k = 40: 204 against 217 us for the fp64 path over 4096 blocks; k = 48: 759
// against 239 us), so larger budgets take the fp64 path.
template <typename T, int D, int MODE> static bool sel_tiled_ok(const SelArgs &a) {
  if constexpr (sizeof(T) != 2 || (D != 32 && D != 64)) return false;
  const int64_t K = a.conv == FBSA_SEL_OWN_FIRST ? (a.topk < a.nblk - 1 ? a.topk : a.nblk - 1)
                                                 : (a.topk < a.nblk ? a.topk : a.nblk);
  return K >= 1 && K <= 32;
}

template <typename T, int D, int MODE> static int launch_sel(const SelArgs &a, void *ws, hipStream_t s) {
  if (a.row1 <= a.row0) return FBSA_OK;
  if (ws && sel_tiled_ok<T, D, MODE>(a)) {
    if constexpr (sizeof(T) == 2 && (D == 32 || D == 64)) {
      // norms of rows [0, nneed): the query rows' row blocks and every candidate they may select
      const int64_t rb1 = (a.row1 + 63) / 64;
      const int64_t nneed = (a.causal || a.conv != FBSA_SEL_OWN_FIRST) ? (rb1 * 64 < a.nblk ? rb1 * 64 : a.nblk)
                                                                        : a.nblk;
      const int64_t n = a.B * a.H * nneed;
      const int64_t npad = a.B * a.H * sel_norm_pitch(a.nblk);
      float *an1 = (float *)ws, *an2 = an1 + npad, *bn1 = an2 + npad, *bn2 = bn1 + npad;
      int e = FBSA_OK;
      if (!a.norms_ready) {
        hipLaunchKernelGGL((sel_norms_kernel<T, D, MODE>), dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, a,
                           nneed, an1, an2, bn1, bn2);
        e = hip_check(hipGetLastError(), "sel_norms_kernel launch");
        if (e) return e;
      }
      SelArgs b = a;
      b.an1 = an1; b.an2 = an2; b.bn1 = bn1; b.bn2 = bn2;
      b.part = (uint64_t *)(((uintptr_t)(bn2 + npad) + 255) & ~(uintptr_t)255);
      const int64_t nrr = rb1 - a.row0 / 64;
      using C = SelTCfg<T, D, MODE>;
      hipLaunchKernelGGL((select_tiled_kernel<T, D, MODE>), dim3((unsigned)(a.B * a.H * nrr * b.nch)), dim3(256),
                         C::LDS, s, b);
      e = hip_check(hipGetLastError(), "select_tiled_kernel launch");
      if (e || b.nch == 1) return e;
      const int64_t nrows = a.B * a.H * (a.row1 - a.row0);
      hipLaunchKernelGGL((select_merge_kernel<T, D, MODE>), dim3((unsigned)((nrows + 3) / 4)), dim3(256), 0, s, b);
      return hip_check(hipGetLastError(), "select_merge_kernel launch");
    }
  }
  const bool convA = a.conv == FBSA_SEL_OWN_FIRST;
  const int64_t K = convA ? (a.topk < a.nblk - 1 ? a.topk : a.nblk - 1) : (a.topk < a.nblk ? a.topk : a.nblk);
  if (K > kSelListMax) {
    int KP = 256;
    while (KP < K) KP <<= 1;
    const size_t lds = (size_t)2 * KP * 8 + (size_t)2 * D * 8 + (size_t)(KP + 2) * 4;
    {
      const int e = lds_optin((const void *)select_wide_kernel<T, D, MODE>, lds, "hipFuncSetAttribute(select_wide)");
      if (e) return e;
    }
    const int64_t nwg = (a.row1 - a.row0) * a.B * a.H;
    hipLaunchKernelGGL((select_wide_kernel<T, D, MODE>), dim3((unsigned)nwg), dim3(256), lds, s, a, KP);
    return hip_check(hipGetLastError(), "select_wide_kernel launch");
  }
  constexpr int R = 8;
  const int64_t ntile = (a.row1 - a.row0 + R - 1) / R;
  const int64_t nwg = ntile * a.B * a.H;
  hipLaunchKernelGGL((select_kernel<T, D, R, MODE>), dim3((unsigned)nwg), dim3(256), 0, s, a);
  return hip_check(hipGetLastError(), "select_kernel launch");
}
template <typename T, int D> static int sel_mode(const SelArgs &a, void *ws, hipStream_t s) {
  switch (a.score) {
    case FBSA_SCORE_DOT: return launch_sel<T, D, FBSA_SCORE_DOT>(a, ws, s);
    case FBSA_SCORE_MAX2: return launch_sel<T, D, FBSA_SCORE_MAX2>(a, ws, s);
    default: return launch_sel<T, D, FBSA_SCORE_QUEST>(a, ws, s);
  }
}
template <typename T> static int sel_d(const SelArgs &a, void *ws, hipStream_t s) {
  switch (a.D) {
    case 16: return sel_mode<T, 16>(a, ws, s);
    case 32: return sel_mode<T, 32>(a, ws, s);
    case 64: return sel_mode<T, 64>(a, ws, s);
    case 128: return sel_mode<T, 128>(a, ws, s);
    case 256: return sel_mode<T, 256>(a, ws, s);
  }
  return fail(FBSA_EUNSUPPORTED, "fbsa_select: operand dim %lld not in {16,32,64,128,256}", (long long)a.D);
}

size_t select_workspace_bytes(const fbsa_select_desc *d) {
  // MFMA path (16-bit operands of dim 32 or 64): four padded float norm arrays
  // and the per-(row, candidate chunk) top-k keys
  if (d->dtype == FBSA_F32 || (d->D != 32 && d->D != 64)) return 0;
  const int64_t n = d->B * d->H * d->nblk;
  int64_t ct, nch;
  sel_chunking(d->B, d->H, d->nblk, d->causal || d->convention != FBSA_SEL_OWN_FIRST,
               (d->flags >> FBSA_SEL_CHUNK_SHIFT) & 0xFFFF, &ct, &nch);
  const int64_t K = d->topk < d->nblk ? d->topk : d->nblk;
  return (size_t)(4 * d->B * d->H * sel_norm_pitch(d->nblk)) * sizeof(float) + 256 +
         (size_t)(n * nch * (K > 0 ? K : 1)) * sizeof(uint64_t);
}

static int run_select_as(const fbsa_select_desc *d, int64_t row0, int64_t row1, const void *av, const void *b1,
                         const void *b2, int32_t *sel, float *sel_score, void *ws, int norms_ready, hipStream_t s) {
  SelArgs a;
  a.a = av; a.b1 = b1; a.b2 = b2; a.sel = sel; a.sel_score = sel_score;
  a.an1 = a.an2 = a.bn1 = a.bn2 = nullptr;
  a.norms_ready = norms_ready;
  a.part = nullptr;
  a.row0 = row0;
  a.row1 = row1;
  sel_chunking(d->B, d->H, d->nblk, d->causal || d->convention != FBSA_SEL_OWN_FIRST,
               (d->flags >> FBSA_SEL_CHUNK_SHIFT) & 0xFFFF, &a.ct, &a.nch);
  a.B = d->B; a.H = d->H; a.nblk = d->nblk; a.D = d->D; a.topk = d->topk; a.kk = d->kk;
  a.conv = d->convention; a.causal = d->causal; a.sink = d->sink; a.score = d->score;
  switch (d->dtype) {
    case FBSA_BF16: return sel_d<bf16>(a, ws, s);
    case FBSA_F16: return sel_d<f16>(a, ws, s);
    default: return sel_d<float>(a, ws, s);
  }
}

int run_select(const fbsa_select_desc *d, int64_t row0, int64_t row1, const void *av, const void *b1, const void *b2,
               int32_t *sel, float *sel_score, void *ws, hipStream_t s) {
  return run_select_as(d, row0, row1, av, b1, b2, sel, sel_score, ws, 0, s);
}

// Mean-pooled q.k selection. With the MFMA engine's workspace, 16-bit
// operands of dim 32 or 64 and a budget of at most 48, q and k are pooled by
// one launch that also writes the selection's row norms (query side into the
// first norm array, candidate side into the third; DOT scores use no others),
// and the selection starts from them; otherwise pool, pool and select run as
// three calls. Either way qp, kp and sel are the same.
template <typename T, int D> static int pooled_pair(const fbsa_pool_desc *dq, const void *q, void *qp,
                                                    const fbsa_pool_desc *dk, const void *k, void *kp,
                                                    const fbsa_select_desc *d, float *nq, float *nk, hipStream_t s) {
  constexpr int DC = D / 8;
  PoolArgs a0 = pool_args(dq, q, qp, nullptr), a1 = pool_args(dk, k, kp, nullptr);
  const int64_t pitch = sel_norm_pitch(d->nblk);
  a0.norm = nq; a0.norm_pitch = pitch; a0.norm_key = 0;
  a1.norm = nk; a1.norm_pitch = pitch; a1.norm_key = 1;
  const int64_t nwg0 = a0.B * a0.Ho * a0.nblk, nwg1 = a1.B * a1.Ho * a1.nblk;
  if (a0.grp == 1 && a1.grp == 1) {  // plain token means: one block per wave
    const dim3 g4((unsigned)((nwg0 + nwg1 + 3) / 4));
    switch (dq->bs) {
      case 16: hipLaunchKernelGGL((pool_mean1_kernel<T, DC, 16>), g4, dim3(256), 0, s, a0, a1, nwg0, nwg0 + nwg1); break;
      case 32: hipLaunchKernelGGL((pool_mean1_kernel<T, DC, 32>), g4, dim3(256), 0, s, a0, a1, nwg0, nwg0 + nwg1); break;
      case 64: hipLaunchKernelGGL((pool_mean1_kernel<T, DC, 64>), g4, dim3(256), 0, s, a0, a1, nwg0, nwg0 + nwg1); break;
      default: hipLaunchKernelGGL((pool_mean1_kernel<T, DC, 128>), g4, dim3(256), 0, s, a0, a1, nwg0, nwg0 + nwg1); break;
    }
    return hip_check(hipGetLastError(), "pool_mean1_kernel (pair) launch");
  }
  const dim3 grid((unsigned)(nwg0 + nwg1));
  switch (dq->bs) {
    case 16: hipLaunchKernelGGL((pool_wave_kernel<T, DC, 16, FBSA_POOL_MEAN_TOK_THEN_GRP>), grid, dim3(256), 0, s, a0, a1, nwg0); break;
    case 32: hipLaunchKernelGGL((pool_wave_kernel<T, DC, 32, FBSA_POOL_MEAN_TOK_THEN_GRP>), grid, dim3(256), 0, s, a0, a1, nwg0); break;
    case 64: hipLaunchKernelGGL((pool_wave_kernel<T, DC, 64, FBSA_POOL_MEAN_TOK_THEN_GRP>), grid, dim3(256), 0, s, a0, a1, nwg0); break;
    default: hipLaunchKernelGGL((pool_wave_kernel<T, DC, 128, FBSA_POOL_MEAN_TOK_THEN_GRP>), grid, dim3(256), 0, s, a0, a1, nwg0); break;
  }
  return hip_check(hipGetLastError(), "pool_wave_kernel (pair) launch");
}

int run_select_mean_pooled(const fbsa_pool_desc *dq, const void *q, void *qp, const fbsa_pool_desc *dk, const void *k,
                           void *kp, const fbsa_select_desc *d, int32_t *sel, float *sel_score, void *ws, hipStream_t s) {
  const int64_t K = d->topk < d->nblk - 1 ? d->topk : d->nblk - 1;
  const bool fused = ws && d->dtype != FBSA_F32 && (d->D == 32 || d->D == 64) && K >= 1 && K <= 32 &&
                     (dq->bs == 16 || dq->bs == 32 || dq->bs == 64 || dq->bs == 128);
  if (!fused) {
    int e = run_pool(dq, q, qp, nullptr, s);
    if (!e) e = run_pool(dk, k, kp, nullptr, s);
    return e ? e : run_select(d, 0, d->nblk, qp, kp, nullptr, sel, sel_score, ws, s);
  }
  const int64_t npad = d->B * d->H * sel_norm_pitch(d->nblk);
  float *nq = (float *)ws, *nk = nq + 2 * npad;
  int e;
  if (d->dtype == FBSA_BF16) e = d->D == 32 ? pooled_pair<bf16, 32>(dq, q, qp, dk, k, kp, d, nq, nk, s)
                                            : pooled_pair<bf16, 64>(dq, q, qp, dk, k, kp, d, nq, nk, s);
  else e = d->D == 32 ? pooled_pair<f16, 32>(dq, q, qp, dk, k, kp, d, nq, nk, s)
                      : pooled_pair<f16, 64>(dq, q, qp, dk, k, kp, d, nq, nk, s);
  return e ? e : run_select_as(d, 0, d->nblk, qp, kp, nullptr, sel, sel_score, ws, 1, s);
}

}  // namespace fbsa
