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

#include "fbsa_common.h"
#include "fbsa_internal.h"

namespace fbsa {

// ---------------------------------------------------------------- rounding
// torch rounds a bf16/fp16 reduction twice: the exact value to the fp32
// accumulator, then fp32 -> dtype (both RNE). The fp32 step is kept opaque so
// the compiler cannot fold the pair into one double -> 16-bit rounding, which
// differs when the fp32 value lands exactly on a 16-bit midpoint.
__device__ __forceinline__ float rne_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return __uint_as_float(0x7FC00000u);  // NaN
  u += 0x7FFFu + ((u >> 16) & 1u);
  return __uint_as_float(u & 0xFFFF0000u);
}
template <typename T> __device__ __forceinline__ float round_dt_f(float f) {
  if constexpr (sizeof(T) == 4) return f;
  else if constexpr (__is_same(T, bf16)) return rne_bf16(f);
  else {
    asm volatile("" : "+v"(f));
    return (float)(T)f;
  }
}
template <typename T> __device__ __forceinline__ float round_dt(double x) {
  float f = (float)x;  // RNE to fp32
  asm volatile("" : "+v"(f));
  return round_dt_f<T>(f);
}

// ---------------------------------------------------------------- pooling
struct PoolArgs {
  const void *x;
  void *out, *out2;
  int64_t B, H, L, D, bs, nblk, grp, l_valid, Ho;
  int64_t sx[3];
  int op;
};

// 16-bit pattern -> fp32 (exact)
template <typename T> __device__ __forceinline__ float half_bits_to_f32(uint32_t h);
template <> __device__ __forceinline__ float half_bits_to_f32<bf16>(uint32_t h) { return __uint_as_float(h << 16); }
template <> __device__ __forceinline__ float half_bits_to_f32<f16>(uint32_t h) {
  const unsigned short hs = (unsigned short)h;
  _Float16 x;
  __builtin_memcpy(&x, &hs, 2);
  return (float)x;
}

// 8 consecutive elements (16 bytes) -> fp64
template <typename T> __device__ __forceinline__ void load8(const T *p, double *v) {
  const uint4 r = *(const uint4 *)p;
  const uint32_t w[4] = {r.x, r.y, r.z, r.w};
  if constexpr (sizeof(T) == 4) {
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = (double)__uint_as_float(w[e]);
    const uint4 r2 = *(const uint4 *)(p + 4);
    const uint32_t w2[4] = {r2.x, r2.y, r2.z, r2.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) v[4 + e] = (double)__uint_as_float(w2[e]);
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[2 * e] = (double)half_bits_to_f32<T>(w[e] & 0xFFFFu);
      v[2 * e + 1] = (double)half_bits_to_f32<T>(w[e] >> 16);
    }
  }
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
          hsum[e] += (double)round_dt<T>(tot / (double)a.bs);
        }
      }
      __syncthreads();
    }
    if (tid < DC) {
      T *o = (T *)a.out + ((b * a.Ho + ho) * a.nblk + i) * a.D + 8 * tid;
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = (T)round_dt<T>(hsum[e] / (double)a.grp);
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
        for (int e = 0; e < 8; ++e) acc[e] += (double)round_dt<T>(g[e] / (double)a.grp);
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
      for (int e = 0; e < 8; ++e) o[e] = (T)round_dt<T>(res[e] / (double)a.bs);
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
template <typename T, int DC, int BS, int OP>
__global__ __launch_bounds__(256) void pool_wave_kernel(PoolArgs a) {
  constexpr int NW = 4, TLW = 64 / DC;
  constexpr int RPH = BS >= TLW ? BS / TLW : 1;            // rows per lane per head (whole block in one wave)
  constexpr int RPW = BS >= NW * TLW ? BS / (NW * TLW) : 1;  // rows per lane when the waves split the block
  __shared__ double red[2][NW][DC][8];
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, c = lane % DC, tl = lane / DC;
  const int64_t blk = blockIdx.x;
  const int64_t i = blk % a.nblk;
  const int64_t ho = (blk / a.nblk) % a.Ho;
  const int64_t b = blk / (a.nblk * a.Ho);
  constexpr int op = OP;
  const int64_t nval = a.l_valid - i * BS < BS ? a.l_valid - i * BS : BS;  // valid tokens in the block (>= 1)
  auto rowptr = [&](int64_t h, int t) {
    const int tc = t < nval ? t : (int)nval - 1;
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
      for (int e = 0; e < 8; ++e) r0[e] += ok ? (double)round_dt<T>(g[e] / (double)a.grp) : 0.0;
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
      const double den = op == FBSA_POOL_MEAN_TOK_THEN_GRP ? (double)a.grp : (double)BS;
      ((T *)a.out)[off] = (T)round_dt<T>(tot / den);
    } else {
      double mn = red[0][0][cc][e], mx = red[1][0][cc][e];
#pragma unroll
      for (int ww = 1; ww < NW; ++ww) { mn = fmin(mn, red[0][ww][cc][e]); mx = fmax(mx, red[1][ww][cc][e]); }
      if (a.op == FBSA_POOL_MAX) ((T *)a.out)[off] = (T)(float)mx;
      else if (a.op == FBSA_POOL_MIN) ((T *)a.out)[off] = (T)(float)mn;
      else { ((T *)a.out)[off] = (T)(float)mn; ((T *)a.out2)[off] = (T)(float)mx; }
    }
  }
}

template <typename T, int DC, int BS> static void launch_pool_op(const PoolArgs &a, int64_t nwg, hipStream_t s) {
  switch (a.op) {
    case FBSA_POOL_MEAN_TOK_THEN_GRP:
      hipLaunchKernelGGL((pool_wave_kernel<T, DC, BS, FBSA_POOL_MEAN_TOK_THEN_GRP>), dim3((unsigned)nwg), dim3(256), 0, s, a);
      return;
    case FBSA_POOL_MEAN_GRP_THEN_TOK:
      hipLaunchKernelGGL((pool_wave_kernel<T, DC, BS, FBSA_POOL_MEAN_GRP_THEN_TOK>), dim3((unsigned)nwg), dim3(256), 0, s, a);
      return;
    default:  // MAX / MIN / MINMAX share one instantiation (the op picks the outputs)
      hipLaunchKernelGGL((pool_wave_kernel<T, DC, BS, FBSA_POOL_MINMAX>), dim3((unsigned)nwg), dim3(256), 0, s, a);
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

int run_pool(const fbsa_pool_desc *d, const void *x, void *out, void *out2, hipStream_t s) {
  PoolArgs a;
  a.x = x; a.out = out; a.out2 = out2;
  a.B = d->B; a.H = d->H; a.L = d->L; a.D = d->D; a.bs = d->bs; a.nblk = d->nblk; a.grp = d->grp;
  a.l_valid = d->l_valid; a.Ho = d->H / d->grp; a.op = d->op;
  for (int k = 0; k < 3; ++k) a.sx[k] = d->sx[k];
  const int64_t nwg = a.B * a.Ho * a.nblk;
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
  int64_t B, H, nblk, D, topk, kk;
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
  const int64_t ntile = (a.nblk + R - 1) / R;
  // heavy (late) row tiles first: blockIdx 0 gets the last tile
  const int64_t t = ntile - 1 - (int64_t)blockIdx.x % ntile;
  const int64_t bh = blockIdx.x / ntile;  // b * H + h
  const int64_t i0 = t * R;
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
    if (i >= a.nblk) continue;
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

template <typename T, int D, int MODE> static int launch_sel(const SelArgs &a, hipStream_t s) {
  constexpr int R = 8;
  const int64_t ntile = (a.nblk + R - 1) / R;
  const int64_t nwg = ntile * a.B * a.H;
  hipLaunchKernelGGL((select_kernel<T, D, R, MODE>), dim3((unsigned)nwg), dim3(256), 0, s, a);
  return hip_check(hipGetLastError(), "select_kernel launch");
}
template <typename T, int D> static int sel_mode(const SelArgs &a, hipStream_t s) {
  switch (a.score) {
    case FBSA_SCORE_DOT: return launch_sel<T, D, FBSA_SCORE_DOT>(a, s);
    case FBSA_SCORE_MAX2: return launch_sel<T, D, FBSA_SCORE_MAX2>(a, s);
    default: return launch_sel<T, D, FBSA_SCORE_QUEST>(a, s);
  }
}
template <typename T> static int sel_d(const SelArgs &a, hipStream_t s) {
  switch (a.D) {
    case 16: return sel_mode<T, 16>(a, s);
    case 32: return sel_mode<T, 32>(a, s);
    case 64: return sel_mode<T, 64>(a, s);
    case 128: return sel_mode<T, 128>(a, s);
    case 256: return sel_mode<T, 256>(a, s);
  }
  return fail(FBSA_EUNSUPPORTED, "fbsa_select: operand dim %lld not in {16,32,64,128,256}", (long long)a.D);
}

int run_select(const fbsa_select_desc *d, const void *av, const void *b1, const void *b2, int32_t *sel,
               float *sel_score, hipStream_t s) {
  SelArgs a;
  a.a = av; a.b1 = b1; a.b2 = b2; a.sel = sel; a.sel_score = sel_score;
  a.B = d->B; a.H = d->H; a.nblk = d->nblk; a.D = d->D; a.topk = d->topk; a.kk = d->kk;
  a.conv = d->convention; a.causal = d->causal; a.sink = d->sink; a.score = d->score;
  switch (d->dtype) {
    case FBSA_BF16: return sel_d<bf16>(a, s);
    case FBSA_F16: return sel_d<f16>(a, s);
    default: return sel_d<float>(a, s);
  }
}

}  // namespace fbsa
