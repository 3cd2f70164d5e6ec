// Row-block max Quest selection for gfx950 (fbsa_select_qmax).
//
// score(i, j) = max over the query vectors t of block i of
//     rnd(rnd(relu(a_t) . b1_j) + rnd(min(a_t, 0) . b2_j))
// with rnd() the rounding of the exact value to fp32 and then to the operand
// dtype, b1 = per-block key max, b2 = per-block key min. Query vectors past
// the end of the input are zero vectors (score 0), as the reference's zero
// padding makes them. The columns of row i are the key blocks j <= i, or the
// row's entry of a candidate list; the row then keeps the top-k columns
// (score descending, ties to the lower block index) written as _finish does
// (non-finite picks -> own block, + own, + sink, ascending) or, for a
// candidate stage, as the bare ascending top-k set.
//
// One workgroup (four waves) per (b, h, query block i), larger i first (the
// rows with the most columns start early). Two 32-bit orderable keys per
// column live in LDS.
//  1. Brackets (16-bit operands, 64 or 128 query vectors per block, D in
//     {64, 128, 256}): each of the four waves holds tok/64 tiles of 16 query
//     vectors, split into their positive and negative parts, as MFMA A
//     operands for the whole row. Tiles of 16 columns (their key max/min rows
//     and norms, precomputed once per launch) stream into LDS through a
//     3-stage ring of direct-to-LDS loads shared by the waves; the two dot
//     products of every (vector, column) pair come from bf16/f16 MFMA with
//     fp32 accumulation. With exact 16-bit products the fp32 result r lies
//     within beta = 4 (D + 4) 2^-24 |a| |b| of the exact dot product for any
//     summation order and rounding (norms rounded up; the constant is taken
//     as 4.1 (D + 4) so the interval also holds the float64 sum of step 2),
//     and rounding is monotone, so
//       lo = rnd(rnd(rp - bp) + rnd(rn - bn)),  hi = rnd(rnd(rp + bp) + rnd(rn + bn))
//     bracket the pair's score. Each column keeps max lo and max hi over its
//     vectors. Norms outside [2^-40, 2^50] count as unbounded (bracket
//     [-inf, inf]), which keeps the MFMA clear of overflow and of flushed
//     subnormals.
//  2. Exact resolution: only a column whose bracket is open and whose hi
//     reaches the k-th largest lo can be selected without its exact score.
//     For those columns the brackets are recomputed per query vector on the
//     matrix cores: a closed bracket is that vector's score, and of the open
//     ones only those whose hi reaches the column's max lo can hold the
//     maximum; only those are recomputed in float64 (exact products, eight
//     lanes per score with a rounding bracket that falls back to the fixed
//     order d = 0..D-1 when it does not close). Other columns keep hi, which is then below at least k
//     exact scores. A row with no more columns than k needs exact values
//     only where a bracket end is not finite (the non-finite -> own rule).
//     fp32 operands, D = 32 and other block sizes skip step 1 and compute
//     every score in float64 (eight lanes per (column, query vector) with the
//     same rounding bracket from D = 64 on).
//  3. Top-k: an 8-bit radix select (2 passes for bf16 scores, 3 for fp16,
//     4 for fp32) finds the k-th largest key and how many of its ties are
//     taken; one wave writes the taken columns in
//     ascending block order with ballots.
#include <math.h>

#include "fbsa_common.h"
#include "fbsa_internal.h"
#include "fbsa_round.h"

namespace fbsa {

struct QmaxArgs {
  const void *a, *b1, *b2;
  const int32_t *cand;
  int32_t *sel;
  float *norms;  // key-side norms: b1 rows, then b2 rows (MFMA engine)
  int64_t B, H, nblk, la, ncand;
  int tok, keff, kk, conv, sink;
  int ncolp;  // LDS column capacity: nblk or ncand, rounded up to 8
};

// Orderable key of a score: larger scores give larger keys; -0 and +0 share
// one key (torch compares them equal, so the lower index wins their tie); any
// NaN becomes the positive quiet NaN, whose key is the largest (torch.topk
// ranks NaN first) and, like every grid value's, has zero low bits.
__device__ __forceinline__ uint32_t qm_key(float v) {
  if (v == 0.f) v = 0.f;
  if (v != v) v = __uint_as_float(0x7FC00000u);
  const uint32_t u = __float_as_uint(v);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float qm_key_value(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}
__device__ __forceinline__ bool qm_key_finite(uint32_t k) {
  const uint32_t u = (k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k;
  return (u & 0x7F800000u) != 0x7F800000u;
}

// Rounded-up Euclidean norm from an fp32 sum of exact squares, or +inf when
// outside [2^-40, 2^50] (no usable error bound); 0 only for a zero vector.
__device__ __forceinline__ float qm_norm(float ss, uint32_t nonzero) {
  if (!nonzero) return 0.f;
  if (!(ss >= 0x1p-80f) || !(ss <= 0x1p100f)) return INFINITY;
  return sqrtf(ss) * (1.0f + 0x1p-10f);
}

// Exact score of one (query vector, key block) pair: float64 FMA in the order
// d = 0..D-1 (16-bit and fp32 products are exact in float64).
template <typename T, int D> __device__ float qm_exact(const T *q, const T *k1, const T *k2) {
  double sp = 0.0, sn = 0.0;
#pragma unroll 1
  for (int d0 = 0; d0 < D; d0 += 8) {
    double v[8], x1[8], x2[8];
    load8<T>(q + d0, v);
    load8<T>(k1 + d0, x1);
    load8<T>(k2 + d0, x2);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      sp = __builtin_fma(v[e] > 0.0 ? v[e] : 0.0, x1[e], sp);
      sn = __builtin_fma(v[e] < 0.0 ? v[e] : 0.0, x2[e], sn);
    }
  }
  return round_dt_f<T>(round_dt<T>(sp) + round_dt<T>(sn));
}

// The same score with D split over the 8 lanes of a group (lane sub = 0..7
// takes d in [sub*D/8, (sub+1)*D/8)); every lane of the group returns it. The
// partial sums meet in another order than qm_exact's, so the result carries
// a bracket: any summation order of the D exact products lies within
// 2 (D - 1) 2^-53 sum|products| of the exact dot product (taken as
// 2.1 D 2^-53 to cover this sum's own rounding), so when the rounded bracket
// closes it equals qm_exact's value; otherwise (rare) qm_exact decides.
// FULL unrolls the loads (all in flight at once) where registers allow.
template <typename T, int D, bool FULL = false>
__device__ float qm_exact8(const T *q, const T *k1, const T *k2, int sub) {
  constexpr int PER = D / 8, UNROLL = FULL ? PER / 8 : 1;
  double sp = 0.0, sn = 0.0, ap = 0.0, an = 0.0;
#pragma unroll UNROLL
  for (int d0 = 0; d0 < PER; d0 += 8) {
    double v[8], x1[8], x2[8];
    load8<T>(q + sub * PER + d0, v);
    load8<T>(k1 + sub * PER + d0, x1);
    load8<T>(k2 + sub * PER + d0, x2);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const double pv = v[e] > 0.0 ? v[e] : 0.0, nv = v[e] < 0.0 ? v[e] : 0.0;
      sp = __builtin_fma(pv, x1[e], sp);
      sn = __builtin_fma(nv, x2[e], sn);
      ap = __builtin_fma(pv, __builtin_fabs(x1[e]), ap);
      an = __builtin_fma(-nv, __builtin_fabs(x2[e]), an);
    }
  }
#pragma unroll
  for (int m = 1; m < 8; m <<= 1) {
    sp += __shfl_xor(sp, m, 64);
    sn += __shfl_xor(sn, m, 64);
    ap += __shfl_xor(ap, m, 64);
    an += __shfl_xor(an, m, 64);
  }
  constexpr double C = 2.1 * D * 0x1p-53;
  const double ep = C * ap, en = C * an;
  const float lo = round_dt_f<T>(round_dt<T>(sp - ep) + round_dt<T>(sn - en));
  const float hi = round_dt_f<T>(round_dt<T>(sp + ep) + round_dt<T>(sn + en));
  if (lo == hi) return lo;
  return qm_exact<T, D>(q, k1, k2);
}

// Sum of squares step for 16-bit pairs packed in one word: s + x0^2 + x1^2
// (exact products; the sum's rounding is covered by the norm's 2^-10 margin).
template <typename T> __device__ __forceinline__ float qm_dot2(uint32_t w, float s) {
  if constexpr (__is_same(T, bf16)) {
    typedef __bf16 v2 __attribute__((ext_vector_type(2)));
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(v2, w), __builtin_bit_cast(v2, w), s, false);
  } else {
    typedef _Float16 v2 __attribute__((ext_vector_type(2)));
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(v2, w), __builtin_bit_cast(v2, w), s, false);
  }
}

// Round an fp32 value to the operand dtype (RNE) for the brackets; no NaN
// handling (a NaN bracket is caught by its caller), infinities stay.
template <typename T> __device__ __forceinline__ float qm_rnd(float f) {
  if constexpr (__is_same(T, bf16)) {
    uint32_t u = __float_as_uint(f);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return __uint_as_float(u & 0xFFFF0000u);
  } else {
    return round_dt_f<T>(f);
  }
}

// Bracket of one (vector, column) score from the fp32 MFMA sums rp, rn and
// their error bounds bp, bn: lo = rnd(rnd(rp - bp) + rnd(rn - bn)), hi =
// rnd(rnd(rp + bp) + rnd(rn + bn)). For bf16 the six roundings go through the
// packed hardware conversion (v_cvt_pk_bf16_f32: round to nearest even, equal
// to the integer rounding above for every non-NaN fp32 input).
template <typename T> __device__ __forceinline__ void qm_bracket(float rp, float rn, float bp, float bn, float &lo,
                                                                 float &hi) {
  if constexpr (__is_same(T, bf16)) {
    typedef __bf16 v2 __attribute__((ext_vector_type(2)));
    typedef float f2 __attribute__((ext_vector_type(2)));
    auto rnd2 = [](float x, float y, float &rx, float &ry) {
      const uint32_t u = __builtin_bit_cast(uint32_t, __builtin_convertvector((f2){x, y}, v2));
      rx = __uint_as_float(u << 16);
      ry = __uint_as_float(u & 0xFFFF0000u);
    };
    float lp, ln, hp, hn;
    rnd2(rp - bp, rn - bn, lp, ln);
    rnd2(rp + bp, rn + bn, hp, hn);
    rnd2(lp + ln, hp + hn, lo, hi);
  } else {
    lo = qm_rnd<T>(qm_rnd<T>(rp - bp) + qm_rnd<T>(rn - bn));
    hi = qm_rnd<T>(qm_rnd<T>(rp + bp) + qm_rnd<T>(rn + bn));
  }
}

// k-th largest of keys[0, n) (1 <= k <= n) by NP 8-bit radix passes from the
// top; *take receives how many keys equal to it are among the k largest.
// Keys of values on the dtype's grid vary only in their top 8*NP bits (bf16:
// 16, fp16: 19 of 24, fp32: all 32); the rest follow from the sign. Every
// thread of the workgroup (at least 256) calls it; hist holds 2 x 256 bins.
template <int NP>
__device__ uint32_t qm_radix_select(const uint32_t *keys, int n, int k, uint32_t *hist, int *sh, int *take) {
  const int tid = threadIdx.x;
  uint32_t prefix = 0, mask = 0;
  int rem = k;
  if (tid < 256) hist[tid] = 0;
  __syncthreads();
#pragma unroll
  for (int pass = 0; pass < NP; ++pass) {
    const int shift = 24 - 8 * pass;
    uint32_t *h = hist + 256 * (pass & 1);
    for (int c = tid; c < n; c += (int)blockDim.x) {
      const uint32_t key = keys[c];
      if ((key & mask) == prefix) atomicAdd(&h[(key >> shift) & 255u], 1u);
    }
    __syncthreads();
    if (tid < 64) {
      // lane l owns bins 4l..4l+3; find the largest bin b with
      // (keys in bins >= b) >= rem
      const int h0 = (int)h[4 * tid], h1 = (int)h[4 * tid + 1], h2 = (int)h[4 * tid + 2], h3 = (int)h[4 * tid + 3];
      const int tot = h0 + h1 + h2 + h3;
      int suf = tot;  // inclusive suffix sum over lanes >= l
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const int y = __shfl_down(suf, off, 64);
        if (tid + off < 64) suf += y;
      }
      const int above = suf - tot;
      if (above < rem && suf >= rem) {
        int acc = above, b;
        if (acc + h3 >= rem) b = 3;
        else {
          acc += h3;
          if (acc + h2 >= rem) b = 2;
          else {
            acc += h2;
            if (acc + h1 >= rem) b = 1;
            else { acc += h1; b = 0; }
          }
        }
        sh[pass & 1] = 4 * tid + b;
        sh[2 + (pass & 1)] = rem - acc;
      }
    }
    if (pass + 1 < NP && tid < 256) hist[256 * ((pass + 1) & 1) + tid] = 0;  // scanned two passes ago
    __syncthreads();
    prefix |= (uint32_t)sh[pass & 1] << shift;
    mask |= 0xFFu << shift;
    rem = sh[2 + (pass & 1)];
  }
  *take = rem;
  if constexpr (NP < 4) {
    const uint32_t low = (1u << (32 - 8 * NP)) - 1u;
    prefix |= (prefix & 0x80000000u) ? 0u : low;  // grid values: 0 bits below a positive key, 1 bits below a negative one
  }
  return prefix;
}

template <typename T> constexpr int qm_passes() { return sizeof(T) == 4 ? 4 : __is_same(T, bf16) ? 2 : 3; }

// Ring of key-block tiles for the bracket pass: 16 rows of b1 and 16 of b2
// (16-byte chunks XOR-swizzled per row so the 16 rows x 1 chunk an MFMA B
// operand reads fall on distinct banks) plus each wave's copy of their 32
// norms.
template <int D> struct QmCfg {
  static constexpr int CPR = D / 8;
  static constexpr int TILE_BYTES = 2 * 16 * D * 2;
  static constexpr int NORM_BYTES = 4 * 256;  // per wave: lanes 0-15 b1, 16-31 b2 (lanes 32-63 unused)
  static constexpr int STAGE_BYTES = TILE_BYTES + NORM_BYTES;
  static constexpr int LPW = TILE_BYTES / 16 / 256;  // 16-byte loads per thread per tile
  static constexpr int NSTAGE = 3;
};

// Dynamic LDS: s_lo, s_hi (u32) and s_col, s_cl (u16), ncolp entries each,
// then the tile ring (bracket pass only).
template <int D, int TOK> static size_t qm_lds_bytes(int64_t ncolp) {
  return (size_t)ncolp * 12 + (TOK > 0 ? (size_t)QmCfg<D>::NSTAGE * QmCfg<D>::STAGE_BYTES : 0);
}

// TOK = 64 / 128: MFMA brackets (16-bit T), each of the four waves holds
// TOK/64 tiles of 16 query vectors; TOK = 0: every column exact (a.tok query
// vectors per block).
template <typename T, int D, int TOK>
__global__ __launch_bounds__(256, 2) void qmax_kernel(QmaxArgs a) {
  constexpr int NT = 256;
  extern __shared__ __align__(16) char qm_lds[];
  uint32_t *s_lo = (uint32_t *)qm_lds;
  uint32_t *s_hi = s_lo + a.ncolp;
  uint16_t *s_col = (uint16_t *)(s_hi + a.ncolp);
  uint16_t *s_cl = s_col + a.ncolp;
  __shared__ uint32_t s_hist[512];
  __shared__ int s_sh[12];  // [2] candidate count, [3] contenders, [4] worklist, [8..11] radix select

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int64_t BH = a.B * a.H;
  const int64_t bh = (int64_t)blockIdx.x % BH;
  const int i = (int)(a.nblk - 1 - (int64_t)blockIdx.x / BH);
  const T *Ab = (const T *)a.a + bh * a.la * D;
  const T *B1 = (const T *)a.b1 + bh * a.nblk * D;
  const T *B2 = (const T *)a.b2 + bh * a.nblk * D;
  int32_t *out = a.sel + (bh * a.nblk + i) * (int64_t)a.kk;
  const int tok = TOK ? TOK : a.tok;
  const int keff = a.keff;
  const int s0 = (a.conv == FBSA_SEL_SORTED_SINK && a.sink) ? 1 : 0;
  const uint64_t lt_mask = (1ull << lane) - 1ull;

  // ---- columns: 0..i, or row i's candidates (ascending; repeats and entries
  // outside [0, i] dropped)
  int count;
  if (a.cand) {
    if (w == 0) {
      const int32_t *cr = a.cand + (bh * a.nblk + i) * a.ncand;
      int n = 0, prev = -1;
      for (int c0 = 0; c0 < (int)a.ncand; c0 += 64) {
        const int c = c0 + lane;
        const int j = c < (int)a.ncand ? cr[c] : -1;
        int pj = __shfl_up(j, 1, 64);
        if (lane == 0) pj = prev;
        const bool keep = c < (int)a.ncand && j >= 0 && j <= i && j != pj;
        const uint64_t m = __ballot(keep);
        if (keep) s_col[n + __popcll(m & lt_mask)] = (uint16_t)j;
        n += __popcll(m);
        prev = __shfl(j, 63, 64);
      }
      if (lane == 0) s_sh[2] = n;
    }
    __syncthreads();
    count = s_sh[2];
  } else {
    count = i + 1;
  }
  auto col_block = [&](int c) -> int { return a.cand ? (int)s_col[c] : c; };

  if (keff > 0) {
    for (int c = tid; c < count; c += NT) { s_lo[c] = 0u; s_hi[c] = 0u; }
    __syncthreads();

    // ---- 1. brackets on the matrix cores
    int nres = count;  // columns resolved exactly (TOK = 0: all of them)
    uint32_t *fin = s_lo;
    if constexpr (TOK > 0) {
      using C = QmCfg<D>;
      constexpr int KS = D / 32, RW = TOK / 64;
      constexpr float CB = 4.1f * (float)(D + 4) * 0x1p-24f;
      const int p = lane & 15, g = lane >> 4;
      char *ring = (char *)(s_cl + a.ncolp);
      const float *N1 = a.norms + bh * a.nblk, *N2 = a.norms + (BH + bh) * a.nblk;
      const int ntiles = (count + 15) / 16;

      // tile tc -> ring stage tc % NSTAGE: wave-load v = l*4 + w carries
      // chunks [64v, 64v + 64) of the tile (b1 rows, then b2 rows)
      auto issue = [&](int tc) {
        char *stg = ring + (tc % C::NSTAGE) * C::STAGE_BYTES;
        const int c0 = tc * 16;
#pragma unroll
        for (int l = 0; l < C::LPW; ++l) {
          const int q = (l * 4 + w) * 64 + lane;
          const int m = q / (16 * C::CPR), r = (q / C::CPR) % 16, cp = q % C::CPR;
          const int cc = c0 + r;
          const int j = col_block(cc < count ? cc : count - 1);
          g2lds16((m ? B2 : B1) + (int64_t)j * D + 8 * (cp ^ swz(r, C::CPR)), stg + (l * 4 + w) * 1024);
        }
        const int cc = c0 + (lane & 15);
        const int j = col_block(cc < count ? cc : count - 1);
        g2lds4(((lane & 16) ? N2 : N1) + j, stg + C::TILE_BYTES + w * 256);
      };
#pragma unroll
      for (int tc = 0; tc < C::NSTAGE - 1; ++tc)
        if (tc < ntiles) issue(tc);

      // query vectors: split into positive and negative parts, with norms
      s16x8 ap[RW][KS], an[RW][KS];
      float cbp[RW][4], cbn[RW][4];
#pragma unroll
      for (int x = 0; x < RW; ++x) {
        // branch-free loads (a row past la is read clamped and zeroed), all in flight together
        const int64_t t = (int64_t)i * TOK + (w * RW + x) * 16 + p;
        const bool tv = t < a.la;
        const T *row = Ab + (tv ? t : a.la - 1) * D + g * 8;
        u32x4 raw[KS];
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) raw[ks] = *(const u32x4 *)(row + ks * 32);
        float sp = 0.f, sn = 0.f;
        uint32_t zp = 0u, zn = 0u;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          u32x4 vp, vn;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const uint32_t v = tv ? raw[ks][e] : 0u;
            const uint32_t m = ((v >> 15) & 0x00010001u) * 0xFFFFu;  // per-half sign masks
            vn[e] = v & m;
            vp[e] = v & ~m;
            sp = qm_dot2<T>(vp[e], sp);
            sn = qm_dot2<T>(vn[e], sn);
            zp |= vp[e] & 0x7FFF7FFFu;
            zn |= vn[e] & 0x7FFF7FFFu;
          }
          ap[x][ks] = __builtin_bit_cast(s16x8, vp);
          an[x][ks] = __builtin_bit_cast(s16x8, vn);
        }
        sp += __shfl_xor(sp, 16, 64);
        sp += __shfl_xor(sp, 32, 64);
        sn += __shfl_xor(sn, 16, 64);
        sn += __shfl_xor(sn, 32, 64);
        zp |= (uint32_t)__shfl_xor((int)zp, 16, 64);
        zp |= (uint32_t)__shfl_xor((int)zp, 32, 64);
        zn |= (uint32_t)__shfl_xor((int)zn, 16, 64);
        zn |= (uint32_t)__shfl_xor((int)zn, 32, 64);
        const float np = qm_norm(sp, zp), nn = qm_norm(sn, zn);
        // result rows of this lane are vectors 4g + r of the tile
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          cbp[x][r] = CB * __shfl(np, 4 * g + r, 64);
          cbn[x][r] = CB * __shfl(nn, 4 * g + r, 64);
        }
      }
      wait_vmcnt<0>();  // the query rows (and the first ring stages)

      for (int tc = 0; tc < ntiles; ++tc) {
        // tile tc has landed once at most min(ahead, NSTAGE-2) later tiles are in flight
        const int ahead = ntiles - 1 - tc;
        wait_ring<C::LPW + 1>(ahead < C::NSTAGE - 2 ? ahead : C::NSTAGE - 2);
        // one barrier per tile: every wave has landed its part of tile tc and
        // finished reading tile tc-1, whose stage the prefetch overwrites
        lds_barrier();
        if (tc + C::NSTAGE - 1 < ntiles) issue(tc + C::NSTAGE - 1);
        const char *stg = ring + (tc % C::NSTAGE) * C::STAGE_BYTES;
        const float nb1 = *(const float *)(stg + C::TILE_BYTES + w * 256 + 4 * p);
        const float nb2 = *(const float *)(stg + C::TILE_BYTES + w * 256 + 64 + 4 * p);

        f32x4 acp[RW], acn[RW];
#pragma unroll
        for (int x = 0; x < RW; ++x) {
          acp[x] = (f32x4){0.f, 0.f, 0.f, 0.f};
          acn[x] = (f32x4){0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          const int cpos = (4 * ks + g) ^ swz(p, C::CPR);
          const s16x8 bx = *(const s16x8 *)(stg + (p * C::CPR + cpos) * 16);
          const s16x8 bm = *(const s16x8 *)(stg + ((16 + p) * C::CPR + cpos) * 16);
#pragma unroll
          for (int x = 0; x < RW; ++x) {
            acp[x] = Mfma16<T>::run(ap[x][ks], bx, acp[x]);
            acn[x] = Mfma16<T>::run(an[x][ks], bm, acn[x]);
          }
        }

        float mlo = -INFINITY, mhi = -INFINITY;
#pragma unroll
        for (int x = 0; x < RW; ++x)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            // 0 * inf (a zero vector against an unbounded one) is an exact 0 product: bound 0
            const float bp = fmaxf(cbp[x][r] * nb1, 0.f), bn = fmaxf(cbn[x][r] * nb2, 0.f);
            float lo, hi;
            qm_bracket<T>(acp[x][r], acn[x][r], bp, bn, lo, hi);
            // unbounded, or inf - inf after an fp16 overflow: the exact path decides
            const bool open = bp == INFINITY || bn == INFINITY || !(lo <= hi);
            lo = open ? -INFINITY : lo;
            hi = open ? INFINITY : hi;
            mlo = fmaxf(mlo, lo);
            mhi = fmaxf(mhi, hi);
          }
        mlo = fmaxf(mlo, __shfl_xor(mlo, 16, 64));
        mlo = fmaxf(mlo, __shfl_xor(mlo, 32, 64));
        mhi = fmaxf(mhi, __shfl_xor(mhi, 16, 64));
        mhi = fmaxf(mhi, __shfl_xor(mhi, 32, 64));
        const int cc = tc * 16 + p;
        if (g == 0 && cc < count) {
          atomicMax(&s_lo[cc], qm_key(mlo));
          atomicMax(&s_hi[cc], qm_key(mhi));
        }
      }
      __syncthreads();

      // ---- contenders: columns that may be selected without an exact score
      uint32_t tau = 0u;
      if (count > keff) {
        int dummy;
        tau = qm_radix_select<qm_passes<T>()>(s_lo, count, keff, s_hist, s_sh + 8, &dummy);
      }
      if (tid == 0) s_sh[3] = 0;
      __syncthreads();
      for (int c = tid; c < count; c += NT) {
        const uint32_t lo = s_lo[c], hi = s_hi[c];
        const bool need = count > keff ? (lo != hi && hi >= tau) : !(qm_key_finite(lo) && qm_key_finite(hi));
        if (need) {
          const int n = atomicAdd(&s_sh[3], 1);
          s_cl[n] = (uint16_t)c;
          s_hi[c] = 0u;  // rebuilt below as the exact column maximum
        }
      }
      __syncthreads();
      nres = s_sh[3];
      fin = s_hi;

      // ---- 2. exact maxima of the contenders, 16 at a time: the brackets are
      // recomputed per query vector on the matrix cores; a closed bracket is
      // the vector's score, and of the open ones only those whose hi reaches
      // the column's max lo can hold the maximum (the vector behind max lo
      // among them), so only those go to float64 (a worklist in the free ring)
      uint32_t *work = (uint32_t *)ring;  // (slot << 8 | vector), at most 16 * TOK per tile
      for (int t0 = 0; t0 < nres; t0 += 16) {
        if (tid == 0) s_sh[4] = 0;
        const bool live = t0 + p < nres;
        const int c = s_cl[live ? t0 + p : nres - 1];
        const int j = col_block(c);
        const T *r1 = B1 + (int64_t)j * D + g * 8, *r2 = B2 + (int64_t)j * D + g * 8;
        const float nb1 = N1[j], nb2 = N2[j];
        const float mlo_c = qm_key_value(s_lo[c]);
        f32x4 acp[RW], acn[RW];
#pragma unroll
        for (int x = 0; x < RW; ++x) {
          acp[x] = (f32x4){0.f, 0.f, 0.f, 0.f};
          acn[x] = (f32x4){0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          const s16x8 bx = *(const s16x8 *)(r1 + ks * 32), bm = *(const s16x8 *)(r2 + ks * 32);
#pragma unroll
          for (int x = 0; x < RW; ++x) {
            acp[x] = Mfma16<T>::run(ap[x][ks], bx, acp[x]);
            acn[x] = Mfma16<T>::run(an[x][ks], bm, acn[x]);
          }
        }
        __syncthreads();  // s_sh[4] cleared; the previous worklist is consumed
        float cmax = -INFINITY;
#pragma unroll
        for (int x = 0; x < RW; ++x)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float bp = fmaxf(cbp[x][r] * nb1, 0.f), bn = fmaxf(cbn[x][r] * nb2, 0.f);
            float lo, hi;
            qm_bracket<T>(acp[x][r], acn[x][r], bp, bn, lo, hi);
            const bool open = bp == INFINITY || bn == INFINITY || !(lo == hi);
            if (!open) cmax = fmaxf(cmax, lo);
            else if (live && !(hi < mlo_c)) {
              const int slot = atomicAdd(&s_sh[4], 1);
              work[slot] = ((uint32_t)p << 8) | (uint32_t)((w * RW + x) * 16 + 4 * g + r);
            }
          }
        cmax = fmaxf(cmax, __shfl_xor(cmax, 16, 64));
        cmax = fmaxf(cmax, __shfl_xor(cmax, 32, 64));
        if (g == 0 && live) atomicMax(&s_hi[c], qm_key(cmax));
        __syncthreads();
        const int nw = s_sh[4];
        for (int it = tid >> 3; it < nw; it += NT / 8) {  // 8 lanes per item
          const uint32_t e = work[it];
          const int c2 = s_cl[t0 + (int)(e >> 8)];
          const int j2 = col_block(c2);
          const int64_t tr = (int64_t)i * TOK + (e & 255u);
          const float v = tr < a.la ? qm_exact8<T, D>(Ab + tr * D, B1 + (int64_t)j2 * D, B2 + (int64_t)j2 * D, tid & 7)
                                    : 0.f;
          if ((tid & 7) == 0) atomicMax(&s_hi[c2], qm_key(v));
        }
        __syncthreads();
      }
    } else {
      // ---- 2. exact scores of every column (eight lanes per (column, query
      // vector) from D = 64 on, one thread below)
      const int64_t items = (int64_t)nres * tok;
      constexpr int LPI = D >= 64 ? 8 : 1;
      for (int64_t it = tid / LPI; it < items; it += NT / LPI) {
        const int c = (int)(it / tok), t = (int)(it % tok);
        const int j = col_block(c);
        const int64_t tr = (int64_t)i * tok + t;
        float v = 0.f;
        if (tr < a.la) {
          if constexpr (D >= 64)
            v = qm_exact8<T, D, true>(Ab + tr * D, B1 + (int64_t)j * D, B2 + (int64_t)j * D, tid & 7);
          else
            v = qm_exact<T, D>(Ab + tr * D, B1 + (int64_t)j * D, B2 + (int64_t)j * D);
        }
        if (tid % LPI == 0) atomicMax(&s_lo[c], qm_key(v));
      }
      __syncthreads();
    }

    // ---- 3. top-k and output
    const bool all = count <= keff;
    uint32_t tau2 = 0u;
    int take_eq = 0;
    if (!all) tau2 = qm_radix_select<qm_passes<T>()>(fin, count, keff, s_hist, s_sh + 8, &take_eq);
    if (w == 0) {
      int nfin = 0, eqseen = 0;
      for (int c0 = 0; c0 < count; c0 += 64) {
        const int c = c0 + lane;
        const uint32_t key = c < count ? fin[c] : 0u;
        bool take;
        if (all) {
          take = c < count;
        } else {
          const bool gt = c < count && key > tau2, eq = c < count && key == tau2;
          const uint64_t em = __ballot(eq);
          take = gt || (eq && eqseen + __popcll(em & lt_mask) < take_eq);
          eqseen += __popcll(em);
        }
        const bool ok = take && qm_key_finite(key);
        const uint64_t fm = __ballot(ok);
        if (ok) out[s0 + nfin + __popcll(fm & lt_mask)] = col_block(c);
        nfin += __popcll(fm);
      }
      for (int x = nfin + lane; x < keff; x += 64) out[s0 + x] = i;  // non-finite picks and -inf fills
    }
  }
  if (tid == 0) {
    if (s0) out[0] = 0;
    if (a.conv == FBSA_SEL_SORTED_SINK) out[s0 + keff] = i;
  }
}

// Key-side norms for the MFMA engine: one thread per key block row of b1 and
// of b2, the same rounded-up bound the query side uses.
template <typename T, int D>
__global__ __launch_bounds__(256) void qm_norms_kernel(QmaxArgs a) {
  const int64_t n = a.B * a.H * a.nblk;
  const int64_t r = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (r >= 2 * n) return;
  const T *row = (const T *)(r < n ? a.b1 : a.b2) + (r < n ? r : r - n) * D;
  float ss = 0.f;
  uint32_t z = 0u;
#pragma unroll 4
  for (int d0 = 0; d0 < D; d0 += 8) {
    const u32x4 w = *(const u32x4 *)(row + d0);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      ss = qm_dot2<T>(w[e], ss);
      z |= w[e] & 0x7FFF7FFFu;
    }
  }
  a.norms[r] = qm_norm(ss, z);
}

template <typename T, int D, int TOK> static int launch_qmax_k(const QmaxArgs &a, hipStream_t s) {
  const size_t lds = qm_lds_bytes<D, TOK>(a.ncolp);
  {
    const int e = lds_optin((const void *)qmax_kernel<T, D, TOK>, lds, "hipFuncSetAttribute(qmax)");
    if (e) return e;
  }
  hipLaunchKernelGGL((qmax_kernel<T, D, TOK>), dim3((unsigned)(a.B * a.H * a.nblk)), dim3(256), lds, s, a);
  return FBSA_OK;
}

template <typename T, int D> static int launch_qmax_d(const QmaxArgs &a, bool exact, hipStream_t s) {
  if constexpr (sizeof(T) == 2 && D >= 64) {
    if (!exact && (a.tok == 64 || a.tok == 128)) {
      const int64_t nrow = 2 * a.B * a.H * a.nblk;
      hipLaunchKernelGGL((qm_norms_kernel<T, D>), dim3((unsigned)((nrow + 255) / 256)), dim3(256), 0, s, a);
      return a.tok == 64 ? launch_qmax_k<T, D, 64>(a, s) : launch_qmax_k<T, D, 128>(a, s);
    }
  }
  return launch_qmax_k<T, D, 0>(a, s);
}

template <typename T> static int launch_qmax(const QmaxArgs &a, int64_t D, bool exact, hipStream_t s) {
  int e = FBSA_OK;
  switch (D) {
    case 32: e = launch_qmax_d<T, 32>(a, exact, s); break;
    case 64: e = launch_qmax_d<T, 64>(a, exact, s); break;
    case 128: e = launch_qmax_d<T, 128>(a, exact, s); break;
    case 256: e = launch_qmax_d<T, 256>(a, exact, s); break;
    default: return fail(FBSA_EUNSUPPORTED, "fbsa_select_qmax: operand dim %lld not in {32,64,128,256}", (long long)D);
  }
  if (e) return e;
  return hip_check(hipGetLastError(), "qmax_kernel launch");
}

size_t select_qmax_workspace_bytes(const fbsa_qmax_desc *d) {
  const bool mfma = d->dtype != FBSA_F32 && (d->tok == 64 || d->tok == 128) && d->D >= 64 &&
                    !(d->flags & FBSA_QMAX_EXACT);
  return mfma ? (size_t)(2 * d->B * d->H * d->nblk) * sizeof(float) : 0;
}

int run_select_qmax(const fbsa_qmax_desc *d, const void *a, const void *b1, const void *b2, const int32_t *cand,
                    int32_t *sel, void *ws, hipStream_t s) {
  QmaxArgs q;
  q.a = a; q.b1 = b1; q.b2 = b2; q.cand = cand; q.sel = sel; q.norms = (float *)ws;
  q.B = d->B; q.H = d->H; q.nblk = d->nblk; q.la = d->la; q.ncand = cand ? d->ncand : 0;
  q.ncolp = (int)(((cand ? d->ncand : d->nblk) + 7) & ~7LL);
  q.tok = (int)d->tok;
  q.keff = (int)(d->topk < d->nblk ? d->topk : d->nblk);
  q.kk = (int)d->kk;
  q.conv = d->convention;
  q.sink = d->sink;
  const bool exact = (d->flags & FBSA_QMAX_EXACT) != 0 || ws == nullptr;
  switch (d->dtype) {
    case FBSA_BF16: return launch_qmax<bf16>(q, d->D, exact, s);
    case FBSA_F16: return launch_qmax<f16>(q, d->D, exact, s);
    default: return launch_qmax<float>(q, d->D, exact, s);
  }
}

}  // namespace fbsa
