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
// One workgroup per (b, h, query block i), larger i first (the rows with the
// most columns start early). Two 32-bit orderable keys per column live in
// LDS.
//  1. Brackets (16-bit operands, 64 or 128 query vectors per block, D in
//     {32, 64, 128, 256}): each of the four waves holds tok/64 tiles of 16
//     query vectors, split into their positive and negative parts, as MFMA A
//     operands for the whole row. For each tile of 16 columns the key max/min
//     rows go straight from global memory (L2) into B operands and the two
//     dot products of every (vector, column) pair come from bf16/f16 MFMA
//     with fp32 accumulation. With exact 16-bit products the fp32 result r
//     lies within beta = 4 (D + 4) 2^-24 |a| |b| of the exact dot product for
//     any summation order and rounding (norms rounded up; the constant is
//     taken as 4.1 (D + 4) so the interval also holds the float64 sum of
//     step 2), and rounding is monotone, so
//       lo = rnd(rnd(rp - bp) + rnd(rn - bn)),  hi = rnd(rnd(rp + bp) + rnd(rn + bn))
//     bracket the pair's score. Each column keeps max lo and max hi over its
//     vectors. Norms outside [2^-40, 2^50] count as unbounded (bracket
//     [-inf, inf]), which keeps the MFMA clear of overflow and of flushed
//     subnormals.
//  2. Exact resolution: only a column whose bracket is open and whose hi
//     reaches the k-th largest lo can be selected without its exact score;
//     those columns are recomputed in float64 (fixed order d = 0..D-1, one
//     thread per (column, query vector), exact products) and the others
//     keep hi, which is then below at least k exact scores. A row with no
//     more columns than k needs exact values only where a bracket end is not
//     finite (the non-finite -> own rule). fp32 operands and other block
//     sizes skip step 1 and resolve every column.
//  3. Top-k: a 4-pass 8-bit radix select finds the k-th largest key and how
//     many of its ties are taken; one wave writes the taken columns in
//     ascending block order with ballots.
#include <math.h>

#include "fbsa_common.h"
#include "fbsa_internal.h"
#include "fbsa_round.h"

namespace fbsa {

constexpr int QM_MAXCOL = 4096;  // columns per row held in LDS

struct QmaxArgs {
  const void *a, *b1, *b2;
  const int32_t *cand;
  int32_t *sel;
  int64_t B, H, nblk, la, ncand;
  int tok, keff, kk, conv, sink;
};

// Orderable key of a score: larger scores give larger keys; -0 and +0 share
// one key (torch compares them equal, so the lower index wins their tie).
__device__ __forceinline__ uint32_t qm_key(float v) {
  if (v == 0.f) v = 0.f;
  const uint32_t u = __float_as_uint(v);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
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
#pragma unroll 2
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

// k-th largest of keys[0, n) (1 <= k <= n) by four 8-bit radix passes; *take
// receives how many keys equal to it are among the k largest. All 256
// threads call it.
__device__ uint32_t qm_radix_select(const uint32_t *keys, int n, int k, uint32_t *hist, int *sh, int *take) {
  const int tid = threadIdx.x;
  uint32_t prefix = 0, mask = 0;
  int rem = k;
  for (int shift = 24; shift >= 0; shift -= 8) {
    hist[tid] = 0;
    __syncthreads();
    for (int c = tid; c < n; c += 256) {
      const uint32_t key = keys[c];
      if ((key & mask) == prefix) atomicAdd(&hist[(key >> shift) & 255u], 1u);
    }
    __syncthreads();
    if (tid < 64) {
      // lane l owns bins 4l..4l+3; find the largest bin b with
      // (keys in bins >= b) >= rem
      const int h0 = (int)hist[4 * tid], h1 = (int)hist[4 * tid + 1], h2 = (int)hist[4 * tid + 2],
                h3 = (int)hist[4 * tid + 3];
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
        sh[0] = 4 * tid + b;
        sh[1] = rem - acc;
      }
    }
    __syncthreads();
    prefix |= (uint32_t)sh[0] << shift;
    mask |= 0xFFu << shift;
    rem = sh[1];
  }
  *take = rem;
  return prefix;
}

// TOK = 64 / 128: MFMA brackets (16-bit T); TOK = 0: every column exact
// (a.tok query vectors per block).
template <typename T, int D, int TOK>
__global__ __launch_bounds__(256) void qmax_kernel(QmaxArgs a) {
  __shared__ uint32_t s_lo[QM_MAXCOL], s_hi[QM_MAXCOL];
  __shared__ uint16_t s_col[QM_MAXCOL], s_cl[QM_MAXCOL];
  __shared__ uint32_t s_hist[256];
  __shared__ int s_sh[4];

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
    for (int c = tid; c < count; c += 256) { s_lo[c] = 0u; s_hi[c] = 0u; }
    __syncthreads();

    // ---- 1. brackets on the matrix cores
    int nres = count;  // columns resolved exactly (TOK = 0: all of them)
    uint32_t *fin = s_lo;
    if constexpr (TOK > 0) {
      constexpr int KS = D / 32, RW = TOK / 64;
      constexpr float CB = 4.1f * (float)(D + 4) * 0x1p-24f;
      const int p = lane & 15, g = lane >> 4;
      s16x8 ap[RW][KS], an[RW][KS];
      float cbp[RW][4], cbn[RW][4];
#pragma unroll
      for (int x = 0; x < RW; ++x) {
        const int64_t t = (int64_t)i * TOK + (w * RW + x) * 16 + p;
        float sp = 0.f, sn = 0.f;
        uint32_t zp = 0u, zn = 0u;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          s16x8 v = {0, 0, 0, 0, 0, 0, 0, 0};
          if (t < a.la) v = *(const s16x8 *)(Ab + t * D + ks * 32 + g * 8);
          s16x8 vp, vn;
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const bool neg = v[e] < 0;  // sign bit of the 16-bit pattern
            vp[e] = neg ? (short)0 : v[e];
            vn[e] = neg ? v[e] : (short)0;
            const float f = half_bits_to_f32<T>((uint32_t)(uint16_t)v[e]);
            const uint32_t mag = (uint32_t)(uint16_t)v[e] & 0x7FFFu;
            if (neg) { sn = __builtin_fmaf(f, f, sn); zn |= mag; }
            else { sp = __builtin_fmaf(f, f, sp); zp |= mag; }
          }
          ap[x][ks] = vp;
          an[x][ks] = vn;
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

      auto load_b = [&](int c0, s16x8 *bx, s16x8 *bm) {
        const int cc = c0 + p;
        const int j = col_block(cc < count ? cc : count - 1);
        const T *r1 = B1 + (int64_t)j * D + g * 8;
        const T *r2 = B2 + (int64_t)j * D + g * 8;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          bx[ks] = *(const s16x8 *)(r1 + ks * 32);
          bm[ks] = *(const s16x8 *)(r2 + ks * 32);
        }
      };
      s16x8 bx[KS], bm[KS];
      if (count > 0) load_b(0, bx, bm);  // a candidate row may list no valid block
      for (int c0 = 0; c0 < count; c0 += 16) {
        // key-side norms (the 4 lanes of a column hold a quarter of each row)
        float s1 = 0.f, s2 = 0.f;
        uint32_t z1 = 0u, z2 = 0u;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float f1 = half_bits_to_f32<T>((uint32_t)(uint16_t)bx[ks][e]);
            const float f2 = half_bits_to_f32<T>((uint32_t)(uint16_t)bm[ks][e]);
            s1 = __builtin_fmaf(f1, f1, s1);
            s2 = __builtin_fmaf(f2, f2, s2);
            z1 |= (uint32_t)(uint16_t)bx[ks][e] & 0x7FFFu;
            z2 |= (uint32_t)(uint16_t)bm[ks][e] & 0x7FFFu;
          }
        s1 += __shfl_xor(s1, 16, 64);
        s1 += __shfl_xor(s1, 32, 64);
        s2 += __shfl_xor(s2, 16, 64);
        s2 += __shfl_xor(s2, 32, 64);
        z1 |= (uint32_t)__shfl_xor((int)z1, 16, 64);
        z1 |= (uint32_t)__shfl_xor((int)z1, 32, 64);
        z2 |= (uint32_t)__shfl_xor((int)z2, 16, 64);
        z2 |= (uint32_t)__shfl_xor((int)z2, 32, 64);
        const float nb1 = qm_norm(s1, z1), nb2 = qm_norm(s2, z2);

        f32x4 acp[RW], acn[RW];
#pragma unroll
        for (int x = 0; x < RW; ++x) {
          acp[x] = (f32x4){0.f, 0.f, 0.f, 0.f};
          acn[x] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int ks = 0; ks < KS; ++ks) {
            acp[x] = Mfma16<T>::run(ap[x][ks], bx[ks], acp[x]);
            acn[x] = Mfma16<T>::run(an[x][ks], bm[ks], acn[x]);
          }
        }
        // the next tile's loads overlap this tile's bracket arithmetic
        if (c0 + 16 < count) load_b(c0 + 16, bx, bm);

        float mlo = -INFINITY, mhi = -INFINITY;
#pragma unroll
        for (int x = 0; x < RW; ++x)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            float bp = cbp[x][r] * nb1, bn = cbn[x][r] * nb2;
            if (bp != bp) bp = 0.f;  // 0 * inf: one side is a zero vector, its product is exact
            if (bn != bn) bn = 0.f;
            float lo, hi;
            if (bp == INFINITY || bn == INFINITY) {
              lo = -INFINITY;
              hi = INFINITY;
            } else {
              const float rp = acp[x][r], rn = acn[x][r];
              lo = round_dt_f<T>(round_dt_f<T>(rp - bp) + round_dt_f<T>(rn - bn));
              hi = round_dt_f<T>(round_dt_f<T>(rp + bp) + round_dt_f<T>(rn + bn));
            }
            mlo = fmaxf(mlo, lo);
            mhi = fmaxf(mhi, hi);
          }
        mlo = fmaxf(mlo, __shfl_xor(mlo, 16, 64));
        mlo = fmaxf(mlo, __shfl_xor(mlo, 32, 64));
        mhi = fmaxf(mhi, __shfl_xor(mhi, 16, 64));
        mhi = fmaxf(mhi, __shfl_xor(mhi, 32, 64));
        const int cc = c0 + p;
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
        tau = qm_radix_select(s_lo, count, keff, s_hist, s_sh, &dummy);
      }
      if (tid == 0) s_sh[3] = 0;
      __syncthreads();
      for (int c = tid; c < count; c += 256) {
        const uint32_t lo = s_lo[c], hi = s_hi[c];
        const bool need = count > keff ? (lo != hi && hi >= tau) : !(qm_key_finite(lo) && qm_key_finite(hi));
        if (need) {
          const int n = atomicAdd(&s_sh[3], 1);
          s_cl[n] = (uint16_t)c;
          s_lo[c] = 0u;
        }
      }
      __syncthreads();
      nres = s_sh[3];
      fin = s_hi;
    }

    // ---- 2. exact scores (one thread per (column, query vector))
    const int64_t items = (int64_t)nres * tok;
    for (int64_t it = tid; it < items; it += 256) {
      const int n = (int)(it / tok), t = (int)(it % tok);
      const int c = TOK > 0 ? (int)s_cl[n] : n;
      const int j = col_block(c);
      const int64_t tr = (int64_t)i * tok + t;
      const float v = tr < a.la ? qm_exact<T, D>(Ab + tr * D, B1 + (int64_t)j * D, B2 + (int64_t)j * D) : 0.f;
      atomicMax(&s_lo[c], qm_key(v));
    }
    __syncthreads();
    if constexpr (TOK > 0) {
      for (int n = tid; n < nres; n += 256) {
        const int c = s_cl[n];
        s_hi[c] = s_lo[c];
      }
      __syncthreads();
    }

    // ---- 3. top-k and output
    const bool all = count <= keff;
    uint32_t tau2 = 0u;
    int take_eq = 0;
    if (!all) tau2 = qm_radix_select(fin, count, keff, s_hist, s_sh, &take_eq);
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

template <typename T, int D> static void launch_qmax_d(const QmaxArgs &a, bool exact, hipStream_t s) {
  const dim3 grid((unsigned)(a.B * a.H * a.nblk)), block(256);
  if constexpr (sizeof(T) == 2) {
    if (!exact && a.tok == 64) { hipLaunchKernelGGL((qmax_kernel<T, D, 64>), grid, block, 0, s, a); return; }
    if (!exact && a.tok == 128) { hipLaunchKernelGGL((qmax_kernel<T, D, 128>), grid, block, 0, s, a); return; }
  }
  hipLaunchKernelGGL((qmax_kernel<T, D, 0>), grid, block, 0, s, a);
}

template <typename T> static int launch_qmax(const QmaxArgs &a, int64_t D, bool exact, hipStream_t s) {
  switch (D) {
    case 32: launch_qmax_d<T, 32>(a, exact, s); break;
    case 64: launch_qmax_d<T, 64>(a, exact, s); break;
    case 128: launch_qmax_d<T, 128>(a, exact, s); break;
    case 256: launch_qmax_d<T, 256>(a, exact, s); break;
    default: return fail(FBSA_EUNSUPPORTED, "fbsa_select_qmax: operand dim %lld not in {32,64,128,256}", (long long)D);
  }
  return hip_check(hipGetLastError(), "qmax_kernel launch");
}

int run_select_qmax(const fbsa_qmax_desc *d, const void *a, const void *b1, const void *b2, const int32_t *cand,
                    int32_t *sel, hipStream_t s) {
  QmaxArgs q;
  q.a = a; q.b1 = b1; q.b2 = b2; q.cand = cand; q.sel = sel;
  q.B = d->B; q.H = d->H; q.nblk = d->nblk; q.la = d->la; q.ncand = cand ? d->ncand : 0;
  q.tok = (int)d->tok;
  q.keff = (int)(d->topk < d->nblk ? d->topk : d->nblk);
  q.kk = (int)d->kk;
  q.conv = d->convention;
  q.sink = d->sink;
  const bool exact = (d->flags & FBSA_QMAX_EXACT) != 0;
  switch (d->dtype) {
    case FBSA_BF16: return launch_qmax<bf16>(q, d->D, exact, s);
    case FBSA_F16: return launch_qmax<f16>(q, d->D, exact, s);
    default: return launch_qmax<float>(q, d->D, exact, s);
  }
}

}  // namespace fbsa
