// Backward of the fused block-sparse attention for gfx950 (CDNA4).
//
// Four stages, none of them with floating-point atomics (results are bitwise
// repeatable):
//   1. prep_kernel     per query row: delta = sum_d dO*O and lse*log2(e)
//                      (rowstat, both stored negated so that they enter the
//                      exponent and the dP accumulators as they are; for each
//                      four rows their four lse values, then their four deltas,
//                      so a lane holding four rows reads each as one vector); with an
//                      output gate also dO*sigmoid(g) and
//                      the gate gradient dO*O*(1 - sigmoid(g)).
//   2. keys_kernel + stable radix sort (rocPRIM) + seg_off_kernel
//                      the block-transposed index: for each (b, hsel, key
//                      block j) the valid (i, slot) pairs that read block j,
//                      ascending, as a CSR.
//   3. dq_kernel       one workgroup per (b, query head, query block i), one
//                      wave per 16 query rows, walking i's selected key blocks
//                      (K and V through a direct-to-LDS ring, as in the
//                      forward): S^T = K Q^T and dP^T = V dO^T on MFMA,
//                      P = exp2(S*scale*log2e + gate*log2e - lse*log2e),
//                      dS = P (dP - delta), dQ^T += K^T dS^T; optional per-head
//                      gate-gradient partials sum(dS) per slot.
//   4. dkdv_kernel     one workgroup per (b, KV head, key block j) or part of
//                      its keys, 16 keys per wave (or wave pair) held in
//                      registers, walking j's transposed list (times the GQA
//                      group's query heads): Q and dO tiles of the reading query
//                      block through the ring, S = Q K^T, dP = dO V^T,
//                      dV^T += dO^T P, dK^T += Q^T dS. A list longer than a
//                      segment is walked by several workgroups writing fp32
//                      partials, which dkdv_reduce_kernel sums in segment order.
//
// Reference semantics: src/triton_kernel.py:77-181 (recompute of P from the
// same scores, the slot-0 triu / future-content masks, gate after scale,
// dS = P (dP - D), dQ = dS K scale, dK = dS^T Q scale, dV = P^T dO), the
// token-causal/padding/duplicate masks of src/qwen_blocksparse.py:67-72, and
// the gate gradient the gather path (src/ssa_model.py:72-74) gives.
#include <rocprim/device/device_radix_sort.hpp>
#include <rocprim/device/device_scan.hpp>

#include "fbsa_common.h"
#include "fbsa_internal.h"
#include "fbsa_tiles.h"

namespace fbsa {

enum { KIND_FULL = 0, KIND_DIAG = 1, KIND_ABS = 2, KIND_PAD = 3 };

#ifndef FBSA_DQ_LDS_BUDGET
#define FBSA_DQ_LDS_BUDGET 32768
#endif
// LDS reads in flight per row product (16-bit types, d >= 128; 0 = compiler-
// scheduled, kept for d <= 64 where the window would cost occupancy)
#ifndef FBSA_DQ_WIN
#define FBSA_DQ_WIN 8
#endif
// dQ walks a row's key blocks in ascending block index (lists of up to 64
// valid slots; more L2 hits on the gathered K/V tiles)
#ifndef FBSA_DQ_SORT
#define FBSA_DQ_SORT 1
#endif
#ifndef FBSA_DKDV_WIN
#define FBSA_DKDV_WIN 8
#endif
// output tiles of transposed reads in flight in the dQ / dK / dV products (d >= 128; 0 = batches of
// 8 waited for at once)
#ifndef FBSA_BWD_TRWIN
#define FBSA_BWD_TRWIN 8
#endif
// 16-bit types: P and dS enter the dK and dV products as hi/lo operand pairs
// (two MFMAs each) for key blocks read by more than FBSA_BWD_SPLIT_ROWS query
// rows (list entries x GQA group x block rows), so long fp32 sums over a key
// block's readers carry no per-term 16-bit rounding of P or dS
#ifndef FBSA_BWD_SPLIT
#define FBSA_BWD_SPLIT 1
#endif
#ifndef FBSA_BWD_SPLIT_ROWS
#define FBSA_BWD_SPLIT_ROWS 16384
#endif

// dQ with 16-bit operands: the row's delta is recomputed as sum P dP over its
// keys (fp32, from the unrounded P), replacing the prep's sum dO O (which
// reads the 16-bit O, formed from 16-bit P); dQ is then corrected by
// -(delta - delta_prep) sum P K from a second product on the same K reads
// (head dims up to FBSA_DQ_CORR_DMAX: at d 256 its accumulators do not fit the
// register budget), and dS enters the dQ product as a hi/lo pair when
// FBSA_DQ_SPLIT is set
#ifndef FBSA_DQ_CORR_DMAX
#define FBSA_DQ_CORR_DMAX 0
#endif
#ifndef FBSA_DQ_SPLIT
#define FBSA_DQ_SPLIT 0
#endif

// extra list segments: a segment's workgroups placed on one XCD
#ifndef FBSA_XSEG_XCD
#define FBSA_XSEG_XCD 1
#endif

// work chunks (KC query rows of one reading query block and head) per dK/dV list segment
#ifndef FBSA_SEG_CHUNKS
#define FBSA_SEG_CHUNKS 512
#endif
#ifndef FBSA_DKDV_UNROLL
#define FBSA_DKDV_UNROLL 1
#endif
#ifndef FBSA_DKDV_LDS_BUDGET
#define FBSA_DKDV_LDS_BUDGET 40960
#endif

static int64_t esize(int dtype) { return dtype == FBSA_F32 ? 4 : 2; }
static size_t al256(size_t x) { return (x + 255) & ~(size_t)255; }

// ----------------------------------------------------------------- layout
// Entries of key block j's transposed list under FBSA_FLAG_DENSE (every query
// block i >= j when causal, every query block otherwise; none for a block past
// l_valid), and the entries of the blocks before j.
__host__ __device__ inline int64_t dense_count(int64_t j, int64_t nblk, int64_t nkb, bool causal) {
  return j < nkb ? (causal ? nblk - j : nblk) : 0;
}
__host__ __device__ inline int64_t dense_prefix(int64_t j, int64_t nblk, int64_t nkb, bool causal) {
  const int64_t m = j < nkb ? j : nkb;
  return causal ? m * nblk - m * (m - 1) / 2 : m * nblk;
}

// dK/dV list segments of at most FBSA_SEG_CHUNKS (512) work chunks per
// workgroup: a segment's fp32 accumulator then sums at most 512 chunks of
// query rows, which keeps the rounding of sums over ~1e5 query rows under 1e-4
// of the result's scale (fp32) and shortens the longest walk. `maxlist` is the
// longest possible list, `walked` the (list entry, KV head) pairs in all.
static int seg_layout(const fbsa_attn_desc *d, BwdLayout *lay, int64_t maxlist, int64_t walked, size_t &off) {
  const int64_t grp = d->Hq / d->Hkv;
  const int64_t kc = d->bs < (d->D >= 256 ? 32 : 64) ? d->bs : (d->D >= 256 ? 32 : 64);
  int64_t segE = (d->dtype == FBSA_F32 ? 512 : FBSA_SEG_CHUNKS) / (grp * (d->bs / kc));
  if (segE < 16) segE = 16;
  lay->nwi = d->B * d->Hkv * d->nblk;
  if (lay->nwi >= 0x7fffffffLL)
    return fail(FBSA_EUNSUPPORTED, "fbsa_bwd: B * Hkv * nblk too large for the 32-bit list segments");
  lay->seg_entries = maxlist > segE ? segE : 0;
  lay->xub = lay->slots_ub = 0;
  lay->seg_cnt = lay->seg_pos = lay->wi_slot = lay->xtab = lay->partials = lay->scan_tmp = off;
  lay->scan_tmp_bytes = 0;
  if (lay->seg_entries) {
    lay->xub = walked / segE + 1;
    lay->slots_ub = 2 * (walked / segE) + 1;
    size_t stmp = 0;
    hipError_t e = rocprim::exclusive_scan(nullptr, stmp, (const uint64_t *)nullptr, (uint64_t *)nullptr,
                                           (uint64_t)0, (size_t)(lay->nwi + 1), rocprim::plus<uint64_t>(),
                                           (hipStream_t)0);
    if (e != hipSuccess) return hip_check(e, "scan workspace query");
    lay->scan_tmp_bytes = stmp;
    lay->seg_cnt = off; off = al256(off + (size_t)(lay->nwi + 1) * 8);
    lay->seg_pos = off; off = al256(off + (size_t)(lay->nwi + 1) * 8);
    lay->wi_slot = off; off = al256(off + (size_t)lay->nwi * 4);
    lay->xtab = off; off = al256(off + (size_t)lay->xub * 16);
    lay->partials = off; off = al256(off + (size_t)lay->slots_ub * 2 * (size_t)(d->bs * d->D) * 4);
    lay->scan_tmp = off; off = al256(off + stmp);
  }
  return FBSA_OK;
}

int bwd_layout(const fbsa_attn_desc *d, BwdLayout *lay) {
  const bool dense = (d->flags & FBSA_FLAG_DENSE) != 0;
  lay->nseg = d->B * d->hsel * d->nblk;
  if (dense) {
    // the transposed lists are implicit: only their offsets are stored
    const int64_t nkb = (d->l_valid + d->bs - 1) / d->bs;
    const int64_t per = dense_prefix(d->nblk, d->nblk, nkb, d->mask == FBSA_MASK_TOKEN_CAUSAL);
    if (lay->nseg >= 0x7fffffffLL || per >= (0x7fffffffLL / (d->B * d->hsel)))
      return fail(FBSA_EUNSUPPORTED, "fbsa_bwd: dense lists of %lld entries exceed the 32-bit transposed index",
                  (long long)(per * d->B * d->hsel));
    lay->n = 0;
    lay->end_bit = 0;
    lay->sort_tmp_bytes = 0;
    const size_t rows = (size_t)(d->B * d->Hq * d->L);
    size_t off = 0;
    lay->rowstat = off; off = al256(off + rows * 8);
    lay->dout_attn = off;
    if (d->flags & FBSA_FLAG_OUT_GATE) off = al256(off + rows * (size_t)d->D * (size_t)esize(d->dtype));
    lay->dgate_part = lay->pmass = lay->keys_in = lay->keys_out = lay->vals_in = lay->vals_out = off;
    lay->seg_off = off; off = al256(off + (size_t)(lay->nseg + 1) * 4);
    lay->sort_tmp = off;
    // fp32: every list longer than a segment is walked in segments, as for an
    // explicit list (closed-form offsets); 16-bit types walk each list whole
    // (their long sums take hi/lo operands; segments of every list would need
    // fp32 partials of about the size of the whole dense gradient)
    const int64_t maxlist = d->dtype == FBSA_F32 ? d->nblk : 0;
    int e = seg_layout(d, lay, maxlist, per * d->B * d->Hkv, off);
    if (e) return e;
    lay->total = off;
    return FBSA_OK;
  }
  lay->n = d->B * d->hsel * d->nblk * d->kk;
  if (d->nblk * d->kk >= 0x7fffffffLL || lay->nseg >= 0x7fffffffLL || lay->n >= 0x7fffffffLL)
    return fail(FBSA_EUNSUPPORTED, "fbsa_bwd: selection too large for the 32-bit transposed index");
  int bits = 1;
  while (((int64_t)1 << bits) <= lay->nseg) ++bits;
  lay->end_bit = bits;
  size_t tmp = 0;
  hipError_t e = rocprim::radix_sort_pairs(nullptr, tmp, (const uint32_t *)nullptr, (uint32_t *)nullptr,
                                           (const int32_t *)nullptr, (int32_t *)nullptr, (unsigned)lay->n, 0u,
                                           (unsigned)bits, (hipStream_t)0);
  if (e != hipSuccess) return hip_check(e, "radix sort workspace query");
  lay->sort_tmp_bytes = tmp;
  const size_t rows = (size_t)(d->B * d->Hq * d->L);
  size_t off = 0;
  lay->rowstat = off; off = al256(off + rows * 8);
  lay->dout_attn = off;
  if (d->flags & FBSA_FLAG_OUT_GATE) off = al256(off + rows * (size_t)d->D * (size_t)esize(d->dtype));
  lay->dgate_part = off; off = al256(off + (size_t)(d->B * d->Hq * d->nblk * d->kk) * 4);
  lay->pmass = off;
  if ((d->flags & FBSA_FLAG_DGATE) && d->dtype != FBSA_F32) off = al256(off + (size_t)(d->B * d->Hq * d->L * d->kk) * 4);
  lay->keys_in = off; off = al256(off + (size_t)lay->n * 4);
  lay->keys_out = off; off = al256(off + (size_t)lay->n * 4);
  lay->vals_in = off; off = al256(off + (size_t)lay->n * 4);
  lay->vals_out = off; off = al256(off + (size_t)lay->n * 4);
  lay->seg_off = off; off = al256(off + (size_t)(lay->nseg + 1) * 4);
  lay->sort_tmp = off; off = al256(off + tmp);
  // the longest possible list: token-causal selections are deduplicated, the
  // other masks count a block chosen in several slots of a row once per slot
  const int64_t maxlist = d->mask == FBSA_MASK_TOKEN_CAUSAL ? d->nblk : d->nblk * d->kk;
  int e2 = seg_layout(d, lay, maxlist, lay->n * (d->Hkv / d->hsel), off);  // hsel is 1 or Hkv
  if (e2) return e2;
  lay->total = off;
  return FBSA_OK;
}

// ----------------------------------------------------------------- stage 1
// Row statistics (workspace and LDS): rows 4k .. 4k + 3 keep their four
// -lse * log2 e at floats 8k .. 8k + 3 and their four -delta at 8k + 4 .. 8k + 7
// (8 bytes a row, as a float pair would take; L is a multiple of 16, so a
// group never spans two heads and a chunk's rows are whole groups)
__device__ __forceinline__ int64_t rs_lse_at(int64_t row) { return (row >> 2) * 8 + (row & 3); }
__device__ __forceinline__ int64_t rs_delta_at(int64_t row) { return (row >> 2) * 8 + 4 + (row & 3); }

// row 4 k4 + r of a chunk's row statistics in LDS (the same layout)
__device__ __forceinline__ float rs_lse(const float *M, int k4, int r) { return M[k4 * 8 + r]; }
__device__ __forceinline__ float rs_delta(const float *M, int k4, int r) { return M[k4 * 8 + 4 + r]; }

struct PrepArgs {
  const void *o, *dout, *og;
  const float *lse;
  float *rowstat;
  void *dout_attn, *dout_gate;
  int64_t Hq, L, rows;
  int64_t so[3], sdo[3], sog[3];
  int og_vec;  // out-gate rows and dout_gate 16-byte aligned: vector loads and stores
};

template <typename T> __device__ __forceinline__ float half_to_f32(uint32_t h) {
  if constexpr (__is_same(T, bf16)) {
    return __uint_as_float(h << 16);
  } else {
    const unsigned short hs = (unsigned short)h;
    _Float16 x;
    __builtin_memcpy(&x, &hs, 2);
    return (float)x;
  }
}

template <typename T> __device__ __forceinline__ void load8f(const T *p, float *v) {
  if constexpr (sizeof(T) == 4) {
    const f32x4 a = *(const f32x4 *)p, b = *(const f32x4 *)(p + 4);
#pragma unroll
    for (int e = 0; e < 4; ++e) { v[e] = a[e]; v[4 + e] = b[e]; }
  } else {
    // 32-bit words split with shifts: bit-casting elements of a 16-bit vector
    // value one by one is miscompiled (every element reads element 0).
    const uint4 r = *(const uint4 *)p;
    const uint32_t wd[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[2 * e] = half_to_f32<T>(wd[e] & 0xFFFFu);
      v[2 * e + 1] = half_to_f32<T>(wd[e] >> 16);
    }
  }
}

template <typename T, int D>
__global__ __launch_bounds__(256) void prep_kernel(PrepArgs a) {
  constexpr int TPR = D / 8;  // threads per row, 8 elements each
  constexpr int RPB = 256 / TPR;
  const int tid = threadIdx.x;
  const int64_t row = (int64_t)blockIdx.x * RPB + tid / TPR;
  const int c = tid % TPR;
  float acc = 0.f;
  if (row < a.rows) {
    int64_t t, h, b;
    if (a.rows < 0x80000000LL) {  // 32-bit division (a short sequence) when the row count allows
      const uint32_t r32 = (uint32_t)row, bh = r32 / (uint32_t)a.L;
      t = r32 - bh * (uint32_t)a.L;
      h = bh % (uint32_t)a.Hq;
      b = bh / (uint32_t)a.Hq;
    } else {
      const int64_t bh = row / a.L;
      t = row % a.L; h = bh % a.Hq; b = bh / a.Hq;
    }
    float ov[8], dv[8];
    load8f<T>((const T *)a.o + b * a.so[0] + h * a.so[1] + t * a.so[2] + 8 * c, ov);
    load8f<T>((const T *)a.dout + b * a.sdo[0] + h * a.sdo[1] + t * a.sdo[2] + 8 * c, dv);
#pragma unroll
    for (int e = 0; e < 8; ++e) acc = __builtin_fmaf(ov[e], dv[e], acc);
    if (a.og) {
      float gv[8], dav[8], dgv[8];
      const T *grow = (const T *)a.og + b * a.sog[0] + h * a.sog[1] + t * a.sog[2] + 8 * c;
      if (a.og_vec) {
        load8f<T>(grow, gv);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) gv[e] = (float)grow[e];
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float s = 1.f / (1.f + __expf(-gv[e]));
        dav[e] = dv[e] * s;
        dgv[e] = dv[e] * ov[e] * (1.f - s);
      }
      T *da = (T *)a.dout_attn + row * D + 8 * c;
      T *dg = (T *)a.dout_gate + row * D + 8 * c;
      if constexpr (sizeof(T) == 4) {
        *(f32x4 *)da = f32x4{dav[0], dav[1], dav[2], dav[3]};
        *(f32x4 *)(da + 4) = f32x4{dav[4], dav[5], dav[6], dav[7]};
      } else {
        *(s16x8 *)da = pack8<T>(dav);  // workspace rows: 16-byte aligned
      }
      if (a.og_vec) {
        if constexpr (sizeof(T) == 4) {
          *(f32x4 *)dg = f32x4{dgv[0], dgv[1], dgv[2], dgv[3]};
          *(f32x4 *)(dg + 4) = f32x4{dgv[4], dgv[5], dgv[6], dgv[7]};
        } else {
          *(s16x8 *)dg = pack8<T>(dgv);
        }
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) dg[e] = (T)dgv[e];
      }
    }
  }
#pragma unroll
  for (int m = TPR / 2; m >= 1; m >>= 1) acc += __shfl_xor(acc, m, 64);
  if (row < a.rows && c == 0) {
    const float l = a.lse[row];
    a.rowstat[rs_lse_at(row)] = l == -INFINITY ? -INFINITY : -l * kLog2e;  // negated: -lse log2 e
    a.rowstat[rs_delta_at(row)] = -acc;                                  // and -delta
  }
}

template <typename T, int D> static void launch_prep(const PrepArgs &a, hipStream_t s) {
  constexpr int RPB = 256 / (D / 8);
  const int64_t nwg = (a.rows + RPB - 1) / RPB;
  hipLaunchKernelGGL((prep_kernel<T, D>), dim3((unsigned)nwg), dim3(256), 0, s, a);
}

template <typename T> static int prep_d(const PrepArgs &a, int64_t D, hipStream_t s) {
  switch (D) {
    case 32: launch_prep<T, 32>(a, s); break;
    case 64: launch_prep<T, 64>(a, s); break;
    case 128: launch_prep<T, 128>(a, s); break;
    case 256: launch_prep<T, 256>(a, s); break;
    default: return fail(FBSA_EUNSUPPORTED, "fbsa_bwd_prep: head dim %lld", (long long)D);
  }
  return hip_check(hipGetLastError(), "prep_kernel launch");
}

int run_bwd_prep(const fbsa_attn_desc *d, const BwdLayout &lay, const void *o, const void *dout, const float *lse,
                 const void *out_gate, void *dout_gate, char *ws, hipStream_t s) {
  PrepArgs a;
  a.o = o; a.dout = dout; a.og = out_gate; a.lse = lse;
  a.rowstat = (float *)(ws + lay.rowstat);
  a.dout_attn = ws + lay.dout_attn;
  a.dout_gate = dout_gate;
  a.Hq = d->Hq; a.L = d->L; a.rows = d->B * d->Hq * d->L;
  for (int x = 0; x < 3; ++x) { a.so[x] = d->so[x]; a.sdo[x] = d->sdo[x]; a.sog[x] = d->sog[x]; }
  const int64_t es = esize(d->dtype);
  a.og_vec = ((uintptr_t)out_gate % 16 == 0) && ((uintptr_t)dout_gate % 16 == 0) && (d->sog[0] * es) % 16 == 0 &&
             (d->sog[1] * es) % 16 == 0 && (d->sog[2] * es) % 16 == 0;
  switch (d->dtype) {
    case FBSA_BF16: return prep_d<bf16>(a, d->D, s);
    case FBSA_F16: return prep_d<f16>(a, d->D, s);
    default: return prep_d<float>(a, d->D, s);
  }
}

// ----------------------------------------------------------------- stage 2
struct IdxArgs {
  const int32_t *sel;
  uint32_t *keys;
  int32_t *vals;
  int64_t nblk, kk, n, nseg, bs, l_valid;
  int mask;
};

// One thread per (b, hsel, i, slot): key = CSR segment of the slot's block
// when the slot is valid under the mask rule, nseg (sorted last) otherwise.
__global__ __launch_bounds__(256) void keys_kernel(IdxArgs a) {
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (e >= a.n) return;
  const int64_t s = e % a.kk, r = e / a.kk, i = r % a.nblk, bhs = r / a.nblk;
  const int32_t *row = a.sel + r * a.kk;
  const int64_t j = row[s];
  const bool inb = j >= 0 && j < a.nblk;
  bool valid;
  if (a.mask == FBSA_MASK_NONE) valid = inb && j * a.bs < a.l_valid;
  else if (a.mask == FBSA_MASK_SLOT_CAUSAL) valid = s == 0 ? inb : (inb && j < i);
  else {
    valid = inb && j <= i && j * a.bs < a.l_valid;
    for (int64_t s2 = 0; s2 < s && valid; ++s2) valid = row[s2] != j;
  }
  a.keys[e] = valid ? (uint32_t)(bhs * a.nblk + j) : (uint32_t)a.nseg;
  a.vals[e] = (int32_t)(i * a.kk + s);
}

// seg_off[x] = first sorted position whose key is >= x, for x in [0, nseg].
__global__ __launch_bounds__(256) void seg_off_kernel(const uint32_t *keys, int64_t n, int64_t nseg, int32_t *seg_off) {
  const int64_t x = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (x > nseg) return;
  int64_t lo = 0, hi = n;
  while (lo < hi) {
    const int64_t mid = (lo + hi) >> 1;
    if ((int64_t)keys[mid] < x) lo = mid + 1;
    else hi = mid;
  }
  seg_off[x] = (int32_t)lo;
}

// seg_off of the implicit dense lists: x = (b * hsel + hs) * nblk + j.
__global__ __launch_bounds__(256) void dense_seg_off_kernel(int32_t *seg_off, int64_t nseg, int64_t nblk, int64_t nkb,
                                                            int causal) {
  const int64_t x = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (x > nseg) return;
  const int64_t grp = x / nblk, j = x % nblk;
  seg_off[x] = (int32_t)(grp * dense_prefix(nblk, nblk, nkb, causal) + dense_prefix(j, nblk, nkb, causal));
}

int run_transpose_index(const fbsa_attn_desc *d, const BwdLayout &lay, const int32_t *sel, char *ws, hipStream_t s) {
  if (d->flags & FBSA_FLAG_DENSE) {
    const int64_t nkb = (d->l_valid + d->bs - 1) / d->bs;
    hipLaunchKernelGGL(dense_seg_off_kernel, dim3((unsigned)((lay.nseg + 1 + 255) / 256)), dim3(256), 0, s,
                       (int32_t *)(ws + lay.seg_off), lay.nseg, d->nblk, nkb,
                       d->mask == FBSA_MASK_TOKEN_CAUSAL ? 1 : 0);
    return hip_check(hipGetLastError(), "dense_seg_off_kernel launch");
  }
  IdxArgs a;
  a.sel = sel;
  a.keys = (uint32_t *)(ws + lay.keys_in);
  a.vals = (int32_t *)(ws + lay.vals_in);
  a.nblk = d->nblk; a.kk = d->kk; a.n = lay.n; a.nseg = lay.nseg; a.bs = d->bs; a.l_valid = d->l_valid;
  a.mask = d->mask;
  hipLaunchKernelGGL(keys_kernel, dim3((unsigned)((lay.n + 255) / 256)), dim3(256), 0, s, a);
  int e = hip_check(hipGetLastError(), "keys_kernel launch");
  if (e) return e;
  size_t tmp = lay.sort_tmp_bytes;
  e = hip_check(rocprim::radix_sort_pairs(ws + lay.sort_tmp, tmp, (const uint32_t *)(ws + lay.keys_in),
                                          (uint32_t *)(ws + lay.keys_out), (const int32_t *)(ws + lay.vals_in),
                                          (int32_t *)(ws + lay.vals_out), (unsigned)lay.n, 0u, (unsigned)lay.end_bit, s),
                "radix sort of the transposed index");
  if (e) return e;
  hipLaunchKernelGGL(seg_off_kernel, dim3((unsigned)((lay.nseg + 1 + 255) / 256)), dim3(256), 0, s,
                     (const uint32_t *)(ws + lay.keys_out), lay.n, lay.nseg, (int32_t *)(ws + lay.seg_off));
  return hip_check(hipGetLastError(), "seg_off_kernel launch");
}

// ----------------------------------------------------------------- stages 3, 4
struct BwdArgs {
  const void *q, *k, *v, *dout;  // dout: gradient of the un-gated attention output
  float *rowstat;  // negated -lse * log2 e and -delta by groups of four rows; dq_kernel replaces delta by sum P dP (16-bit types)
  // o, lse (bf16, no output gate; else null): dq_kernel forms the row
  // statistics itself (the prep stage is skipped) and writes both to rowstat
  const void *o;
  const float *lse;
  int64_t so[3];
  const int32_t *sel;
  const float *gate;
  void *dq, *dk, *dv;
  float *dgate_part;
  float *pmass;  // 16-bit gate gradient: [b, hq, i][slot][row] probability mass of a row on a slot
  const int32_t *seg_off, *ent;
  const int32_t *wi_slot;  // list segments (null: none): first partial slot of a work item, or -1
  const int4 *xtab;        // extra segments: (work item, first entry, end entry, partial slot)
  const uint64_t *seg_tot; // extra segments << 32 | partial slots, in total
  float *partials;         // [slot][dK, dV][bs rows][D] fp32
  int64_t seg_entries, seg_entries_xub;  // segment length; bound on extra segments (grid size)
  int64_t B, Hq, Hkv, L, nblk, kk, hsel, l_valid;
  int64_t sq[3], sk[3], sv[3], sdo[3];
  float scale2, scale;
  int mask, grp;
  int dense;  // FBSA_FLAG_DENSE: slot s is block s; lists implicit (i = j + position when causal)
};

// ROWS: the block rows one workgroup owns (one wave per 16), BS unless a
// block is split over several workgroups.
template <typename T, int BS, int D, int BUDGET, int META, int ROWS = BS> struct BwdCfg {
  static constexpr int ES = sizeof(T);
  static constexpr int NW = ROWS / 16;
  static constexpr int NT = NW * 64;
  // key / query rows per chunk: 64, 32 at d 256 (16-bit), 16 for fp32 at d >= 128 (registers)
  static constexpr int KCW = ES == 4 && D >= 128 ? 16 : (D >= 256 ? 32 : 64);
  static constexpr int KC = BS < KCW ? BS : KCW;
  static constexpr int NCH = BS / KC;
  static constexpr int CPR = D * ES / 16;
  static constexpr int TILE_BYTES = KC * D * ES;
  static constexpr int META_BYTES = META ? KC * 8 : 0;  // the chunk's (lse2, delta) rows, a quarter per wave
  static constexpr int STAGE_BYTES = 2 * TILE_BYTES + META_BYTES;
  static constexpr int LPT = 2 * TILE_BYTES / (NT * 16);
  static constexpr int NS0 = BUDGET / STAGE_BYTES;
  static constexpr int NSTAGE = NS0 < 2 ? 2 : (NS0 > 4 ? 4 : NS0);
  static_assert(LPT * NT * 16 == 2 * TILE_BYTES, "stage must split evenly over threads");
  static_assert(TILE_BYTES % 1024 == 0, "tile must be whole wave-loads");
};

// bs 64 with 16-bit d <= 64: held to four workgroups per CU (at most 128
// VGPRs, four waves per SIMD) like the dK/dV kernel; the chunk loop is a short
// latency-bound chain, so resident waves matter more than registers
#ifndef FBSA_DQ_MINWG
#define FBSA_DQ_MINWG 4
#endif
template <typename T, int BS, int D> constexpr int dq_minwg() {
  return (BS == 64 && D <= 64 && sizeof(T) == 2) ? FBSA_DQ_MINWG : 1;
}

// DG: the gate gradient is asked for (its sums and the slot masses are
// compiled into the chunk loop only then)
template <typename T, int BS, int D, bool DENSE = false, bool DG = false>
__global__ __launch_bounds__(BS * 4, (dq_minwg<T, BS, D>())) void dq_kernel(BwdArgs a) {
  using C = BwdCfg<T, BS, D, FBSA_DQ_LDS_BUDGET, 0>;
  extern __shared__ __attribute__((aligned(16))) char smem[];
  char *stages = smem;
  int *s_blk = (int *)(smem + C::NSTAGE * C::STAGE_BYTES);
  int *s_kind = s_blk + a.kk;
  float *s_gate = (float *)(s_kind + a.kk);
  int *s_raw = (int *)(s_gate + a.kk);        // DG: the selection slot of each compact slot
  float *s_dgw = (float *)(s_raw + a.kk);     // DG: [2][NW] per-wave dS sums of the last slot
  float *s_ddl = s_dgw + 2 * C::NW;           // DG: [BS] per-row delta - delta_prep
  __shared__ int s_nvalid;
  constexpr bool EXACT = sizeof(T) == 2;
  constexpr bool CORR = EXACT && D <= FBSA_DQ_CORR_DMAX;
  constexpr bool DQSPLIT = EXACT && FBSA_DQ_SPLIT;

  // (the wave index in a scalar register: every per-wave LDS and copy address is scalar
  // work; not with the gate gradient, whose scalar registers are short)
  const int tid = threadIdx.x, w = DG ? tid >> 6 : __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63,
            g = lane >> 4, p = lane & 15;
  const int64_t total = a.B * a.Hq * a.nblk;
  // (32-bit division: launch indices are below 2^31)
  uint32_t t = (uint32_t)xcd_remap(blockIdx.x, total);
  const int hin = (int)(t % (uint32_t)a.grp); t /= (uint32_t)a.grp;
  const int64_t i = t % (uint32_t)a.nblk; t /= (uint32_t)a.nblk;
  const int hk = (int)(t % (uint32_t)a.Hkv);
  const int64_t b = t / (uint32_t)a.Hkv;
  const int hq = hk * a.grp + hin;
  const int hs = a.hsel == 1 ? 0 : hk;

  // plan: compact list of valid slots (same rule as the forward; dense: implicit)
  const int64_t rowoff = ((b * a.hsel + hs) * a.nblk + i) * a.kk;
  const int32_t *selrow = DENSE ? nullptr : a.sel + rowoff;
  const int nkb = (int)((a.l_valid + BS - 1) / BS);  // key blocks holding a valid key
  if (!DENSE && w == 0) {
    int nout = 0;
    for (int s0 = 0; s0 < a.kk; s0 += 64) {
      const int s = s0 + lane;
      bool valid = false;
      int kind = KIND_FULL, j = 0;
      if (s < a.kk) {
        j = selrow[s];
        const bool inb = j >= 0 && j < a.nblk;
        if (a.mask == FBSA_MASK_NONE) {
          valid = inb && (int64_t)j * BS < a.l_valid;
          if (valid && (int64_t)(j + 1) * BS > a.l_valid) kind = KIND_PAD;
        } else if (a.mask == FBSA_MASK_SLOT_CAUSAL) {
          if (s == 0) { valid = inb; kind = KIND_DIAG; }
          else valid = inb && j < i;
        } else {
          valid = inb && j <= i && (int64_t)j * BS < a.l_valid;
          for (int s2 = 0; s2 < s && valid; ++s2) valid = selrow[s2] != j;
          if (valid && (j == i || (int64_t)(j + 1) * BS > a.l_valid)) kind = KIND_ABS;
        }
      }
      const uint64_t m = __ballot(valid);
      const int pos = nout + __popcll(m & ((1ull << lane) - 1ull));
      if (valid) {
        s_blk[pos] = j;
        s_kind[pos] = kind;
        s_gate[pos] = a.gate ? a.gate[rowoff + s] * kLog2e : 0.f;
        if (DG) s_raw[pos] = s;
      }
      // a masked slot's gate gradient is 0
      if (DG && s < a.kk && !valid) a.dgate_part[((b * a.Hq + hq) * a.nblk + i) * a.kk + s] = 0.f;
      nout += __popcll(m);
    }
    if (lane == 0) s_nvalid = nout;
    if (FBSA_DQ_SORT && nout > 1 && nout <= 64) {
      // ascending key blocks, as the forward walks them; equal blocks keep their
      // slot order (the selection slot of each entry moves with it)
      int j = 0x7fffffff, kind = 0, rs = 0;
      float gt = 0.f;
      if (lane < nout) {
        j = s_blk[lane]; kind = s_kind[lane]; gt = s_gate[lane];
        if (DG) rs = s_raw[lane];
      }
      int rank = 0;
      for (int m = 0; m < nout; ++m) {
        const int jm = s_blk[m];
        rank += jm < j || (jm == j && m < lane);
      }
      __builtin_amdgcn_wave_barrier();
      if (lane < nout) {
        s_blk[rank] = j; s_kind[rank] = kind; s_gate[rank] = gt;
        if (DG) s_raw[rank] = rs;
      }
    }
  }

  const int tq = w * 16 + p;
  const int64_t qpos = i * BS + tq;
  RowFrag<T, D> qf, df;
  qf.load((const T *)a.q + b * a.sq[0] + hq * a.sq[1] + qpos * a.sq[2], g);
  df.load((const T *)a.dout + b * a.sdo[0] + hq * a.sdo[1] + qpos * a.sdo[2], g);
  // the row statistics: from the prep stage, or (fused) formed here exactly as
  // prep_kernel forms them (below, once the ring's first loads are in flight)
  const bool fused = __is_same(T, bf16) && a.o != nullptr;  // uniform
  RowFrag<T, D> of;
  float lraw = 0.f;
  float2 rs = make_float2(0.f, 0.f);
  if (fused) {
    of.load((const T *)a.o + b * a.so[0] + hq * a.so[1] + qpos * a.so[2], g);
    lraw = a.lse[(b * a.Hq + hq) * a.L + qpos];
  } else {
    const int64_t row = (b * a.Hq + hq) * a.L + qpos;
    rs = make_float2(a.rowstat[rs_lse_at(row)], a.rowstat[rs_delta_at(row)]);
  }
  __syncthreads();
  const int nv = DENSE ? (a.mask == FBSA_MASK_TOKEN_CAUSAL && i + 1 < nkb ? (int)i + 1 : nkb) : s_nvalid;
  const int nchunks = nv * C::NCH;
  auto blk_of = [&](int slot) { return DENSE ? slot : s_blk[slot]; };
  auto kind_of = [&](int slot) {
    if (!DENSE) return s_kind[slot];
    const int64_t jj = slot;
    const bool pad = (jj + 1) * BS > a.l_valid;
    return a.mask == FBSA_MASK_TOKEN_CAUSAL ? ((jj == i || pad) ? (int)KIND_ABS : (int)KIND_FULL)
                                            : (pad ? (int)KIND_PAD : (int)KIND_FULL);
  };

  const T *kbase = (const T *)a.k + b * a.sk[0] + hk * a.sk[1];
  const T *vbase = (const T *)a.v + b * a.sv[0] + hk * a.sv[1];
  // a per-thread copy plan (offsets computed once, uniform row-0 bases per
  // chunk); d <= 64 issues through the compiler builtin (four workgroups per
  // CU, measured faster there than the asm form), d > 64 through the asm form
  TilePairPlan<T, C::KC, D, C::NW, C::LPT> plan;
  plan.init(a.sk[2], a.sv[2], w, lane);
  auto issue = [&](int c) {
    const int slot = c / C::NCH, ch = c % C::NCH;
    const int64_t row0 = (int64_t)__builtin_amdgcn_readfirstlane(blk_of(slot) * BS + ch * C::KC);
    plan.template issue<(D <= 64)>(stages + (c % C::NSTAGE) * C::STAGE_BYTES, (const char *)(kbase + row0 * a.sk[2]),
                                   (const char *)(vbase + row0 * a.sv[2]), w);
  };

  // dP^T accumulators start at -delta (16-bit types without the gate gradient, whose
  // registers are short: dS = P (dP - delta) is then one product; the others keep
  // the separate subtraction)
  constexpr bool DINIT = EXACT && !DG;
  f32x4 dqacc[D / 16], bacc[CORR ? D / 16 : 1];  // bacc: sum P K (the delta correction)
#pragma unroll
  for (int mt = 0; mt < D / 16; ++mt) dqacc[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int mt = 0; mt < (CORR ? D / 16 : 1); ++mt) bacc[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
  float dgl = 0.f, pml = 0.f, dacc = 0.f;  // slot's dS sum and P mass; this lane's sum of P dP
  constexpr bool want_dg = DG;
  // this workgroup's rows' slot masses ([compact slot][row]; lanes g == 0 of
  // each wave write and read back their own rows)
  float *pm = EXACT && want_dg ? a.pmass + ((b * a.Hq + hq) * a.nblk + i) * a.kk * BS : nullptr;
  float *dgrow = want_dg ? a.dgate_part + ((b * a.Hq + hq) * a.nblk + i) * a.kk : nullptr;

#pragma unroll
  for (int c = 0; c < C::NSTAGE - 1; ++c)
    if (c < nchunks) issue(c);
  // the register-operand loads above and the first stages have landed (issued
  // together, so their latencies overlap): the compiler then waits for nothing
  // inside the ring loop, where its own waits would also drain the prefetch
  wait_vmcnt<0>();

  // fused row statistics: per 8-element chunk c = 4 ks + g an fma chain over
  // dO*O from 0, then the chunks' pairwise tree c + c ^ m for m = D/16 .. 1 (the
  // lane's own chunks first, then across the lanes g), as prep_kernel sums them
  float lse2 = -rs.x, delta = -rs.y;  // stored negated
  if constexpr (__is_same(T, bf16)) if (fused) {
    constexpr int KS = D / 32;
    float cs[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const s16x8 ov = of.h[ks], dv = df.h[ks];
      float acc = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e)
        acc = __builtin_fmaf(half_to_f32<T>((uint32_t)(uint16_t)ov[e]), half_to_f32<T>((uint32_t)(uint16_t)dv[e]), acc);
      cs[ks] = acc;
    }
#pragma unroll
    for (int m = KS / 2; m >= 1; m >>= 1)
#pragma unroll
      for (int ks = 0; ks < m; ++ks) cs[ks] += cs[ks + m];
    float dsum = cs[0] + shfl_xor_f(cs[0], 32);  // chunk pairs c, c ^ 2 (lanes g, g ^ 2)
    dsum += shfl_xor_f(dsum, 16);                 // c, c ^ 1
    lse2 = lraw == -INFINITY ? INFINITY : lraw * kLog2e;
    delta = dsum;
  }
  f32x4 dinit[C::KC / 16];
#pragma unroll
  for (int m = 0; m < C::KC / 16; ++m) dinit[m] = f32x4{-delta, -delta, -delta, -delta};

  for (int c = 0; c < nchunks; ++c) {
    // stage c has landed for this wave (up to NSTAGE - 2 later stages may be in flight);
    // after the barrier every wave is also done with chunk c - 1, whose stage is refilled
    const int ahead = nchunks - 1 - c;
    wait_ring<C::LPT>(ahead < C::NSTAGE - 2 ? ahead : C::NSTAGE - 2);
    lds_barrier();
    if (c + C::NSTAGE - 1 < nchunks) issue(c + C::NSTAGE - 1);

    const char *Ks = stages + (c % C::NSTAGE) * C::STAGE_BYTES;
    const char *Vs = Ks + C::TILE_BYTES;
    const int slot = c / C::NCH, ch = c % C::NCH;
    if (want_dg && ch == 0 && slot > 0 && w == 0) {
      // the previous slot's per-wave sums are in (written before this barrier)
      float v = lane < C::NW ? s_dgw[((slot - 1) & 1) * C::NW + lane] : 0.f;
#pragma unroll
      for (int x = 1; x < C::NW; x <<= 1) v += shfl_xor_f(v, x);
      if (lane == 0) dgrow[s_raw[slot - 1]] = v;
    }
    const int kind = kind_of(slot);
    const float gt = DENSE ? 0.f : s_gate[slot];
    const int64_t j = blk_of(slot);

    f32x4 sacc[C::KC / 16], dpacc[C::KC / 16];
    mm_rows_frag<T, D, C::KC / 16, (D >= 128 ? FBSA_DQ_WIN : 0)>(Ks, qf, sacc, g, p);   // S^T: key 16m+4g+r, query p
    mm_rows_frag<T, D, C::KC / 16, (D >= 128 ? FBSA_DQ_WIN : 0)>(Vs, df, dpacc, g, p,
                                                                  DINIT ? dinit : nullptr);  // dP^T (- delta)

    const float off = gt - lse2;
    float ds[C::KC / 16][4], pp[C::KC / 16][4];
#pragma unroll
    for (int m = 0; m < C::KC / 16; ++m)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float pv = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[m][r], a.scale2, off));
        pp[m][r] = pv;
        ds[m][r] = DINIT ? pv * dpacc[m][r] : pv * (dpacc[m][r] - delta);
      }
    // masked keys (key row 16m + r of the chunk valid iff <= lim): a uniform
    // branch, so unmasked chunks (the common case) skip the compares
    if (kind != KIND_FULL) {
      const int64_t lim64 = kind == KIND_DIAG ? (int64_t)tq
                            : kind == KIND_PAD  ? a.l_valid - j * BS - 1
                                                : ((i - j) * BS + tq < a.l_valid - j * BS - 1 ? (i - j) * BS + tq
                                                                                              : a.l_valid - j * BS - 1);
      const int lim = (int)(lim64 < -1 ? -1 : lim64) - ch * C::KC - 4 * g;
#pragma unroll
      for (int m = 0; m < C::KC / 16; ++m)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (16 * m + r > lim) { ds[m][r] = 0.f; pp[m][r] = 0.f; }
    }
    if constexpr (EXACT) {
#pragma unroll
      for (int m = 0; m < C::KC / 16; ++m)
#pragma unroll
        for (int r = 0; r < 4; ++r) dacc = __builtin_fmaf(pp[m][r], dpacc[m][r], dacc);
    }
    if (want_dg) {
#pragma unroll
      for (int m = 0; m < C::KC / 16; ++m)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          dgl += ds[m][r];
          if constexpr (EXACT) pml += pp[m][r];
        }
    }
    if (want_dg && ch == C::NCH - 1) {
#pragma unroll
      for (int x = 1; x < 64; x <<= 1) dgl += shfl_xor_f(dgl, x);
      if (lane == 0) s_dgw[(slot & 1) * C::NW + w] = dgl;
      dgl = 0.f;
      if constexpr (EXACT) {
        // the slot's P mass per query row (its four lanes' parts)
        pml += shfl_xor_f(pml, 16);
        pml += shfl_xor_f(pml, 32);
        if (g == 0) pm[(uint32_t)(slot * BS + tq)] = pml;  // uniform base + 32-bit lane offset
        pml = 0.f;
      }
    }
    // dQ^T += K^T dS^T (and, with the delta correction, sum P K from the same reads)
    if constexpr (CORR)
      mm_tr_acc<T, D, C::KC, (D >= 128 ? FBSA_BWD_TRWIN : 0), DQSPLIT, 2>(Ks, ds, dqacc, g, p, pp, bacc);
    else
      mm_tr_acc<T, D, C::KC, (D >= 128 ? FBSA_BWD_TRWIN : 0), DQSPLIT>(Ks, ds, dqacc, g, p);
  }

  // the row's delta as sum P dP (its four lanes' parts); with DINIT dacc holds
  // sum P (dP - delta_prep), which is delta - delta_prep since the row's P sums
  // to 1 (to fp32 rounding). dgate and dQ take the difference to the prep's
  // delta, dK/dV read the new delta from the row stats
  float ddl = 0.f;
  if constexpr (EXACT) {
    float dx = dacc + shfl_xor_f(dacc, 16);
    dx += shfl_xor_f(dx, 32);
    ddl = DINIT ? dx : dx - delta;
    const float dnew = DINIT ? delta + dx : dx;
    if (g == 0) {
      const int64_t row = (b * a.Hq + hq) * a.L + qpos;
      if (fused) a.rowstat[rs_lse_at(row)] = lse2 == INFINITY ? -INFINITY : -lse2;
      a.rowstat[rs_delta_at(row)] = -dnew;
    }
  }

  T *dqrow = (T *)a.dq + ((b * a.Hq + hq) * a.L + qpos) * D;
#pragma unroll
  for (int mt = 0; mt < D / 16; ++mt) {
    const int d0 = 16 * mt + 4 * g;
    if constexpr (sizeof(T) == 4) {
      *(f32x4 *)(dqrow + d0) = f32x4{dqacc[mt][0] * a.scale, dqacc[mt][1] * a.scale, dqacc[mt][2] * a.scale,
                                     dqacc[mt][3] * a.scale};
    } else {
      s16x4 pk;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float y = CORR ? __builtin_fmaf(-ddl, bacc[mt][r], dqacc[mt][r]) : dqacc[mt][r];
        pk[r] = bits16<T>((T)(y * a.scale));
      }
      *(s16x4 *)(dqrow + d0) = pk;
    }
  }
  if (want_dg) {
    // the last slot's sums, and for 16-bit types each slot's correction: minus
    // the sum over rows of (delta - delta_prep) times the row's P mass on the
    // slot (wave 0, each lane taking BS / 64 rows)
    if (EXACT && g == 0) s_ddl[tq] = ddl;
    __syncthreads();
    if (w == 0) {
      if (nv > 0) {
        float v = lane < C::NW ? s_dgw[((nv - 1) & 1) * C::NW + lane] : 0.f;
#pragma unroll
        for (int x = 1; x < C::NW; x <<= 1) v += shfl_xor_f(v, x);
        if (lane == 0) dgrow[s_raw[nv - 1]] = v;
      }
      if constexpr (EXACT) {
        for (int c = 0; c < nv; ++c) {
          float v = 0.f;
          for (int r = lane; r < BS; r += 64) v += pm[(uint32_t)(c * BS + r)] * s_ddl[r];
#pragma unroll
          for (int x = 1; x < 64; x <<= 1) v += shfl_xor_f(v, x);
          if (lane == 0) dgrow[s_raw[c]] -= v;
        }
      }
    }
  }
}

// A dK/dV wave keeps its 16 keys' K and V fragments and their dK and dV
// accumulators in registers: 2 D (16-bit) or 4 D (fp32) values per lane besides
// the per-chunk S, dP and tile reads. Eight waves (bs 128) share a SIMD two by
// two, leaving 256 registers each, too few from 16-bit d 256 or fp32 d 128 on
// (the remainder went to scratch); there a workgroup takes half a key block (four
// waves, one per SIMD, 512 registers each) and the two halves of a block run
// back to back on one XCD, so the second read of each Q / dO tile is an L2 hit. Such a workgroup holds a whole CU's registers, so its ring can take
// most of the LDS.
// For 16-bit d 256 the keys' work is split over two waves by role instead: wave
// 0 of a pair holds K, forms S and P and accumulates dV; wave 1 holds V, forms
// dP, takes P from its partner through LDS and accumulates dK. Each wave then
// holds one fragment and one accumulator (half the registers), two waves share
// each SIMD, and the MFMA and LDS work per key is unchanged; P and dS are the
// same expressions in the same order, so results do not change.
template <typename T, int D> constexpr bool dkdv_heavy() { return D >= 256 || (sizeof(T) == 4 && D >= 128); }
template <typename T, int D> constexpr int dkdv_roles() { return sizeof(T) == 2 && D >= 256 ? 2 : 1; }
template <typename T, int BS, int D> constexpr int dkdv_keys() {  // keys per workgroup
  return dkdv_roles<T, D>() == 2 ? (BS < 64 ? BS : 64) : (BS == 128 && dkdv_heavy<T, D>() ? 64 : BS);
}
template <typename T, int BS, int D> constexpr int dkdv_rows() { return dkdv_keys<T, BS, D>() * dkdv_roles<T, D>(); }
// Minimum resident workgroups for the register budget; the compiler counts a
// workgroup as at least one wave per SIMD, so 2 means two waves per SIMD for
// workgroups of up to four waves, and 1 does for eight-wave workgroups.
template <typename T, int BS, int D> constexpr int dkdv_minwg() {
  return dkdv_roles<T, D>() == 2 ? (dkdv_rows<T, BS, D>() >= 128 ? 1 : 2)
                                 : (BS == 64 && D <= 64 && sizeof(T) == 2) ? 4 : 1;
}
#ifndef FBSA_DKDV_HEAVY_LDS_BUDGET
#define FBSA_DKDV_HEAVY_LDS_BUDGET 102400
#endif
// Two roles, one barrier per chunk: the P hand-over of chunk c is consumed after
// the ring barrier of chunk c + 1 (so a stage is read in two iterations and the
// ring needs one stage more for the same prefetch depth)
#ifndef FBSA_DKDV_PIPE
#define FBSA_DKDV_PIPE 1
#endif
#ifndef FBSA_DKDV_PIPE_LDS_BUDGET
#define FBSA_DKDV_PIPE_LDS_BUDGET 132096
#endif
// the one-role chunk loop unrolled by the ring depth (16-bit, d <= 64, every
// stage offset within a 16-bit LDS instruction offset)
template <typename T, int BS, int D> constexpr bool dkdv_unrolled();
template <typename T, int BS, int D> constexpr bool dkdv_pipe() {
  return dkdv_roles<T, D>() == 2 && dkdv_rows<T, BS, D>() >= 128 && FBSA_DKDV_PIPE;
}
template <typename T, int BS, int D>
using DkdvCfg = BwdCfg<T, BS, D,
                       dkdv_pipe<T, BS, D>() ? FBSA_DKDV_PIPE_LDS_BUDGET
                       : dkdv_heavy<T, D>() && (dkdv_roles<T, D>() == 2 ? dkdv_rows<T, BS, D>() >= 64
                                                                     : dkdv_rows<T, BS, D>() == 64)
                           ? FBSA_DKDV_HEAVY_LDS_BUDGET / dkdv_minwg<T, BS, D>()
                           : FBSA_DKDV_LDS_BUDGET,
                       1, dkdv_rows<T, BS, D>()>;
template <typename T, int BS, int D> constexpr bool dkdv_unrolled() {
  return sizeof(T) == 2 && D <= 64 && dkdv_roles<T, D>() == 1 && DkdvCfg<T, BS, D>::KC >= 64 &&
         DkdvCfg<T, BS, D>::NSTAGE * DkdvCfg<T, BS, D>::STAGE_BYTES <= 60000 && FBSA_DKDV_UNROLL;
}

// Latency bound (each chunk is a short chain of LDS reads, MFMAs and
// exponentials), so occupancy decides: for bs 64 with 16-bit d <= 64 the
// kernel is held to four waves per SIMD (at most 128 VGPRs) and its two-stage
// ring (35 KB of LDS) fits four workgroups per CU.
template <typename T, int BS, int D, bool DENSE = false>
__global__ __launch_bounds__((dkdv_rows<T, BS, D>() * 4), (dkdv_minwg<T, BS, D>())) void dkdv_kernel(BwdArgs a) {
  using C = DkdvCfg<T, BS, D>;
  constexpr bool SPLIT = FBSA_BWD_SPLIT && sizeof(T) == 2;
  constexpr int ROLES = dkdv_roles<T, D>(), KEYS = dkdv_keys<T, BS, D>();
  constexpr int NPART = BS / KEYS;  // workgroups per key block
  constexpr int MAXE = 128;  // transposed-list entries staged in LDS per batch
  constexpr int HR = C::KC >= 64 ? 32 : C::KC;  // query rows per part of a chunk
  extern __shared__ __attribute__((aligned(16))) char smem[];
  char *stages = smem;
  int4 *s_meta = (int4 *)(smem + C::NSTAGE * C::STAGE_BYTES);  // per entry: query block, mask kind, gate bits
  float4 *s_xch = (float4 *)(s_meta + MAXE);  // two roles: P of each key group's part, [HR/16][KEYS/16][64 lanes]

  // one role per wave: the wave index as a scalar (its tile-part selects and
  // copy bases then stay on the scalar unit; measured 3% faster at d 64, slower
  // for the two-role kernels)
  const int tid = threadIdx.x, w = ROLES == 1 ? __builtin_amdgcn_readfirstlane(tid >> 6) : tid >> 6, lane = tid & 63,
            g = lane >> 4, p = lane & 15;
  // Launch order. Causal selection gives low key blocks far longer transposed
  // lists than high ones. When every XCD's contiguous share of the (b, KV head,
  // block) units is whole rows of key blocks, the shares carry equal work and
  // neighbouring blocks (read by overlapping query blocks) share an L2: XCD-
  // contiguous ranges. Otherwise (a share is part of a row) such ranges would
  // leave most of the work on a few XCDs: units go round-robin over the XCDs
  // instead. Either way a block's NPART workgroups run back to back on one XCD.
  // A long list is walked in segments: the extra segments (all but a work
  // item's first) come first in launch order, then one workgroup set per work
  // item with its first segment (or whole list).
  const int64_t nunits = a.B * a.Hkv * a.nblk;
  const int64_t nx = a.wi_slot ? (int64_t)(*a.seg_tot >> 32) : 0;
  int64_t bid = blockIdx.x;
  int kpart = 0, slot = -1, e0 = 0, e1 = 0;
  int64_t t;
  const bool extra = bid < nx * NPART;
  if (extra) {
    // the NPART workgroups of an extra segment on one XCD too (they read the
    // same Q / dO tiles)
    const int4 xe = a.xtab[FBSA_XSEG_XCD ? gqa_unit(bid, nx, NPART, &kpart) : bid / NPART];
    if (!FBSA_XSEG_XCD) kpart = (int)(bid % NPART);
    t = xe.x; e0 = xe.y; e1 = xe.z; slot = xe.w;
  } else {
    bid -= nx * NPART;
    if (bid >= nunits * NPART) return;  // past the segments actually present
    if (nunits % 8 == 0 && (nunits / 8) % a.nblk == 0) {
      t = xcd_remap(bid, nunits * NPART);
      kpart = (int)(t % NPART);
      t /= NPART;
    } else {
      t = gqa_unit(bid, nunits, NPART, &kpart);
    }
  }
  const int64_t wi = t;
  // (32-bit division: work-item indices are below 2^31)
  const uint32_t t32 = (uint32_t)t;
  const int64_t j = t32 % (uint32_t)a.nblk;
  const int hk = (int)(t32 / (uint32_t)a.nblk % (uint32_t)a.Hkv);
  const int64_t b = t32 / (uint32_t)a.nblk / (uint32_t)a.Hkv;
  const int hs = a.hsel == 1 ? 0 : hk;
  const int64_t seg = (b * a.hsel + hs) * a.nblk + j;
  if (!extra) {
    e0 = a.seg_off[seg];
    e1 = a.seg_off[seg + 1];
    if (a.wi_slot && (slot = a.wi_slot[wi]) >= 0) e1 = e0 + (int)a.seg_entries;
  }

  // hi/lo operands for key blocks whose whole list sums more than
  // FBSA_BWD_SPLIT_ROWS query rows (a uniform branch): the per-term 16-bit
  // rounding of P and dS then stays out of long sums, while short lists (most
  // blocks of a random top-k selection) keep one MFMA per product
  const bool split = SPLIT && (int64_t)(a.seg_off[seg + 1] - a.seg_off[seg]) * a.grp * BS > FBSA_BWD_SPLIT_ROWS;
  auto tr_acc = [&](auto SPC, const char *tile, const float (&x)[HR / 16][4], f32x4 *acc) {
    mm_tr_acc<T, D, HR, (D >= 128 ? FBSA_BWD_TRWIN : 0), decltype(SPC)::value>(tile, x, acc, g, p);
  };

  const int role = ROLES == 2 ? (w & 1) : 0, kw = ROLES == 2 ? (w >> 1) : w;
  const int u = kpart * KEYS + kw * 16 + p;  // this lane's key row within block j (B-operand column)
  const int64_t kpos = j * BS + u;
  const T *krow = (const T *)a.k + b * a.sk[0] + hk * a.sk[1] + kpos * a.sk[2];
  const T *vrow = (const T *)a.v + b * a.sv[0] + hk * a.sv[1] + kpos * a.sv[2];
  RowFrag<T, D> kf, vf;  // two roles: kf holds K (role 0) or V (role 1), vf is unused
  kf.load(ROLES == 2 && role ? vrow : krow, g);
  if constexpr (ROLES == 1) vf.load(vrow, g);
  const bool keyok = kpos < a.l_valid;

  // two roles: dvacc accumulates dV (role 0) or dK (role 1)
  f32x4 dkacc[ROLES == 2 ? 1 : D / 16], dvacc[D / 16];
#pragma unroll
  for (int mt = 0; mt < D / 16; ++mt) {
    if constexpr (ROLES == 1) dkacc[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
    dvacc[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  // Direct-to-LDS copy plan for a chunk's Q / dO tile pair: which tensor each
  // of this thread's LPT loads reads is uniform across the wave (a tile is a
  // whole number of 1 KiB wave-loads) and its byte offset from the chunk's
  // first row is fixed, so an issue is a scalar base plus a precomputed offset.
  int32_t toff[C::LPT];
  bool tdo[C::LPT];
#pragma unroll
  for (int n = 0; n < C::LPT; ++n) {
    const int u = (n * C::NW + w) * 64 + lane;
    const int part = u / (C::KC * C::CPR);
    const int rem = u - part * (C::KC * C::CPR);
    const int row = rem / C::CPR, pos = rem % C::CPR;
    toff[n] = (int32_t)(((int64_t)row * (part ? a.sdo[2] : a.sq[2]) + (pos ^ swz(row, C::CPR)) * (16 / C::ES)) * C::ES);
    tdo[n] = (n * C::NW + w) * 64 >= C::KC * C::CPR;  // == (part != 0), uniform across the wave
  }

  // Q / dO / row-statistics bases of the group's first query head and the
  // per-head and per-row byte steps
  const char *qh0 = (const char *)a.q + (b * a.sq[0] + (int64_t)hk * a.grp * a.sq[1]) * C::ES;
  const char *dh0 = (const char *)a.dout + (b * a.sdo[0] + (int64_t)hk * a.grp * a.sdo[1]) * C::ES;
  const float *rh0 = a.rowstat + 2 * (b * a.Hq + (int64_t)hk * a.grp) * a.L;  // 8 bytes a row
  const int64_t qhs = a.sq[1] * C::ES, dhs = a.sdo[1] * C::ES;
  const uint32_t qrs = (uint32_t)(a.sq[2] * C::ES), drs = (uint32_t)(a.sdo[2] * C::ES);

  // dense lists: entry at position e of block j's list is query block dense_i0 + e
  const int64_t dense_i0 = DENSE ? (a.mask == FBSA_MASK_TOKEN_CAUSAL ? j : 0) - a.seg_off[seg] : 0;
  // the list walk, instantiated with and without the hi/lo operands and with
  // and without a gate bias (both choices uniform per workgroup and made once,
  // outside the loops)
  auto walk = [&](auto SPC, auto GCC) {
    constexpr bool GC = decltype(GCC)::value;  // gate bias present (else the exponent's offset is -lse)
    for (int eb = e0; eb < e1; eb += MAXE) {
      const int ne = e1 - eb < MAXE ? e1 - eb : MAXE;
      __syncthreads();  // the previous batch's entries are no longer read
      for (int x = tid; x < ne; x += C::NT) {
        // dense: the list of block j is query blocks j.. (causal) or 0.., slot j
        int i, s;
        if (DENSE) {
          i = (int)(dense_i0 + eb + x);
          s = (int)j;
        } else {
          const uint32_t ev = (uint32_t)a.ent[eb + x];  // i * kk + slot (below 2^31)
          i = (int)(ev / (uint32_t)a.kk);
          s = (int)(ev % (uint32_t)a.kk);
        }
        int kind = KIND_FULL;
        if (a.mask == FBSA_MASK_SLOT_CAUSAL) kind = s == 0 ? KIND_DIAG : KIND_FULL;
        else if (a.mask == FBSA_MASK_NONE) kind = (j + 1) * BS > a.l_valid ? KIND_PAD : KIND_FULL;
        else if (a.mask == FBSA_MASK_TOKEN_CAUSAL)
          kind = (j == i || (j + 1) * BS > a.l_valid) ? KIND_ABS : KIND_FULL;
        const float gt = a.gate ? a.gate[((b * a.hsel + hs) * a.nblk + i) * a.kk + s] * kLog2e : 0.f;
        s_meta[x] = int4{i, kind, __float_as_int(gt), 0};
      }
      __syncthreads();
      // chunk c = (entry, query head of the group, KC-row chunk), the chunk index fastest;
      // the issue side and the compute side each step their own counters (no divisions)
      const int nchunks = ne * a.grp * C::NCH;
      int ix = 0, ig = 0, ic = 0, istg = 0;  // next chunk to issue and its stage
      // the current query head's Q, dO and row-statistics bases, stepped when
      // the head changes; a chunk's rows add a 32 x 32 -> 64-bit product
      // (row < L < 2^31, row strides below 4 GiB: checked by the host)
      const char *qh = qh0, *dh = dh0;
      const float *rh = rh0;
      auto issue = [&]() {
        // uniform: kept in scalar registers, so the tile and row-statistics
        // addresses below are formed by scalar instructions
        const uint32_t row0 =
            (uint32_t)__builtin_amdgcn_readfirstlane((int)((uint32_t)s_meta[ix].x * (uint32_t)BS + (uint32_t)(ic * C::KC)));
        const char *qb = qh + (uint64_t)row0 * qrs;
        const char *db = dh + (uint64_t)row0 * drs;
        char *st = stages + istg * C::STAGE_BYTES;
  #pragma unroll
        for (int n = 0; n < C::LPT; ++n) g2lds16_s(tdo[n] ? db : qb, (unsigned)toff[n], st + (n * C::NW + w) * 1024);
        // wave w copies rows w KC/NW .. (w + 1) KC/NW - 1 of the row statistics (two per lane)
        if (lane < C::KC / (2 * C::NW))
          g2lds16(rh + 2 * (row0 + w * (C::KC / C::NW)) + 4 * lane, st + 2 * C::TILE_BYTES + w * (C::KC / C::NW) * 8);
        if (++ic == C::NCH) {
          ic = 0;
          if (++ig == a.grp) {
            ig = 0;
            ++ix;
            qh = qh0; dh = dh0; rh = rh0;
          } else {
            qh += qhs; dh += dhs; rh += 2 * a.L;
          }
        }
        if (++istg == C::NSTAGE) istg = 0;
      };
      if constexpr (dkdv_pipe<T, BS, D>()) {
        // Two roles, one barrier per chunk. Iteration c: barrier; refill the
        // stage of chunk c - 2; finish chunk c - 1 (role 0: dV += dO^T P from
        // its registers; role 1: P from the exchange buffer written before this
        // barrier, dS, dK += Q^T dS); start chunk c (role 0: S, P into exchange
        // buffer c & 1; role 1: dP kept in registers). A stage is read in two
        // iterations, so AHEAD = NSTAGE - 2 chunks are prefetched.
        static_assert(C::KC == HR && C::NSTAGE >= 3, "one part per chunk, three stages or more");
        constexpr int AHEAD = C::NSTAGE - 2;
        constexpr int XS = (KEYS / 16) * 64;  // float4 stride between the parts m of a buffer
  #pragma unroll
        for (int c = 0; c < AHEAD; ++c)
          if (c < nchunks) issue();
        wait_vmcnt<0>();
        int cx = 0, cg = 0, cch = 0, cstg = 0;  // chunk c and its stage
        float x[HR / 16][4];                   // pending chunk: P (role 0) or dP (role 1)
        const char *pQ = stages, *pD = stages;
        const float *pM = (const float *)stages;
        for (int c = 0; c <= nchunks; ++c) {
          if (c < nchunks) {
            const int ahead = nchunks - 1 - c;
            wait_ring<C::LPT + 1>(ahead < AHEAD - 1 ? ahead : AHEAD - 1);
          }
          lds_barrier();
          if (c + AHEAD < nchunks) issue();
          if (c > 0) {
            if (role == 0) {
              tr_acc(SPC, pD, x, dvacc);  // dV^T += dO^T P
            } else {
              const float4 *xs = s_xch + ((c - 1) & 1) * (HR / 16) * XS + kw * 64 + lane;
  #pragma unroll
              for (int m = 0; m < HR / 16; ++m) {
                const float4 pv = xs[m * XS];
                const float pr[4] = {pv.x, pv.y, pv.z, pv.w};
  #pragma unroll
                for (int r = 0; r < 4; ++r) x[m][r] = pr[r] * (x[m][r] + rs_delta(pM, 4 * m + g, r));
              }
              tr_acc(SPC, pQ, x, dvacc);  // dK^T += Q^T dS
            }
          }
          if (c == nchunks) break;

          const char *Qs = stages + cstg * C::STAGE_BYTES;
          const char *Ds = Qs + C::TILE_BYTES;
          const float *Ms = (const float *)(Qs + 2 * C::TILE_BYTES);
          const int4 meta = s_meta[cx];
          const int ch = cch;
          const int kind = meta.y;
          const float gt = __int_as_float(meta.z);
          const int64_t i = meta.x;
          if (++cch == C::NCH) {
            cch = 0;
            if (++cg == a.grp) { cg = 0; ++cx; }
          }
          if (++cstg == C::NSTAGE) cstg = 0;
          int tmin = -(1 << 30);
          bool kok = true;
          if (kind == KIND_DIAG) tmin = u;
          else if (kind == KIND_PAD) kok = keyok;
          else if (kind == KIND_ABS) {
            const int64_t tm = (int64_t)u - (i - j) * BS;
            tmin = (int)(tm < -(1 << 30) ? -(1 << 30) : tm);
            kok = keyok;
          }
          tmin -= ch * C::KC + 4 * g;  // compare against 16m + r

          f32x4 xacc[HR / 16];
          mm_rows_frag<T, D, HR / 16, (D >= 128 ? FBSA_DKDV_WIN : 0)>(role ? Ds : Qs, kf, xacc, g, p);  // S or dP
          if (role == 0) {
            float4 *xs = s_xch + (c & 1) * (HR / 16) * XS + kw * 64 + lane;
  #pragma unroll
            for (int m = 0; m < HR / 16; ++m) {
  #pragma unroll
              for (int r = 0; r < 4; ++r) {
                const float ml = rs_lse(Ms, 4 * m + g, r);
                const bool ok = kok && (16 * m + r >= tmin);
                float ev = __builtin_amdgcn_exp2f(__builtin_fmaf(xacc[m][r], a.scale2, GC ? gt + ml : ml));
                asm volatile("" : "+v"(ev));
                x[m][r] = ok ? ev : 0.f;
              }
              xs[m * XS] = make_float4(x[m][0], x[m][1], x[m][2], x[m][3]);
            }
          } else {
  #pragma unroll
            for (int m = 0; m < HR / 16; ++m)
  #pragma unroll
              for (int r = 0; r < 4; ++r) x[m][r] = xacc[m][r];
          }
          pQ = Qs; pD = Ds; pM = Ms;
        }
        continue;
      }

  #pragma unroll
      for (int c = 0; c < C::NSTAGE - 1; ++c)
        if (c < nchunks) issue();
      // the register-operand loads above and the first stages have landed (issued
      // together, so their latencies overlap): the compiler then waits for nothing
      // inside the ring loop, where its own waits would also drain the prefetch
      wait_vmcnt<0>();


      int cx = 0, cg = 0, cch = 0, cstg = 0;  // chunk c and its stage
      if constexpr (dkdv_unrolled<T, BS, D>()) {
        // one role at 16-bit d <= 64: the chunk loop unrolled by the ring depth,
        // each copy reading a fixed stage, so every LDS operand address is a
        // loop-invariant per-lane base plus an instruction offset (no address
        // arithmetic per chunk); otherwise the same steps as the loop below
        int c = 0;
        while (c < nchunks) {
          static_for<C::NSTAGE>([&](auto SC) {
            constexpr int S = decltype(SC)::value;
            if (c >= nchunks) return;
            const int ahead = nchunks - 1 - c;
            wait_ring<C::LPT + 1>(ahead < C::NSTAGE - 2 ? ahead : C::NSTAGE - 2);
            lds_barrier();
            if (c + C::NSTAGE - 1 < nchunks) issue();
            const int4 meta = s_meta[cx];
            const int ch = cch;
            const int kind = meta.y;
            const float gt = __int_as_float(meta.z);
            const int64_t i = meta.x;
            if (++cch == C::NCH) {
              cch = 0;
              if (++cg == a.grp) { cg = 0; ++cx; }
            }
            int tmin = -(1 << 30);
            bool kok = true;
            if (kind == KIND_DIAG) tmin = u;
            else if (kind == KIND_PAD) kok = keyok;
            else if (kind == KIND_ABS) {
              const int64_t tm = (int64_t)u - (i - j) * BS;
              tmin = (int)(tm < -(1 << 30) ? -(1 << 30) : tm);
              kok = keyok;
            }
            tmin -= ch * C::KC + 4 * g;  // compare against 16m + r
            static_for<C::KC / HR>([&](auto HC) {
              constexpr int h = decltype(HC)::value;
              constexpr int QOFF = S * C::STAGE_BYTES + h * HR * C::CPR * 16, DOFF = QOFF + C::TILE_BYTES;
              const float *Mh = (const float *)(stages + S * C::STAGE_BYTES + 2 * C::TILE_BYTES) + 2 * h * HR;
              const int th = tmin - h * HR;
              // dP accumulators start at -delta: dS = P (dP - delta) is then one product
              f32x4 sacc[HR / 16], dpacc[HR / 16], dinit[HR / 16];
#pragma unroll
              for (int m = 0; m < HR / 16; ++m)
#pragma unroll
                for (int r = 0; r < 4; ++r) dinit[m][r] = rs_delta(Mh, 4 * m + g, r);
              mm_rows_frag<T, D, HR / 16, 0, QOFF>(stages, kf, sacc, g, p);          // S: query 16m+4g+r, key u
              mm_rows_frag<T, D, HR / 16, 0, DOFF>(stages, vf, dpacc, g, p, dinit);  // dP - delta
              float pp[HR / 16][4], ds[HR / 16][4];
#pragma unroll
              for (int m = 0; m < HR / 16; ++m)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                  const float ml = rs_lse(Mh, 4 * m + g, r);  // -lse log2 e
                  const float ev = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[m][r], a.scale2, GC ? gt + ml : ml));
                  pp[m][r] = ev;
                  ds[m][r] = ev * dpacc[m][r];
                }
              if (kind != KIND_FULL) {
#pragma unroll
                for (int m = 0; m < HR / 16; ++m)
#pragma unroll
                  for (int r = 0; r < 4; ++r)
                    if (!(kok && (16 * m + r >= th))) { pp[m][r] = 0.f; ds[m][r] = 0.f; }
              }
              constexpr bool SP = decltype(SPC)::value;
              mm_tr_acc<T, D, HR, 0, SP, 1, DOFF>(stages, pp, dvacc, g, p);  // dV^T += dO^T P
              mm_tr_acc<T, D, HR, 0, SP, 1, QOFF>(stages, ds, dkacc, g, p);  // dK^T += Q^T dS
            });
            ++c;
          });
        }
        continue;
      }
      for (int c = 0; c < nchunks; ++c) {
        // stage c has landed for this wave (LPT + 1 loads per stage; up to NSTAGE - 2 later
        // stages may still be in flight); after the barrier every wave's part has landed and
        // every wave is done with chunk c - 1, whose stage the refill below overwrites
        const int ahead = nchunks - 1 - c;
        wait_ring<C::LPT + 1>(ahead < C::NSTAGE - 2 ? ahead : C::NSTAGE - 2);
        lds_barrier();
        if (c + C::NSTAGE - 1 < nchunks) issue();

        const char *Qs = stages + cstg * C::STAGE_BYTES;
        const char *Ds = Qs + C::TILE_BYTES;
        const float *Ms = (const float *)(Qs + 2 * C::TILE_BYTES);
        const int4 meta = s_meta[cx];
        const int ch = cch;
        const int kind = meta.y;
        const float gt = __int_as_float(meta.z);
        const int64_t i = meta.x;
        if (++cch == C::NCH) {
          cch = 0;
          if (++cg == a.grp) { cg = 0; ++cx; }
        }
        if (++cstg == C::NSTAGE) cstg = 0;

        // valid iff query row (within block i) >= tmin, and the key is in range
        int tmin = -(1 << 30);
        bool kok = true;
        if (kind == KIND_DIAG) tmin = u;
        else if (kind == KIND_PAD) kok = keyok;
        else if (kind == KIND_ABS) {
          const int64_t tm = (int64_t)u - (i - j) * BS;
          tmin = (int)(tm < -(1 << 30) ? -(1 << 30) : tm);
          kok = keyok;
        }
        tmin -= ch * C::KC + 4 * g;  // compare against 16m + r

        // the chunk's query rows in parts of HR (32) rows, one after the other:
        // the per-part S, dP, P, dS and row statistics stay in few registers
        // (unrolled at d <= 64: the parts' LDS addresses become instruction offsets)
        constexpr int HUNROLL = D <= 64 ? 2 : 1;
  #pragma unroll HUNROLL
        for (int h = 0; h < C::KC / HR; ++h) {
          const char *Qh = Qs + h * HR * C::CPR * 16, *Dh = Ds + h * HR * C::CPR * 16;
          const float *Mh = Ms + 2 * h * HR;  // 8 bytes a row
          const int th = tmin - h * HR;
          if constexpr (ROLES == 2) {
            f32x4 xacc[HR / 16];
            mm_rows_frag<T, D, HR / 16, (D >= 128 ? FBSA_DKDV_WIN : 0)>(role ? Dh : Qh, kf, xacc, g, p);  // role 0: S, role 1: dP
            // element m of this lane at s_xch[(m * KEYS/16 + kw) * 64 + lane]: a wave's
            // 16-byte accesses are consecutive, on distinct banks
            float4 *xs = s_xch + kw * 64 + lane;
            constexpr int XS = (KEYS / 16) * 64;  // stride between the parts m
            float x[HR / 16][4];
            if (role == 0) {
  #pragma unroll
              for (int m = 0; m < HR / 16; ++m) {
  #pragma unroll
                for (int r = 0; r < 4; ++r) {
                  const float ml = rs_lse(Mh, 4 * m + g, r);
                  const bool ok = kok && (16 * m + r >= th);
                  float ev = __builtin_amdgcn_exp2f(__builtin_fmaf(xacc[m][r], a.scale2, GC ? gt + ml : ml));
                  asm volatile("" : "+v"(ev));
                  x[m][r] = ok ? ev : 0.f;
                }
                xs[m * XS] = make_float4(x[m][0], x[m][1], x[m][2], x[m][3]);
              }
            }
            lds_barrier();  // P of this part is in LDS for the role-1 waves
            if (role == 0) {
              tr_acc(SPC, Dh, x, dvacc);  // dV^T += dO^T P
            } else {
  #pragma unroll
              for (int m = 0; m < HR / 16; ++m) {
                const float4 pv = xs[m * XS];
                const float pr[4] = {pv.x, pv.y, pv.z, pv.w};
  #pragma unroll
                for (int r = 0; r < 4; ++r) x[m][r] = pr[r] * (xacc[m][r] + rs_delta(Mh, 4 * m + g, r));
              }
              tr_acc(SPC, Qh, x, dvacc);  // dK^T += Q^T dS
            }
            continue;
          }
          // dP accumulators start at -delta: dS = P (dP - delta) is then one product
          f32x4 sacc[HR / 16], dpacc[HR / 16], dinit[HR / 16];
  #pragma unroll
          for (int m = 0; m < HR / 16; ++m)
  #pragma unroll
            for (int r = 0; r < 4; ++r) dinit[m][r] = rs_delta(Mh, 4 * m + g, r);
          mm_rows_frag<T, D, HR / 16, (D >= 128 ? FBSA_DKDV_WIN : 0)>(Qh, kf, sacc, g, p);  // S: query 16m+4g+r, key u
          mm_rows_frag<T, D, HR / 16, (D >= 128 ? FBSA_DKDV_WIN : 0)>(Dh, vf, dpacc, g, p, dinit);  // dP - delta
          float pp[HR / 16][4], ds[HR / 16][4];
          // every exponential is computed unconditionally; masked elements of
          // a masked chunk kind are then replaced by zeros in one uniform branch
          // (unmasked chunks, the common case, skip the compares)
  #pragma unroll
          for (int m = 0; m < HR / 16; ++m)
  #pragma unroll
            for (int r = 0; r < 4; ++r) {
              const float ml = rs_lse(Mh, 4 * m + g, r);  // -lse log2 e
              const float ev = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[m][r], a.scale2, GC ? gt + ml : ml));
              pp[m][r] = ev;
              ds[m][r] = ev * dpacc[m][r];
            }
          if (kind != KIND_FULL) {
  #pragma unroll
            for (int m = 0; m < HR / 16; ++m)
  #pragma unroll
              for (int r = 0; r < 4; ++r)
                if (!(kok && (16 * m + r >= th))) { pp[m][r] = 0.f; ds[m][r] = 0.f; }
          }
          tr_acc(SPC, Dh, pp, dvacc);  // dV^T += dO^T P
          tr_acc(SPC, Qh, ds, dkacc);  // dK^T += Q^T dS
        }
      }
    }
  };
  auto walk_g = [&](auto SPC) {
    if (a.gate) walk(SPC, std::true_type{});
    else walk(SPC, std::false_type{});
  };
  if constexpr (SPLIT) {
    if (split) walk_g(std::true_type{});
    else walk_g(std::false_type{});
  } else {
    walk_g(std::false_type{});
  }

  if (slot >= 0) {  // one segment of a split list: fp32 partials, summed by dkdv_reduce_kernel
    float *pk = a.partials + ((int64_t)slot * 2 * BS + u) * D;  // dK rows, then dV rows
    float *pv = pk + (int64_t)BS * D;
#pragma unroll
    for (int mt = 0; mt < D / 16; ++mt) {
      const int d0 = 16 * mt + 4 * g;
      if constexpr (ROLES == 2) {
        *(f32x4 *)((role ? pk : pv) + d0) = dvacc[mt];
      } else {
        *(f32x4 *)(pk + d0) = dkacc[mt];
        *(f32x4 *)(pv + d0) = dvacc[mt];
      }
    }
    return;
  }
  if constexpr (ROLES == 2) {
    T *row = (T *)(role ? a.dk : a.dv) + ((b * a.Hkv + hk) * a.L + kpos) * D;
    const float sc = role ? a.scale : 1.f;
#pragma unroll
    for (int mt = 0; mt < D / 16; ++mt) {
      s16x4 pk;
#pragma unroll
      for (int r = 0; r < 4; ++r) pk[r] = bits16<T>((T)(dvacc[mt][r] * sc));
      *(s16x4 *)(row + 16 * mt + 4 * g) = pk;
    }
    return;
  }
  T *dkrow = (T *)a.dk + ((b * a.Hkv + hk) * a.L + kpos) * D;
  T *dvrow = (T *)a.dv + ((b * a.Hkv + hk) * a.L + kpos) * D;
#pragma unroll
  for (int mt = 0; mt < D / 16; ++mt) {
    const int d0 = 16 * mt + 4 * g;
    if constexpr (sizeof(T) == 4) {
      *(f32x4 *)(dkrow + d0) = f32x4{dkacc[mt][0] * a.scale, dkacc[mt][1] * a.scale, dkacc[mt][2] * a.scale,
                                     dkacc[mt][3] * a.scale};
      *(f32x4 *)(dvrow + d0) = dvacc[mt];
    } else {
      s16x4 pk, pv;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        pk[r] = bits16<T>((T)(dkacc[mt][r] * a.scale));
        pv[r] = bits16<T>((T)dvacc[mt][r]);
      }
      *(s16x4 *)(dkrow + d0) = pk;
      *(s16x4 *)(dvrow + d0) = pv;
    }
  }
}

// List segments. Work item wi = (b, KV head, key block) walks the transposed
// list of its selection head; longer than E entries it is cut into
// S = ceil(len / E) segments. cnt[wi] = (S - 1) << 32 | S for a split item, 0
// otherwise, and cnt[nwi] = 0, so that an exclusive scan gives each item's first
// extra segment and first partial slot (high / low halves) and their totals.
__global__ __launch_bounds__(256) void seg_count_kernel(const int32_t *seg_off, int64_t nwi, int64_t nblk, int64_t Hkv,
                                                        int64_t hsel, int64_t E, uint64_t *cnt) {
  const int64_t wi = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (wi > nwi) return;
  uint64_t c = 0;
  if (wi < nwi) {
    const int64_t j = wi % nblk, hk = (wi / nblk) % Hkv, b = wi / (nblk * Hkv);
    const int64_t seg = (b * hsel + (hsel == 1 ? 0 : hk)) * nblk + j;
    const int64_t len = seg_off[seg + 1] - seg_off[seg];
    if (len > E) {
      const uint64_t S = (uint64_t)((len + E - 1) / E);
      c = ((S - 1) << 32) | S;
    }
  }
  cnt[wi] = c;
}

// From the scanned counts: each work item's first partial slot (-1 when not
// split) and the table rows of its extra segments 1 .. S-1.
__global__ __launch_bounds__(256) void seg_table_kernel(const int32_t *seg_off, const uint64_t *pos, int64_t nwi,
                                                        int64_t nblk, int64_t Hkv, int64_t hsel, int64_t E,
                                                        int32_t *wi_slot, int4 *xtab) {
  const int64_t wi = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (wi >= nwi) return;
  const uint64_t p0 = pos[wi], p1 = pos[wi + 1];
  const int ns = (int)((p1 - p0) & 0xffffffffu);
  if (ns == 0) {
    wi_slot[wi] = -1;
    return;
  }
  const int slot0 = (int)(p0 & 0xffffffffu), x0 = (int)(p0 >> 32);
  wi_slot[wi] = slot0;
  const int64_t j = wi % nblk, hk = (wi / nblk) % Hkv, b = wi / (nblk * Hkv);
  const int64_t seg = (b * hsel + (hsel == 1 ? 0 : hk)) * nblk + j;
  const int e0 = seg_off[seg], e1 = seg_off[seg + 1];
  for (int s = 1; s < ns; ++s) {
    const int a0 = e0 + s * (int)E, a1 = e1 - a0 < (int)E ? e1 : a0 + (int)E;
    xtab[x0 + s - 1] = int4{(int)wi, a0, a1, slot0 + s};
  }
}

// dK, dV of a split work item: its S partials summed in segment order.
template <typename T>
__global__ __launch_bounds__(256) void dkdv_reduce_kernel(const int32_t *wi_slot, const uint64_t *pos,
                                                          const float *partials, void *dk, void *dv, int64_t nblk,
                                                          int64_t Hkv, int64_t L, int64_t bs, int64_t D, float scale) {
  // grid: x = work item, y = a slice of RG * 2048 of its 2 bs D elements (RG
  // 8-element groups per thread, 256 threads), so that a block split into many
  // segments is summed by several workgroups with many loads in flight, while an
  // unsplit item (most of them when lists are short) costs few empty workgroups
  constexpr int RG = 4;
  const int64_t wi = blockIdx.x;
  const int slot0 = wi_slot[wi];
  if (slot0 < 0) return;
  const int64_t n = bs * D;  // a multiple of 8: an 8-element group lies in dK or in dV
  const int ns = (int)((pos[wi + 1] - pos[wi]) & 0xffffffffu);
  const int64_t j = wi % nblk, hk = (wi / nblk) % Hkv, b = wi / (nblk * Hkv);
  int64_t xs[RG];
  float acc[RG][8];
#pragma unroll
  for (int gq = 0; gq < RG; ++gq) {
    xs[gq] = 8 * (((int64_t)blockIdx.y * RG + gq) * 256 + threadIdx.x);
#pragma unroll
    for (int r = 0; r < 8; ++r) acc[gq][r] = 0.f;
  }
#pragma unroll 2
  for (int s = 0; s < ns; ++s) {
    const float *seg = partials + (int64_t)(slot0 + s) * 2 * n;  // dK rows, then dV rows
#pragma unroll
    for (int gq = 0; gq < RG; ++gq) {
      if (xs[gq] < 2 * n) {
        const f32x4 p0 = *(const f32x4 *)(seg + xs[gq]), p1 = *(const f32x4 *)(seg + xs[gq] + 4);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          acc[gq][r] += p0[r];
          acc[gq][4 + r] += p1[r];
        }
      }
    }
  }
#pragma unroll
  for (int gq = 0; gq < RG; ++gq) {
    const int64_t x = xs[gq];
    if (x >= 2 * n) continue;
    const int which = x >= n;  // 0: dK, 1: dV
    const int64_t e = x - which * n;
    const float sc = which ? 1.f : scale;
    float y[8];
#pragma unroll
    for (int r = 0; r < 8; ++r) y[r] = acc[gq][r] * sc;
    T *dst = (T *)(which ? dv : dk) + ((b * Hkv + hk) * L + j * bs) * D + e;  // 16-byte aligned
    if constexpr (sizeof(T) == 4) {
      *(f32x4 *)dst = f32x4{y[0], y[1], y[2], y[3]};
      *(f32x4 *)(dst + 4) = f32x4{y[4], y[5], y[6], y[7]};
    } else {
      *(s16x8 *)dst = pack8<T>(y);
    }
  }
}

// dgate[b, hs, i, s] = sum over the heads sharing selection hs (fixed order)
__global__ __launch_bounds__(256) void dgate_reduce_kernel(const float *part, float *dgate, int64_t n, int64_t Hq,
                                                           int64_t hsel, int64_t nblk, int64_t kk, int64_t grp) {
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (e >= n) return;
  const int64_t s = e % kk, i = (e / kk) % nblk, hs = (e / (kk * nblk)) % hsel, b = e / (kk * nblk * hsel);
  const int64_t h0 = hsel == 1 ? 0 : hs * grp, nh = hsel == 1 ? Hq : grp;
  float acc = 0.f;
  for (int64_t h = h0; h < h0 + nh; ++h) acc += part[((b * Hq + h) * nblk + i) * kk + s];
  dgate[e] = acc;
}

static void fill_bwd(const fbsa_attn_desc *d, const BwdLayout &lay, char *ws, BwdArgs &a, const void *dout) {
  a.wi_slot = nullptr; a.xtab = nullptr; a.seg_tot = nullptr; a.partials = nullptr;
  a.o = nullptr; a.lse = nullptr;
  for (int x = 0; x < 3; ++x) a.so[x] = d->so[x];
  a.seg_entries = a.seg_entries_xub = 0;
  a.B = d->B; a.Hq = d->Hq; a.Hkv = d->Hkv; a.L = d->L; a.nblk = d->nblk; a.kk = d->kk; a.hsel = d->hsel;
  a.l_valid = d->l_valid;
  for (int x = 0; x < 3; ++x) { a.sq[x] = d->sq[x]; a.sk[x] = d->sk[x]; a.sv[x] = d->sv[x]; a.sdo[x] = d->sdo[x]; }
  if (d->flags & FBSA_FLAG_OUT_GATE) {
    a.dout = ws + lay.dout_attn;
    a.sdo[0] = d->Hq * d->L * d->D; a.sdo[1] = d->L * d->D; a.sdo[2] = d->D;
  } else {
    a.dout = dout;
  }
  a.rowstat = (float *)(ws + lay.rowstat);
  a.seg_off = (const int32_t *)(ws + lay.seg_off);
  a.ent = (const int32_t *)(ws + lay.vals_out);
  a.scale = d->scale;
  a.scale2 = d->scale * kLog2e;
  a.mask = d->mask;
  a.grp = (int)(d->Hq / d->Hkv);
  a.dense = (d->flags & FBSA_FLAG_DENSE) ? 1 : 0;
  if (a.dense) a.ent = nullptr;
}

template <typename K> static int set_lds(K kern, size_t lds, const char *what) {
  if (lds > 160 * 1024 - 64) return fail(FBSA_EUNSUPPORTED, "%s needs %zu bytes of LDS", what, lds);
  return lds_optin((const void *)kern, lds, "hipFuncSetAttribute(bwd)");
}

template <typename T, int BS, int D, bool DENSE, bool DG> static int launch_dq_as(const BwdArgs &a, hipStream_t s) {
  using C = BwdCfg<T, BS, D, FBSA_DQ_LDS_BUDGET, 0>;
  // slot tables (block, kind, gate: 12 bytes per slot; with the gate gradient
  // also each entry's selection slot) and the gate gradient's per-wave and
  // per-row scratch
  const size_t lds = (size_t)C::NSTAGE * C::STAGE_BYTES +
                     (DENSE ? 0 : (size_t)a.kk * (DG ? 16 : 12) + (DG ? (2 * C::NW + BS) * 4 : 0));
  int e = set_lds(dq_kernel<T, BS, D, DENSE, DG>, lds, "fbsa_bwd_dq");
  if (e) return e;
  hipLaunchKernelGGL((dq_kernel<T, BS, D, DENSE, DG>), dim3((unsigned)(a.B * a.Hq * a.nblk)), dim3(C::NT), lds, s, a);
  return hip_check(hipGetLastError(), "dq_kernel launch");
}

template <typename T, int BS, int D, bool DENSE> static int launch_dkdv_as(const BwdArgs &a, hipStream_t s) {
  using C = DkdvCfg<T, BS, D>;
  constexpr int HR = C::KC >= 64 ? 32 : C::KC;
  const size_t xch = dkdv_roles<T, D>() == 2
                         ? (size_t)(dkdv_pipe<T, BS, D>() ? 2 : 1) * (dkdv_keys<T, BS, D>() / 16) * 64 * (HR / 16) * 16
                         : 0;
  const size_t lds = (size_t)C::NSTAGE * C::STAGE_BYTES + 128 * 16 + xch;
  int e = set_lds(dkdv_kernel<T, BS, D, DENSE>, lds, "fbsa_bwd_dkdv");
  if (e) return e;
  const int64_t nwg = (a.B * a.Hkv * a.nblk + (a.wi_slot ? a.seg_entries_xub : 0)) * (BS / dkdv_keys<T, BS, D>());
  hipLaunchKernelGGL((dkdv_kernel<T, BS, D, DENSE>), dim3((unsigned)nwg), dim3(C::NT), lds, s, a);
  return hip_check(hipGetLastError(), "dkdv_kernel launch");
}

// the dense (list-less) forms are their own instantiations (the list path's
// code is unchanged by them)
template <typename T, int BS, int D> static int launch_dq(const BwdArgs &a, hipStream_t s) {
  if (a.dense) return launch_dq_as<T, BS, D, true, false>(a, s);  // dense lists carry no gate
  return a.dgate_part ? launch_dq_as<T, BS, D, false, true>(a, s) : launch_dq_as<T, BS, D, false, false>(a, s);
}
template <typename T, int BS, int D> static int launch_dkdv(const BwdArgs &a, hipStream_t s) {
  return a.dense ? launch_dkdv_as<T, BS, D, true>(a, s) : launch_dkdv_as<T, BS, D, false>(a, s);
}

template <typename T, int BS> static int bwd_d(const BwdArgs &a, int64_t D, bool dq, hipStream_t s) {
  switch (D) {
    case 32: return dq ? launch_dq<T, BS, 32>(a, s) : launch_dkdv<T, BS, 32>(a, s);
    case 64: return dq ? launch_dq<T, BS, 64>(a, s) : launch_dkdv<T, BS, 64>(a, s);
    case 128: return dq ? launch_dq<T, BS, 128>(a, s) : launch_dkdv<T, BS, 128>(a, s);
    case 256: return dq ? launch_dq<T, BS, 256>(a, s) : launch_dkdv<T, BS, 256>(a, s);
  }
  return fail(FBSA_EUNSUPPORTED, "fbsa_bwd: head dim %lld not in {32,64,128,256}", (long long)D);
}

template <typename T> static int bwd_bs(const BwdArgs &a, int64_t bs, int64_t D, bool dq, hipStream_t s) {
  switch (bs) {
    case 16: return bwd_d<T, 16>(a, D, dq, s);
    case 32: return bwd_d<T, 32>(a, D, dq, s);
    case 64: return bwd_d<T, 64>(a, D, dq, s);
    case 128: return bwd_d<T, 128>(a, D, dq, s);
  }
  return fail(FBSA_EUNSUPPORTED, "fbsa_bwd: block size %lld not in {16,32,64,128}", (long long)bs);
}

static int bwd_dispatch(const fbsa_attn_desc *d, const BwdArgs &a, bool dq, hipStream_t s) {
  switch (d->dtype) {
    case FBSA_BF16: return bwd_bs<bf16>(a, d->bs, d->D, dq, s);
    case FBSA_F16: return bwd_bs<f16>(a, d->bs, d->D, dq, s);
    case FBSA_F32: return bwd_bs<float>(a, d->bs, d->D, dq, s);
  }
  return fail(FBSA_EINVAL, "fbsa_bwd: bad dtype %d", d->dtype);
}

int run_bwd_dq(const fbsa_attn_desc *d, const BwdLayout &lay, const void *q, const void *k, const void *v,
               const void *dout, const int32_t *sel, const float *gate, void *dq, float *dgate, char *ws,
               hipStream_t s, const void *o, const float *lse) {
  BwdArgs a;
  fill_bwd(d, lay, ws, a, dout);
  a.o = o; a.lse = lse;
  a.q = q; a.k = k; a.v = v; a.sel = sel; a.gate = gate; a.dq = dq; a.dk = a.dv = nullptr;
  a.dgate_part = dgate ? (float *)(ws + lay.dgate_part) : nullptr;
  a.pmass = (float *)(ws + lay.pmass);
  int e = bwd_dispatch(d, a, true, s);
  if (e || !dgate) return e;
  const int64_t n = d->B * d->hsel * d->nblk * d->kk;
  hipLaunchKernelGGL(dgate_reduce_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s,
                     (const float *)(ws + lay.dgate_part), dgate, n, d->Hq, d->hsel, d->nblk, d->kk,
                     d->Hq / d->Hkv);
  return hip_check(hipGetLastError(), "dgate_reduce_kernel launch");
}

// The segment tables of lists walked in segments (from the transposed index
// alone): run by run_bwd_dkdv, or earlier on another stream (segments_done).
int run_bwd_segments(const fbsa_attn_desc *d, const BwdLayout &lay, char *ws, hipStream_t s) {
  int e = FBSA_OK;
  if (lay.seg_entries) {
    uint64_t *cnt = (uint64_t *)(ws + lay.seg_cnt), *pos = (uint64_t *)(ws + lay.seg_pos);
    hipLaunchKernelGGL(seg_count_kernel, dim3((unsigned)((lay.nwi + 1 + 255) / 256)), dim3(256), 0, s,
                       (const int32_t *)(ws + lay.seg_off), lay.nwi, d->nblk, d->Hkv, d->hsel, lay.seg_entries, cnt);
    if ((e = hip_check(hipGetLastError(), "seg_count_kernel launch"))) return e;
    size_t tmp = lay.scan_tmp_bytes;
    if ((e = hip_check(rocprim::exclusive_scan(ws + lay.scan_tmp, tmp, (const uint64_t *)cnt, pos, (uint64_t)0,
                                               (size_t)(lay.nwi + 1), rocprim::plus<uint64_t>(), s),
                       "scan of the list segments")))
      return e;
    hipLaunchKernelGGL(seg_table_kernel, dim3((unsigned)((lay.nwi + 255) / 256)), dim3(256), 0, s,
                       (const int32_t *)(ws + lay.seg_off), (const uint64_t *)pos, lay.nwi, d->nblk, d->Hkv, d->hsel,
                       lay.seg_entries, (int32_t *)(ws + lay.wi_slot), (int4 *)(ws + lay.xtab));
    e = hip_check(hipGetLastError(), "seg_table_kernel launch");
  }
  return e;
}

int run_bwd_dkdv(const fbsa_attn_desc *d, const BwdLayout &lay, const void *q, const void *k, const void *v,
                 const void *dout, const float *gate, void *dk, void *dv, char *ws, hipStream_t s, bool segments_done) {
  BwdArgs a;
  fill_bwd(d, lay, ws, a, dout);
  a.q = q; a.k = k; a.v = v; a.sel = nullptr; a.gate = gate; a.dq = nullptr; a.dk = dk; a.dv = dv;
  a.dgate_part = nullptr;
  int e;
  if (!segments_done && (e = run_bwd_segments(d, lay, ws, s))) return e;
  if (lay.seg_entries) {
    uint64_t *pos = (uint64_t *)(ws + lay.seg_pos);
    a.wi_slot = (const int32_t *)(ws + lay.wi_slot);
    a.xtab = (const int4 *)(ws + lay.xtab);
    a.seg_tot = pos + lay.nwi;
    a.partials = (float *)(ws + lay.partials);
    a.seg_entries = lay.seg_entries;
    a.seg_entries_xub = lay.xub;
  }
  if ((e = bwd_dispatch(d, a, false, s)) || !lay.seg_entries) return e;
  const dim3 g((unsigned)lay.nwi, (unsigned)((2 * d->bs * d->D + 4 * 8 * 256 - 1) / (4 * 8 * 256))), blk(256);
  const uint64_t *pos = (const uint64_t *)(ws + lay.seg_pos);
  const float *part = (const float *)(ws + lay.partials);
  const int32_t *wsl = (const int32_t *)(ws + lay.wi_slot);
  switch (d->dtype) {
    case FBSA_BF16:
      hipLaunchKernelGGL(dkdv_reduce_kernel<bf16>, g, blk, 0, s, wsl, pos, part, dk, dv, d->nblk, d->Hkv, d->L, d->bs,
                         d->D, d->scale);
      break;
    case FBSA_F16:
      hipLaunchKernelGGL(dkdv_reduce_kernel<f16>, g, blk, 0, s, wsl, pos, part, dk, dv, d->nblk, d->Hkv, d->L, d->bs,
                         d->D, d->scale);
      break;
    default:
      hipLaunchKernelGGL(dkdv_reduce_kernel<float>, g, blk, 0, s, wsl, pos, part, dk, dv, d->nblk, d->Hkv, d->L, d->bs,
                         d->D, d->scale);
  }
  return hip_check(hipGetLastError(), "dkdv_reduce_kernel launch");
}

}  // namespace fbsa
