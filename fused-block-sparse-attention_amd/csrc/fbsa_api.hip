// C ABI layer: host-side validation, error reporting and dispatch.
#include <stdarg.h>
#include <stdio.h>
#include <math.h>

#include <map>
#include <mutex>
#include <utility>

#include "fbsa_common.h"
#include "fbsa_internal.h"

namespace fbsa {

static thread_local char g_err[1024] = "";

int fail(int code, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof g_err, fmt, ap);
  va_end(ap);
  return code;
}

int hip_check(hipError_t e, const char *what) {
  if (e == hipSuccess) return FBSA_OK;
  (void)hipGetLastError();  // clear the sticky per-thread error so later calls are not blamed
  return fail(FBSA_EHIP, "%s: %s", what, hipGetErrorString(e));
}

int lds_optin(const void *fn, size_t bytes, const char *what) {
  if (bytes <= 64 * 1024) return FBSA_OK;
  int dev = 0;
  int e = hip_check(hipGetDevice(&dev), "hipGetDevice");
  if (e) return e;
  // grants per (device, kernel); a mutex because autograd runs the backward on
  // its own device thread while other host threads may launch
  static std::mutex mu;
  static std::map<std::pair<int, const void *>, size_t> granted;
  std::lock_guard<std::mutex> lock(mu);
  size_t &g = granted[std::make_pair(dev, fn)];
  if (bytes <= g) return FBSA_OK;
  e = hip_check(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes), what);
  if (e) return e;
  g = bytes;
  return FBSA_OK;
}

static int64_t esize(int dtype) { return dtype == FBSA_F32 ? 4 : 2; }

static bool aligned(const void *p, int64_t a) { return ((uintptr_t)p % (uintptr_t)a) == 0; }

// Shape and layout checks shared by the attention entry points.
static int check_attn(const fbsa_attn_desc *d, const char *fn) {
  if (!d) return fail(FBSA_EINVAL, "%s: null descriptor", fn);
  if (d->dtype < FBSA_F32 || d->dtype > FBSA_F16) return fail(FBSA_EINVAL, "%s: bad dtype %d", fn, d->dtype);
  if (d->mask < FBSA_MASK_NONE || d->mask > FBSA_MASK_TOKEN_CAUSAL) return fail(FBSA_EINVAL, "%s: bad mask %d", fn, d->mask);
  if (d->B < 1 || d->Hq < 1 || d->Hkv < 1 || d->L < 1 || d->nblk < 1 || d->kk < 1)
    return fail(FBSA_EINVAL, "%s: sizes must be positive (B=%lld Hq=%lld Hkv=%lld L=%lld nblk=%lld kk=%lld)", fn,
                (long long)d->B, (long long)d->Hq, (long long)d->Hkv, (long long)d->L, (long long)d->nblk, (long long)d->kk);
  if (d->Hq % d->Hkv) return fail(FBSA_EINVAL, "%s: Hq=%lld not a multiple of Hkv=%lld", fn, (long long)d->Hq, (long long)d->Hkv);
  if (d->bs != 16 && d->bs != 32 && d->bs != 64 && d->bs != 128)
    return fail(FBSA_EUNSUPPORTED, "%s: block size %lld not in {16,32,64,128}", fn, (long long)d->bs);
  if (d->D != 32 && d->D != 64 && d->D != 128 && d->D != 256)
    return fail(FBSA_EUNSUPPORTED, "%s: head dim %lld not in {32,64,128,256}", fn, (long long)d->D);
  if (d->L != d->nblk * d->bs)
    return fail(FBSA_EINVAL, "%s: L=%lld must equal nblk*bs=%lld", fn, (long long)d->L, (long long)(d->nblk * d->bs));
  if (d->hsel != 1 && d->hsel != d->Hkv) return fail(FBSA_EINVAL, "%s: hsel=%lld must be 1 or Hkv", fn, (long long)d->hsel);
  if (d->l_valid < 1 || d->l_valid > d->L) return fail(FBSA_EINVAL, "%s: l_valid=%lld outside [1, L]", fn, (long long)d->l_valid);
  if (!isfinite(d->scale)) return fail(FBSA_EINVAL, "%s: scale is not finite", fn);
  if (d->B * d->Hq * d->nblk > 0x7fffffffLL) return fail(FBSA_EUNSUPPORTED, "%s: B*Hq*nblk exceeds the grid limit", fn);
  const int64_t es = esize(d->dtype);
  const int64_t *st[4] = {d->sq, d->sk, d->sv, d->so};
  const char *nm[4] = {"q", "k", "v", "o"};
  for (int t = 0; t < 4; ++t)
    for (int x = 0; x < 3; ++x)
      if (st[t][x] < 0 || (st[t][x] * es) % 16)
        return fail(FBSA_EINVAL, "%s: %s stride[%d]=%lld must be a non-negative multiple of 16 bytes", fn, nm[t], x,
                    (long long)st[t][x]);
  // the kernels form row offsets as 32 x 32 -> 64-bit products
  if (d->L >= 0x80000000LL) return fail(FBSA_EUNSUPPORTED, "%s: L=%lld must be below 2^31", fn, (long long)d->L);
  const int64_t rs[5] = {d->sq[2], d->sk[2], d->sv[2], d->so[2], d->sdo[2]};
  for (int t = 0; t < 5; ++t)
    if (rs[t] * es >= 0x100000000LL)
      return fail(FBSA_EUNSUPPORTED, "%s: a row stride of %lld elements is 4 GiB or more", fn, (long long)rs[t]);
  return FBSA_OK;
}

// FBSA_FLAG_DENSE: the implicit all-blocks list (kk = nblk, no sel, no gate).
static int check_dense(const fbsa_attn_desc *d, const void *sel, const void *gate, const char *fn) {
  if (!(d->flags & FBSA_FLAG_DENSE)) {
    if (!sel) return fail(FBSA_EINVAL, "%s: sel is NULL (only FBSA_FLAG_DENSE selects without a list)", fn);
    return FBSA_OK;
  }
  if (d->kk != d->nblk) return fail(FBSA_EINVAL, "%s: FBSA_FLAG_DENSE needs kk == nblk (kk=%lld, nblk=%lld)", fn,
                                    (long long)d->kk, (long long)d->nblk);
  if (d->mask == FBSA_MASK_SLOT_CAUSAL)
    return fail(FBSA_EINVAL, "%s: FBSA_FLAG_DENSE takes FBSA_MASK_TOKEN_CAUSAL or FBSA_MASK_NONE", fn);
  if (gate) return fail(FBSA_EINVAL, "%s: FBSA_FLAG_DENSE takes no gate", fn);
  return FBSA_OK;
}

static void fill_fwd(const fbsa_attn_desc *d, FwdArgs &a) {
  a.B = d->B; a.Hq = d->Hq; a.Hkv = d->Hkv; a.L = d->L; a.nblk = d->nblk; a.kk = d->kk; a.hsel = d->hsel;
  a.l_valid = d->l_valid;
  for (int x = 0; x < 3; ++x) {
    a.sq[x] = d->sq[x]; a.sk[x] = d->sk[x]; a.sv[x] = d->sv[x]; a.so[x] = d->so[x]; a.sog[x] = d->sog[x];
  }
  a.scale2 = d->scale * kLog2e;
  a.mask = d->mask;
  a.grp = (int)(d->Hq / d->Hkv);
  a.dense = (d->flags & FBSA_FLAG_DENSE) ? 1 : 0;
}

}  // namespace fbsa

using namespace fbsa;

extern "C" {

const char *fbsa_last_error(void) { return g_err; }

int fbsa_version(void) { return 1; }

int fbsa_fwd(const fbsa_attn_desc *d, const void *q, const void *k, const void *v, const int32_t *sel,
             const float *gate, const void *out_gate, void *o, float *lse, void *stream) {
  if (!d) return fail(FBSA_EINVAL, "fbsa_fwd: null descriptor");
  return fbsa_fwd_rows(d, 0, d->nblk, q, k, v, sel, gate, out_gate, o, lse, stream);
}

int fbsa_fwd_rows(const fbsa_attn_desc *d, int64_t i_begin, int64_t i_end, const void *q, const void *k,
                  const void *v, const int32_t *sel, const float *gate, const void *out_gate, void *o, float *lse,
                  void *stream) {
  int e = check_attn(d, "fbsa_fwd");
  if (e) return e;
  if (i_begin < 0 || i_end < i_begin || i_end > d->nblk)
    return fail(FBSA_EINVAL, "fbsa_fwd: query-block range [%lld, %lld) outside [0, %lld)", (long long)i_begin,
                (long long)i_end, (long long)d->nblk);
  if (d->flags & ~FBSA_FLAG_DENSE) return fail(FBSA_EINVAL, "fbsa_fwd: unknown flags 0x%x", d->flags);
  if ((e = check_dense(d, sel, gate, "fbsa_fwd"))) return e;
  if (!q || !k || !v || !o) return fail(FBSA_EINVAL, "fbsa_fwd: null tensor pointer");
  if (!aligned(q, 16) || !aligned(k, 16) || !aligned(v, 16) || !aligned(o, 16))
    return fail(FBSA_EINVAL, "fbsa_fwd: q/k/v/o must be 16-byte aligned");
  if (!aligned(sel, 4) || (gate && !aligned(gate, 4)) || (lse && !aligned(lse, 4)))
    return fail(FBSA_EINVAL, "fbsa_fwd: sel/gate/lse must be 4-byte aligned");
  if (out_gate && !aligned(out_gate, esize(d->dtype)))
    return fail(FBSA_EINVAL, "fbsa_fwd: out_gate misaligned");
  FwdArgs a;
  fill_fwd(d, a);
  a.i0 = i_begin;
  a.ni = i_end - i_begin;
  a.q = q; a.k = k; a.v = v; a.o = o; a.lse = lse; a.sel = sel; a.gate = gate; a.og = out_gate;
  return run_fwd(d, a, (hipStream_t)stream);
}

size_t fbsa_block_mass_workspace_bytes(const fbsa_attn_desc *d) {
  return d ? (size_t)(d->B * d->Hq * d->L) * sizeof(float) : 0;
}

int fbsa_block_mass(const fbsa_attn_desc *d, const void *q, const void *k, float *mass, void *ws, void *stream) {
  int e = check_attn(d, "fbsa_block_mass");
  if (e) return e;
  if (d->dtype == FBSA_F32) return fail(FBSA_EUNSUPPORTED, "fbsa_block_mass: 16-bit operands only (bf16, f16)");
  if ((d->bs != 64 && d->bs != 128) || d->D < 64)
    return fail(FBSA_EUNSUPPORTED, "fbsa_block_mass: needs bs in {64, 128} and D in {64, 128, 256}");
  if (d->l_valid != d->L) return fail(FBSA_EINVAL, "fbsa_block_mass: L must be a whole number of blocks (l_valid = L)");
  if (!q || !k || !mass || !ws) return fail(FBSA_EINVAL, "fbsa_block_mass: null pointer");
  if (!aligned(q, 16) || !aligned(k, 16) || !aligned(mass, 4) || !aligned(ws, 16))
    return fail(FBSA_EINVAL, "fbsa_block_mass: misaligned pointer");
  return run_block_mass(d, q, k, mass, (float *)ws, (hipStream_t)stream);
}

static int check_pool(const fbsa_pool_desc *d, const void *x, const void *out, const void *out2) {
  if (!d) return fail(FBSA_EINVAL, "fbsa_pool: null descriptor");
  if (d->dtype < FBSA_F32 || d->dtype > FBSA_F16) return fail(FBSA_EINVAL, "fbsa_pool: bad dtype %d", d->dtype);
  if (d->op < FBSA_POOL_MEAN_TOK_THEN_GRP || d->op > FBSA_POOL_MINMAX) return fail(FBSA_EINVAL, "fbsa_pool: bad op %d", d->op);
  if (d->B < 1 || d->H < 1 || d->L < 1 || d->D < 8 || d->bs < 1 || d->nblk < 1 || d->grp < 1)
    return fail(FBSA_EINVAL, "fbsa_pool: sizes must be positive (D >= 8)");
  if (d->D % 8 || d->D > 2048) return fail(FBSA_EUNSUPPORTED, "fbsa_pool: D=%lld must be a multiple of 8 and <= 2048", (long long)d->D);
  if (d->H % d->grp) return fail(FBSA_EINVAL, "fbsa_pool: H=%lld not a multiple of grp=%lld", (long long)d->H, (long long)d->grp);
  if ((d->op >= FBSA_POOL_MAX) && d->grp != 1) return fail(FBSA_EINVAL, "fbsa_pool: min/max pooling needs grp == 1");
  if (d->nblk != (d->L + d->bs - 1) / d->bs) return fail(FBSA_EINVAL, "fbsa_pool: nblk must be ceil(L/bs)");
  if (d->l_valid < 1 || d->l_valid > d->L) return fail(FBSA_EINVAL, "fbsa_pool: l_valid outside [1, L]");
  if (!x || !out || (d->op == FBSA_POOL_MINMAX && !out2)) return fail(FBSA_EINVAL, "fbsa_pool: null pointer");
  const int64_t es = esize(d->dtype);
  if (!aligned(x, 16) || !aligned(out, es) || (out2 && !aligned(out2, es))) return fail(FBSA_EINVAL, "fbsa_pool: misaligned pointer");
  for (int k = 0; k < 3; ++k)
    if (d->sx[k] < 0 || (d->sx[k] * es) % 16) return fail(FBSA_EINVAL, "fbsa_pool: stride[%d] must be a non-negative multiple of 16 bytes", k);
  if (d->B * (d->H / d->grp) * d->nblk > 0x7fffffffLL) return fail(FBSA_EUNSUPPORTED, "fbsa_pool: grid too large");
  return FBSA_OK;
}

int fbsa_pool(const fbsa_pool_desc *d, const void *x, void *out, void *out2, void *stream) {
  const int e = check_pool(d, x, out, out2);
  return e ? e : run_pool(d, x, out, out2, (hipStream_t)stream);
}

size_t fbsa_select_workspace_bytes(const fbsa_select_desc *d) { return d ? select_workspace_bytes(d) : 0; }

int fbsa_select(const fbsa_select_desc *d, const void *a, const void *b1, const void *b2, int32_t *sel,
                float *sel_score, void *workspace, size_t workspace_bytes, void *stream) {
  if (!d) return fail(FBSA_EINVAL, "fbsa_select: null descriptor");
  return fbsa_select_rows(d, 0, d->nblk, a, b1, b2, sel, sel_score, workspace, workspace_bytes, stream);
}

// Argument checks of the selection entry points (no device work).
static int check_select(const fbsa_select_desc *d, int64_t row_begin, int64_t row_end, const void *a,
                        const void *b1, const void *b2, const int32_t *sel, const float *sel_score) {
  if (!d) return fail(FBSA_EINVAL, "fbsa_select: null descriptor");
  if (row_begin < 0 || row_end < row_begin || row_end > d->nblk)
    return fail(FBSA_EINVAL, "fbsa_select: row range [%lld, %lld) outside [0, %lld)", (long long)row_begin,
                (long long)row_end, (long long)d->nblk);
  if (d->dtype < FBSA_F32 || d->dtype > FBSA_F16) return fail(FBSA_EINVAL, "fbsa_select: bad dtype %d", d->dtype);
  if (d->score < FBSA_SCORE_DOT || d->score > FBSA_SCORE_QUEST) return fail(FBSA_EINVAL, "fbsa_select: bad score %d", d->score);
  if (d->convention != FBSA_SEL_OWN_FIRST && d->convention != FBSA_SEL_SORTED_SINK)
    return fail(FBSA_EINVAL, "fbsa_select: bad convention %d", d->convention);
  if (d->B < 1 || d->H < 1 || d->nblk < 1 || d->topk < 0) return fail(FBSA_EINVAL, "fbsa_select: bad sizes");
  if (d->nblk > 0x7fffffffLL - 64) return fail(FBSA_EUNSUPPORTED, "fbsa_select: nblk %lld exceeds 32-bit block indices", (long long)d->nblk);
  if (d->flags & ~(0xFFFF << FBSA_SEL_CHUNK_SHIFT)) return fail(FBSA_EINVAL, "fbsa_select: unknown flags 0x%x", d->flags);
  int64_t K, kk;
  if (d->convention == FBSA_SEL_OWN_FIRST) { K = d->topk < d->nblk - 1 ? d->topk : d->nblk - 1; kk = 1 + K; }
  else { K = d->topk < d->nblk ? d->topk : d->nblk; kk = K + 1 + (d->sink ? 1 : 0); }
  if (d->kk != kk) return fail(FBSA_EINVAL, "fbsa_select: kk=%lld but the convention gives %lld", (long long)d->kk, (long long)kk);
  if (K > kSelWideMax)
    return fail(FBSA_EUNSUPPORTED, "fbsa_select: top-k budget %lld > %lld is not supported", (long long)K,
                (long long)kSelWideMax);
  if (!a || !b1 || !sel || (d->score != FBSA_SCORE_DOT && !b2)) return fail(FBSA_EINVAL, "fbsa_select: null pointer");
  const int64_t es = esize(d->dtype);
  if (!aligned(a, es) || !aligned(b1, 16) || (b2 && !aligned(b2, 16)) || !aligned(sel, 4) || (sel_score && !aligned(sel_score, 4)))
    return fail(FBSA_EINVAL, "fbsa_select: misaligned pointer");
  const int64_t ntile = (d->nblk + 7) / 8;
  if (ntile * d->B * d->H > 0x7fffffffLL) return fail(FBSA_EUNSUPPORTED, "fbsa_select: grid too large");
  return FBSA_OK;
}

int fbsa_select_rows(const fbsa_select_desc *d, int64_t row_begin, int64_t row_end, const void *a, const void *b1,
                     const void *b2, int32_t *sel, float *sel_score, void *workspace, size_t workspace_bytes,
                     void *stream) {
  const int ce = check_select(d, row_begin, row_end, a, b1, b2, sel, sel_score);
  if (ce) return ce;
  // Quest scores of wide operands (D >= 128, past the MFMA engine's widths)
  // under _finish for every row and without chosen-slot scores: the row-per-
  // workgroup exact kernel of fbsa_select_qmax with one query vector per block
  // (float64 scores, radix top-k; same blocks and tie-break, several times
  // faster than the streaming fp64 kernel at these widths)
  if (d->score == FBSA_SCORE_QUEST && d->convention == FBSA_SEL_SORTED_SINK && !sel_score && row_begin == 0 &&
      row_end == d->nblk && d->D >= 128 && d->nblk <= 4096) {
    fbsa_qmax_desc q = {};
    q.dtype = d->dtype; q.convention = FBSA_SEL_SORTED_SINK; q.sink = d->sink; q.flags = FBSA_QMAX_EXACT;
    q.B = d->B; q.H = d->H; q.nblk = d->nblk; q.D = d->D; q.tok = 1; q.la = d->nblk;
    q.topk = d->topk; q.kk = d->kk; q.ncand = 0;
    if (!aligned(a, 16)) return fail(FBSA_EINVAL, "fbsa_select: misaligned pointer");
    return run_select_qmax(&q, a, b1, b2, nullptr, sel, nullptr, (hipStream_t)stream);
  }
  // the workspace enables the MFMA path; without one the fp64 kernel runs (same results)
  const size_t need = select_workspace_bytes(d);
  void *ws = (workspace && workspace_bytes >= need && need > 0) ? workspace : nullptr;
  if (ws && !aligned(ws, 16)) return fail(FBSA_EINVAL, "fbsa_select: workspace must be 16-byte aligned");
  return run_select(d, row_begin, row_end, a, b1, b2, sel, sel_score, ws, (hipStream_t)stream);
}

int fbsa_select_mean_pooled(const fbsa_pool_desc *dq, const void *q, void *qp, const fbsa_pool_desc *dk,
                            const void *k, void *kp, const fbsa_select_desc *d, int32_t *sel, float *sel_score,
                            void *workspace, size_t workspace_bytes, void *stream) {
  int e = check_pool(dq, q, qp, nullptr);
  if (!e) e = check_pool(dk, k, kp, nullptr);
  if (e) return e;
  if (dq->op != FBSA_POOL_MEAN_TOK_THEN_GRP || dk->op != FBSA_POOL_MEAN_TOK_THEN_GRP)
    return fail(FBSA_EINVAL, "fbsa_select_mean_pooled: both pools must be MEAN_TOK_THEN_GRP");
  if (!d) return fail(FBSA_EINVAL, "fbsa_select_mean_pooled: null select descriptor");
  if (d->score != FBSA_SCORE_DOT) return fail(FBSA_EINVAL, "fbsa_select_mean_pooled: score must be DOT");
  if (dq->dtype != dk->dtype || dq->dtype != d->dtype || dq->B != dk->B || dq->B != d->B || dq->L != dk->L ||
      dq->D != dk->D || dq->D != d->D || dq->bs != dk->bs || dq->nblk != dk->nblk || dq->nblk != d->nblk ||
      dq->l_valid != dk->l_valid || dq->H / dq->grp != d->H || dk->H / dk->grp != d->H)
    return fail(FBSA_EINVAL, "fbsa_select_mean_pooled: pool and select descriptors disagree");
  e = check_select(d, 0, d->nblk, qp, kp, nullptr, sel, sel_score);
  if (e) return e;
  const size_t need = select_workspace_bytes(d);
  void *ws = (workspace && workspace_bytes >= need && need > 0) ? workspace : nullptr;
  if (ws && !aligned(ws, 16)) return fail(FBSA_EINVAL, "fbsa_select_mean_pooled: workspace must be 16-byte aligned");
  return run_select_mean_pooled(dq, q, qp, dk, k, kp, d, sel, sel_score, ws, (hipStream_t)stream);
}

size_t fbsa_select_qmax_workspace_bytes(const fbsa_qmax_desc *d) { return d ? select_qmax_workspace_bytes(d) : 0; }

int fbsa_select_qmax(const fbsa_qmax_desc *d, const void *a, const void *b1, const void *b2, const int32_t *cand,
                     int32_t *sel, void *workspace, size_t workspace_bytes, void *stream) {
  if (!d) return fail(FBSA_EINVAL, "fbsa_select_qmax: null descriptor");
  if (d->dtype < FBSA_F32 || d->dtype > FBSA_F16) return fail(FBSA_EINVAL, "fbsa_select_qmax: bad dtype %d", d->dtype);
  if (d->convention != FBSA_SEL_SORTED_SINK && d->convention != FBSA_SEL_SORTED_TOPK)
    return fail(FBSA_EINVAL, "fbsa_select_qmax: convention %d is not SORTED_SINK or SORTED_TOPK", d->convention);
  if (d->flags & ~FBSA_QMAX_EXACT) return fail(FBSA_EINVAL, "fbsa_select_qmax: unknown flags 0x%x", d->flags);
  if (d->B < 1 || d->H < 1 || d->nblk < 1 || d->tok < 1 || d->topk < 0)
    return fail(FBSA_EINVAL, "fbsa_select_qmax: bad sizes");
  if (d->la < (d->nblk - 1) * d->tok + 1 || d->la > d->nblk * d->tok)
    return fail(FBSA_EINVAL, "fbsa_select_qmax: la=%lld must cover blocks 0..nblk-1 (((nblk-1)*tok, nblk*tok])",
                (long long)d->la);
  if (d->D != 32 && d->D != 64 && d->D != 128 && d->D != 256)
    return fail(FBSA_EUNSUPPORTED, "fbsa_select_qmax: operand dim %lld not in {32,64,128,256}", (long long)d->D);
  if (d->nblk > 65536) return fail(FBSA_EUNSUPPORTED, "fbsa_select_qmax: nblk %lld > 65536", (long long)d->nblk);
  if (cand && d->ncand < 1) return fail(FBSA_EINVAL, "fbsa_select_qmax: ncand must be >= 1 with a candidate list");
  const int64_t ncol = cand ? d->ncand : d->nblk;
  // two 32-bit keys and two 16-bit indices per column in LDS, beside the tile ring
  if (ncol > 8192) return fail(FBSA_EUNSUPPORTED, "fbsa_select_qmax: %lld columns per row > 8192", (long long)ncol);
  const int64_t K = d->topk < d->nblk ? d->topk : d->nblk;
  const int64_t kk = d->convention == FBSA_SEL_SORTED_SINK ? K + 1 + (d->sink ? 1 : 0) : K;
  if (kk < 1) return fail(FBSA_EINVAL, "fbsa_select_qmax: SORTED_TOPK needs topk >= 1");
  if (d->kk != kk) return fail(FBSA_EINVAL, "fbsa_select_qmax: kk=%lld but the convention gives %lld", (long long)d->kk, (long long)kk);
  if (!a || !b1 || !b2 || !sel) return fail(FBSA_EINVAL, "fbsa_select_qmax: null pointer");
  if (!aligned(a, 16) || !aligned(b1, 16) || !aligned(b2, 16) || !aligned(sel, 4) || (cand && !aligned(cand, 4)))
    return fail(FBSA_EINVAL, "fbsa_select_qmax: misaligned pointer (a, b1, b2 need 16 bytes)");
  if (d->B * d->H * d->nblk > 0x7fffffffLL) return fail(FBSA_EUNSUPPORTED, "fbsa_select_qmax: grid too large");
  // the workspace enables the MFMA engine; without one every score is float64 (same result)
  const size_t need = select_qmax_workspace_bytes(d);
  void *ws = (workspace && need > 0 && workspace_bytes >= need) ? workspace : nullptr;
  if (ws && !aligned(ws, 16)) return fail(FBSA_EINVAL, "fbsa_select_qmax: workspace must be 16-byte aligned");
  return run_select_qmax(d, a, b1, b2, cand, sel, ws, (hipStream_t)stream);
}

}  // extern "C"

// ---- backward ----
namespace fbsa {

static int check_bwd(const fbsa_attn_desc *d, const char *fn, BwdLayout *lay, const void *ws, size_t ws_bytes) {
  int e = check_attn(d, fn);
  if (e) return e;
  if (d->flags & ~(FBSA_FLAG_OUT_GATE | FBSA_FLAG_DENSE | FBSA_FLAG_DGATE)) return fail(FBSA_EINVAL, "%s: unknown flags 0x%x", fn, d->flags);
  if ((d->flags & FBSA_FLAG_DENSE) && (e = check_dense(d, nullptr, nullptr, fn))) return e;
  e = bwd_layout(d, lay);
  if (e) return e;
  if (!ws || !aligned(ws, 256)) return fail(FBSA_EINVAL, "%s: workspace must be non-null and 256-byte aligned", fn);
  if (ws_bytes < lay->total)
    return fail(FBSA_EWORKSPACE, "%s: workspace of %zu bytes, %zu needed", fn, ws_bytes, lay->total);
  return FBSA_OK;
}

static int check_dout(const fbsa_attn_desc *d, const void *dout, const char *fn) {
  if (d->flags & FBSA_FLAG_OUT_GATE) return FBSA_OK;  // the stages read the workspace copy
  if (!dout || !aligned(dout, 16)) return fail(FBSA_EINVAL, "%s: dout must be non-null and 16-byte aligned", fn);
  const int64_t es = esize(d->dtype);
  for (int x = 0; x < 3; ++x)
    if (d->sdo[x] < 0 || (d->sdo[x] * es) % 16)
      return fail(FBSA_EINVAL, "%s: dout stride[%d] must be a non-negative multiple of 16 bytes", fn, x);
  return FBSA_OK;
}

static int check_qkv(const void *q, const void *k, const void *v, const char *fn) {
  if (!q || !k || !v) return fail(FBSA_EINVAL, "%s: null q/k/v", fn);
  if (!aligned(q, 16) || !aligned(k, 16) || !aligned(v, 16)) return fail(FBSA_EINVAL, "%s: q/k/v must be 16-byte aligned", fn);
  return FBSA_OK;
}

}  // namespace fbsa

extern "C" {

size_t fbsa_bwd_workspace_bytes(const fbsa_attn_desc *d) {
  BwdLayout lay;
  if (check_attn(d, "fbsa_bwd_workspace_bytes")) return 0;
  if (bwd_layout(d, &lay)) return 0;
  return lay.total;
}

}  // extern "C"

namespace fbsa {

// Argument checks of the prep and dQ stages (after check_bwd), shared by the
// stage entry points and fbsa_bwd.
static int check_prep_args(const fbsa_attn_desc *d, const void *o, const void *dout, const float *lse,
                           const void *out_gate, const void *dout_gate) {
  const bool og = (d->flags & FBSA_FLAG_OUT_GATE) != 0;
  if (og != (out_gate != nullptr) || og != (dout_gate != nullptr))
    return fail(FBSA_EINVAL, "fbsa_bwd_prep: out_gate and dout_gate must be given exactly when FBSA_FLAG_OUT_GATE is set");
  if (!o || !dout || !lse || !aligned(o, 16) || !aligned(dout, 16) || !aligned(lse, 4))
    return fail(FBSA_EINVAL, "fbsa_bwd_prep: o/dout (16-byte aligned) and lse must be non-null");
  const int64_t es = esize(d->dtype);
  for (int x = 0; x < 3; ++x)
    if (d->sdo[x] < 0 || (d->sdo[x] * es) % 16)
      return fail(FBSA_EINVAL, "fbsa_bwd_prep: dout stride[%d] must be a non-negative multiple of 16 bytes", x);
  if (og && (!aligned(out_gate, es) || !aligned(dout_gate, 16)))
    return fail(FBSA_EINVAL, "fbsa_bwd_prep: out_gate / dout_gate misaligned");
  return FBSA_OK;
}

// A second stream per (host thread, device) for fbsa_bwd's index stage, which
// only reads sel and so runs beside the dQ stage: created on first use with
// the default priority, kept for the life of the process. Per thread, so that
// concurrent calls from other threads (or a capture on one of them) never
// share it.
static int side_stream(hipStream_t *out) {
  constexpr int kMaxDev = 64;
  thread_local hipStream_t streams[kMaxDev] = {};
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_check(e, "fbsa_bwd: hipGetDevice");
  if (dev < 0 || dev >= kMaxDev) return fail(FBSA_EUNSUPPORTED, "fbsa_bwd: device ordinal %d beyond %d", dev, kMaxDev);
  if (!streams[dev]) {
    e = hipStreamCreateWithFlags(&streams[dev], hipStreamNonBlocking);
    if (e != hipSuccess) {
      streams[dev] = nullptr;
      return hip_check(e, "fbsa_bwd: hipStreamCreateWithFlags");
    }
  }
  *out = streams[dev];
  return FBSA_OK;
}

static int check_dq_args(const fbsa_attn_desc *d, const void *q, const void *k, const void *v, const void *dout,
                         const int32_t *sel, const float *gate, void *dq, float *dgate) {
  int e = check_qkv(q, k, v, "fbsa_bwd_dq");
  if (!e) e = check_dout(d, dout, "fbsa_bwd_dq");
  if (e) return e;
  if ((e = check_dense(d, sel, gate, "fbsa_bwd_dq"))) return e;
  if ((d->flags & FBSA_FLAG_DENSE) && dgate) return fail(FBSA_EINVAL, "fbsa_bwd_dq: FBSA_FLAG_DENSE has no gate gradient");
  if (dgate && d->dtype != FBSA_F32 && !(d->flags & FBSA_FLAG_DGATE))
    return fail(FBSA_EINVAL, "fbsa_bwd_dq: a 16-bit gate gradient needs FBSA_FLAG_DGATE in the descriptor "
                             "(the workspace then holds the per-row slot masses)");
  if ((sel && !aligned(sel, 4)) || (gate && !aligned(gate, 4)) || (dgate && !aligned(dgate, 4)))
    return fail(FBSA_EINVAL, "fbsa_bwd_dq: sel/gate/dgate must be 4-byte aligned");
  if (!dq || !aligned(dq, 16)) return fail(FBSA_EINVAL, "fbsa_bwd_dq: dq must be non-null and 16-byte aligned");
  return FBSA_OK;
}

}  // namespace fbsa

extern "C" {

int fbsa_bwd_prep(const fbsa_attn_desc *d, const void *o, const void *dout, const float *lse, const void *out_gate,
                  void *dout_gate, void *workspace, size_t workspace_bytes, void *stream) {
  BwdLayout lay;
  int e = check_bwd(d, "fbsa_bwd_prep", &lay, workspace, workspace_bytes);
  if (!e) e = check_prep_args(d, o, dout, lse, out_gate, dout_gate);
  if (e) return e;
  return run_bwd_prep(d, lay, o, dout, lse, out_gate, dout_gate, (char *)workspace, (hipStream_t)stream);
}

int fbsa_transpose_index(const fbsa_attn_desc *d, const int32_t *sel, void *workspace, size_t workspace_bytes,
                         void *stream) {
  BwdLayout lay;
  int e = check_bwd(d, "fbsa_transpose_index", &lay, workspace, workspace_bytes);
  if (e) return e;
  if ((e = check_dense(d, sel, nullptr, "fbsa_transpose_index"))) return e;
  if (sel && !aligned(sel, 4)) return fail(FBSA_EINVAL, "fbsa_transpose_index: sel must be 4-byte aligned");
  return run_transpose_index(d, lay, sel, (char *)workspace, (hipStream_t)stream);
}

int fbsa_bwd_dq(const fbsa_attn_desc *d, const void *q, const void *k, const void *v, const void *dout,
                const int32_t *sel, const float *gate, void *dq, float *dgate, void *workspace, size_t workspace_bytes,
                void *stream) {
  BwdLayout lay;
  int e = check_bwd(d, "fbsa_bwd_dq", &lay, workspace, workspace_bytes);
  if (!e) e = check_dq_args(d, q, k, v, dout, sel, gate, dq, dgate);
  if (e) return e;
  return run_bwd_dq(d, lay, q, k, v, dout, sel, gate, dq, dgate, (char *)workspace, (hipStream_t)stream);
}

int fbsa_bwd_dkdv(const fbsa_attn_desc *d, const void *q, const void *k, const void *v, const void *dout,
                  const float *gate, void *dk, void *dv, void *workspace, size_t workspace_bytes, void *stream) {
  BwdLayout lay;
  int e = check_bwd(d, "fbsa_bwd_dkdv", &lay, workspace, workspace_bytes);
  if (!e) e = check_qkv(q, k, v, "fbsa_bwd_dkdv");
  if (!e) e = check_dout(d, dout, "fbsa_bwd_dkdv");
  if (e) return e;
  if ((d->flags & FBSA_FLAG_DENSE) && gate) return fail(FBSA_EINVAL, "fbsa_bwd_dkdv: FBSA_FLAG_DENSE takes no gate");
  if (gate && !aligned(gate, 4)) return fail(FBSA_EINVAL, "fbsa_bwd_dkdv: gate must be 4-byte aligned");
  if (!dk || !dv || !aligned(dk, 16) || !aligned(dv, 16))
    return fail(FBSA_EINVAL, "fbsa_bwd_dkdv: dk/dv must be non-null and 16-byte aligned");
  return run_bwd_dkdv(d, lay, q, k, v, dout, gate, dk, dv, (char *)workspace, (hipStream_t)stream);
}

int fbsa_bwd(const fbsa_attn_desc *d, const void *q, const void *k, const void *v, const void *o, const void *dout,
             const float *lse, const int32_t *sel, const float *gate, const void *out_gate, void *dq, void *dk,
             void *dv, float *dgate, void *dout_gate, void *workspace, size_t workspace_bytes, void *stream) {
  // bf16 without an output gate: the prep stage only forms the row statistics,
  // which the dQ stage then forms itself (bit for bit the same), saving the
  // prep's pass over O and dO (fp16 keeps the prep: its sums were not
  // bit-identical between the two kernels' code)
  BwdLayout lay;
  int e = check_bwd(d, "fbsa_bwd", &lay, workspace, workspace_bytes);
  if (e) return e;
  if ((d->flags & FBSA_FLAG_OUT_GATE) || d->dtype != FBSA_BF16) {
    e = fbsa_bwd_prep(d, o, dout, lse, out_gate, dout_gate, workspace, workspace_bytes, stream);
    if (!e) e = fbsa_transpose_index(d, sel, workspace, workspace_bytes, stream);
    if (!e) e = fbsa_bwd_dq(d, q, k, v, dout, sel, gate, dq, dgate, workspace, workspace_bytes, stream);
    if (!e) e = fbsa_bwd_dkdv(d, q, k, v, dout, gate, dk, dv, workspace, workspace_bytes, stream);
    return e;
  }
  e = check_prep_args(d, o, dout, lse, out_gate, dout_gate);
  if (!e) e = check_dq_args(d, q, k, v, dout, sel, gate, dq, dgate);
  if (!e) e = check_qkv(q, k, v, "fbsa_bwd_dkdv");
  if (!e && ((d->flags & FBSA_FLAG_DENSE) && gate)) e = fail(FBSA_EINVAL, "fbsa_bwd_dkdv: FBSA_FLAG_DENSE takes no gate");
  if (!e && (!dk || !dv || !aligned(dk, 16) || !aligned(dv, 16)))
    e = fail(FBSA_EINVAL, "fbsa_bwd_dkdv: dk/dv must be non-null and 16-byte aligned");
  if (!e && sel && !aligned(sel, 4)) e = fail(FBSA_EINVAL, "fbsa_transpose_index: sel must be 4-byte aligned");
  if (e) return e;
  // the index (and the segment tables of long lists) depend on sel alone and run
  // on a second stream beside dQ; dK/dV waits for both. Under stream capture
  // (where creating the library's stream would be refused) they run in order
  // on the caller's stream.
  const hipStream_t s = (hipStream_t)stream;
  char *ws = (char *)workspace;
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  if ((e = hip_check(hipStreamIsCapturing(s, &cap), "fbsa_bwd: hipStreamIsCapturing"))) return e;
  if (cap != hipStreamCaptureStatusNone) {
    e = run_transpose_index(d, lay, sel, ws, s);
    if (!e) e = run_bwd_dq(d, lay, q, k, v, dout, sel, gate, dq, dgate, ws, s, o, lse);
    if (!e) e = run_bwd_dkdv(d, lay, q, k, v, dout, gate, dk, dv, ws, s);
    return e;
  }
  hipStream_t s2 = nullptr;
  if ((e = side_stream(&s2))) return e;
  hipEvent_t forked = nullptr, indexed = nullptr;
  hipError_t he = hipEventCreateWithFlags(&forked, hipEventDisableTiming);
  if (he == hipSuccess) he = hipEventCreateWithFlags(&indexed, hipEventDisableTiming);
  if (he == hipSuccess) he = hipEventRecord(forked, s);
  if (he == hipSuccess) he = hipStreamWaitEvent(s2, forked, 0);
  e = hip_check(he, "fbsa_bwd: stream fork");
  const bool forked_ok = !e;
  if (!e) e = run_transpose_index(d, lay, sel, ws, s2);
  if (!e) e = run_bwd_segments(d, lay, ws, s2);
  // once s2 has been forked it is joined back into s on every path, errors
  // included, so that no work of this call is left behind the caller's stream
  const hipError_t re = forked_ok ? hipEventRecord(indexed, s2) : hipSuccess;
  if (!e) e = hip_check(re, "fbsa_bwd: hipEventRecord");
  if (!e) e = run_bwd_dq(d, lay, q, k, v, dout, sel, gate, dq, dgate, ws, s, o, lse);
  if (forked_ok && re == hipSuccess) {
    const hipError_t we = hipStreamWaitEvent(s, indexed, 0);
    if (we != hipSuccess) (void)hipStreamSynchronize(s2);
    if (!e) e = hip_check(we, "fbsa_bwd: stream join");
  } else if (forked_ok) {
    (void)hipStreamSynchronize(s2);
  }
  if (!e) e = run_bwd_dkdv(d, lay, q, k, v, dout, gate, dk, dv, ws, s, true);
  if (forked) (void)hipEventDestroy(forked);  // released once the streams are past them
  if (indexed) (void)hipEventDestroy(indexed);
  return e;
}

}  // extern "C"

// ---------------------------------------------------------------------------
// Selection without an allocation (fbsa_select_noalloc). The MFMA selection's
// workspace (key norms and the per-chunk partial top-k lists) is taken from a
// static device array instead of a caller's buffer. The array's name is a
// host-side stand-in: its device address is looked up once per device
// (hipGetSymbolAddress, with that device current) and only that address is
// handed to kernels. Every call on a device shares its array; the kernels
// write every byte they later read (norms first, then the lists), so nothing
// needs clearing between calls, and calls that overlap on one device race.
namespace fbsa {

static constexpr size_t kSelectScratchBytes = (size_t)FBSA_SELECT_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[kSelectScratchBytes];

static constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static void *g_scratch_ptr[kMaxDevices];

// Device address of the current device's scratch array (looked up on first use).
static int scratch_address(void **out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_check(e, "fbsa_select_noalloc: hipGetDevice");
  if (dev < 0 || dev >= kMaxDevices)
    return fail(FBSA_EUNSUPPORTED, "fbsa_select_noalloc: device ordinal %d beyond %d", dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void *p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_check(e, "fbsa_select_noalloc: hipGetSymbolAddress(scratch)");
    if (!p || !aligned(p, 256)) return fail(FBSA_EHIP, "fbsa_select_noalloc: scratch address not 256-byte aligned");
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return FBSA_OK;
}

}  // namespace fbsa

extern "C" {

int fbsa_select_noalloc(const fbsa_select_desc *d, const void *a, const void *b1, const void *b2, int32_t *sel,
                        float *sel_score, void *stream) {
  int e = check_select(d, 0, d ? d->nblk : 0, a, b1, b2, sel, sel_score);
  if (e) return e;
  const size_t need = select_workspace_bytes(d);
  if (need > kSelectScratchBytes)
    return fail(FBSA_EWORKSPACE,
                "fbsa_select_noalloc: this selection needs %zu bytes of scratch, more than the %zu bytes of the "
                "static scratch (call fbsa_select with a workspace instead)",
                need, kSelectScratchBytes);
  void *ws = nullptr;
  if (need && (e = scratch_address(&ws))) return e;
  return fbsa_select_rows(d, 0, d->nblk, a, b1, b2, sel, sel_score, ws, need, stream);
}

}  // extern "C"
