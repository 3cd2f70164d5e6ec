// Kernel argument blocks and launch entry points shared by the C ABI layer.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "fbsa.h"

namespace fbsa {

struct FwdArgs {
  const void *q, *k, *v;
  void *o;
  float *lse;
  const int32_t *sel;
  const float *gate;
  const void *og;
  int64_t B, Hq, Hkv, L, nblk, kk, hsel, l_valid;
  int64_t i0, ni;  // query blocks [i0, i0 + ni) of this launch
  int64_t sq[3], sk[3], sv[3], so[3], sog[3];
  float scale2;  // softmax scale * log2(e)
  int mask;
  int grp;
  int dense;     // FBSA_FLAG_DENSE: slot s is block s, sel and gate unused
};

// Top-k budgets of fbsa_select: up to kSelListMax on the wave-list kernels,
// up to kSelWideMax on the row-per-workgroup kernel (its keys live in LDS).
constexpr int64_t kSelListMax = 62;
constexpr int64_t kSelWideMax = 4096;

// Opts kernel `fn` into `bytes` of dynamic LDS on the current device (needed
// above 64 KiB). Thread-safe; the grant is remembered per (device, kernel), so
// the attribute is set once per device and size increase.
int lds_optin(const void *fn, size_t bytes, const char *what);

int run_fwd(const fbsa_attn_desc *d, const FwdArgs &a, hipStream_t s);
int run_pool(const fbsa_pool_desc *d, const void *x, void *out, void *out2, hipStream_t s);
int run_select_mean_pooled(const fbsa_pool_desc *dq, const void *q, void *qp, const fbsa_pool_desc *dk, const void *k,
                           void *kp, const fbsa_select_desc *d, int32_t *sel, float *sel_score, void *ws, hipStream_t s);
int run_block_mass(const fbsa_attn_desc *d, const void *q, const void *k, float *mass, float *lse, hipStream_t s);
size_t select_workspace_bytes(const fbsa_select_desc *d);
int run_select(const fbsa_select_desc *d, int64_t row0, int64_t row1, const void *a, const void *b1, const void *b2,
               int32_t *sel, float *sel_score, void *ws, hipStream_t s);
size_t select_qmax_workspace_bytes(const fbsa_qmax_desc *d);
int run_select_qmax(const fbsa_qmax_desc *d, const void *a, const void *b1, const void *b2, const int32_t *cand,
                    int32_t *sel, void *ws, hipStream_t s);

// ---- backward ----
// Byte offsets of the backward workspace regions (each 256-byte aligned).
struct BwdLayout {
  int64_t n;       // sort entries: B * hsel * nblk * kk
  int64_t nseg;    // CSR segments: B * hsel * nblk
  int end_bit;     // radix-sort key bits
  size_t rowstat, dout_attn, dgate_part, pmass, keys_in, keys_out, vals_in, vals_out, seg_off, sort_tmp;
  size_t sort_tmp_bytes, total;
  // dK/dV list segments: a (b, KV head, key block) whose list is longer than
  // seg_entries (0: never) is walked by several workgroups that write fp32
  // partials, summed in segment order by a second kernel
  int64_t nwi;       // work items B * Hkv * nblk
  int64_t seg_entries, xub, slots_ub;  // segment length, bounds on extra segments and partial slots
  size_t seg_cnt, seg_pos, wi_slot, xtab, partials, scan_tmp, scan_tmp_bytes;
};

int bwd_layout(const fbsa_attn_desc *d, BwdLayout *lay);
int run_bwd_prep(const fbsa_attn_desc *d, const BwdLayout &lay, const void *o, const void *dout, const float *lse,
                 const void *out_gate, void *dout_gate, char *ws, hipStream_t s);
int run_transpose_index(const fbsa_attn_desc *d, const BwdLayout &lay, const int32_t *sel, char *ws, hipStream_t s);
// o, lse non-null (bf16, no output gate): the dQ stage forms the row
// statistics itself, in place of the prep stage
int run_bwd_dq(const fbsa_attn_desc *d, const BwdLayout &lay, const void *q, const void *k, const void *v,
               const void *dout, const int32_t *sel, const float *gate, void *dq, float *dgate, char *ws,
               hipStream_t s, const void *o = nullptr, const float *lse = nullptr);
int run_bwd_segments(const fbsa_attn_desc *d, const BwdLayout &lay, char *ws, hipStream_t s);
int run_bwd_dkdv(const fbsa_attn_desc *d, const BwdLayout &lay, const void *q, const void *k, const void *v,
                 const void *dout, const float *gate, void *dk, void *dv, char *ws, hipStream_t s, bool segments_done = false);

}  // namespace fbsa
