// Kernel argument blocks and launch entry points shared by the C ABI layer.
#pragma once
#include <hip/hip_runtime.h>
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
  int64_t sq[3], sk[3], sv[3], so[3], sog[3];
  float scale2;  // softmax scale * log2(e)
  int mask;
  int grp;
};

int run_fwd(const fbsa_attn_desc *d, const FwdArgs &a, hipStream_t s);
int run_pool(const fbsa_pool_desc *d, const void *x, void *out, void *out2, hipStream_t s);
int run_select(const fbsa_select_desc *d, const void *a, const void *b1, const void *b2, int32_t *sel,
               float *sel_score, hipStream_t s);

}  // namespace fbsa
