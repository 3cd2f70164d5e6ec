// Dense causal per-block attention mass for gfx950 (CDNA4): the teacher that
// SelectOracle selects from.
//
//   mass[b, h, i, j] = mean over the query rows t of block i of
//                      sum over the keys s of block j, s <= t, of softmax_s(S[t, :])
//   S[t, s]          = rnd(rnd(q_t . k_s) * scale)  (rounded to the operand dtype,
//                      as torch rounds a 16-bit matmul and the scale multiply)
//
// with the softmax in fp32 (src/eval_qwen_ppl.py:65-108, capture_mass; the
// group mean over each KV head's query heads is left to the caller, as there).
// Two passes over the causal key range of every query block, one workgroup per
// (b, query head, query block), one wave per 16 query rows, K tiles through a
// direct-to-LDS ring like the forward:
//   pass 1: per query row, the log-sum-exp of S over keys s <= t;
//   pass 2: per key block, the sum of exp(S - lse) over the block's rows and
//           keys, reduced over the lanes of each wave and then over the waves
//           (two LDS slots alternate between consecutive key blocks, ordered
//           by the ring's per-chunk barrier).
#include "fbsa_common.h"
#include "fbsa_internal.h"

namespace fbsa {

struct MassArgs {
  const void *q, *k;
  float *mass;  // (B, Hq, nblk, nblk)
  float *lse;   // (B, Hq, L) natural log, pass 1 output / pass 2 input
  int64_t B, Hq, Hkv, L, nblk;
  int64_t sq[3], sk[3];
  float scale;
  int grp;
};

template <typename T, int BS, int D> struct MassCfg {
  static constexpr int NW = BS / 16;
  static constexpr int NT = NW * 64;
  static constexpr int KC = D >= 256 ? 32 : 64;  // keys per chunk
  static constexpr int NCH = BS / KC;
  static constexpr int CPR = D * 2 / 16;
  static constexpr int TILE_BYTES = KC * D * 2;
  static constexpr int LPT = TILE_BYTES / (NT * 16);
  static constexpr int NSTAGE = 3;
  static_assert(LPT * NT * 16 == TILE_BYTES, "tile must split evenly over threads");
  static_assert(KC <= BS, "chunk larger than a block");
};

template <typename T> __device__ __forceinline__ float round_to_t(float x) { return (float)(T)x; }

template <typename T, int BS, int D, int PASS>
__global__ __launch_bounds__(BS * 4) void mass_kernel(MassArgs a) {
  using C = MassCfg<T, BS, D>;
  extern __shared__ __attribute__((aligned(16))) char smem[];
  char *stages = smem;
  float *s_part = (float *)(smem + C::NSTAGE * C::TILE_BYTES);  // [2][NW] per-wave block sums

  const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63, g = lane >> 4,
            p = lane & 15;
  // heavy (late) query blocks first
  int64_t t = blockIdx.x;
  const int i = (int)(a.nblk - 1 - t % a.nblk);
  t /= a.nblk;
  const int hq = (int)(t % a.Hq);
  const int64_t b = t / a.Hq;
  const int hk = hq / a.grp;
  const int qrow = 16 * w + p;  // this lane's query row within block i

  // Q fragments (B operands of S^T = K Q^T): lane (p, g) holds q[qrow][32 ks + 8 g .. + 7]
  s16x8 qf[D / 32];
  {
    const T *qr = (const T *)a.q + b * a.sq[0] + hq * a.sq[1] + ((int64_t)i * BS + qrow) * a.sq[2];
#pragma unroll
    for (int ks = 0; ks < D / 32; ++ks) qf[ks] = *(const s16x8 *)(qr + 32 * ks + 8 * g);
  }
  float lse_row = 0.f;
  if constexpr (PASS == 2) lse_row = a.lse[(b * a.Hq + hq) * a.L + (int64_t)i * BS + qrow];

  // direct-to-LDS plan: per-lane byte offsets of this thread's LPT loads of a K chunk
  int32_t koff[C::LPT];
#pragma unroll
  for (int n = 0; n < C::LPT; ++n) {
    const int u = (n * C::NW + w) * 64 + lane;
    const int row = u / C::CPR, pos = u % C::CPR;
    koff[n] = (int32_t)(((int64_t)row * a.sk[2] + (pos ^ swz(row, C::CPR)) * 8) * 2);
  }
  const char *kbase = (const char *)((const T *)a.k + b * a.sk[0] + hk * a.sk[1]);
  const int64_t kstep = a.sk[2] * 2;
  const int nchunks = (i + 1) * C::NCH;
  auto issue = [&](int c) {
    const char *kb = kbase + ((int64_t)c * C::KC) * kstep;  // chunk c = keys c KC .. c KC + KC - 1
    char *st = stages + (c % C::NSTAGE) * C::TILE_BYTES;
#pragma unroll
    for (int n = 0; n < C::LPT; ++n) g2lds16(kb + koff[n], st + (n * C::NW + w) * 1024);
  };
#pragma unroll
  for (int c = 0; c < C::NSTAGE - 1; ++c)
    if (c < nchunks) issue(c);
  // the register-operand loads above and the first stages have landed (issued
  // together, so their latencies overlap): the compiler then waits for nothing
  // inside the ring loop, where its own waits would also drain the prefetch
  wait_vmcnt<0>();


  float mx = -INFINITY, sm = 0.f;  // pass 1: this lane's running max and sum
  float acc = 0.f;                 // pass 2: this lane's sum over the current key block
  for (int c = 0; c < nchunks; ++c) {
    const int ahead = nchunks - 1 - c;
    wait_ring<C::LPT>(ahead < C::NSTAGE - 2 ? ahead : C::NSTAGE - 2);
    lds_barrier();  // chunk c landed for every wave; chunk c-1's stage is free
    if (c + C::NSTAGE - 1 < nchunks) issue(c + C::NSTAGE - 1);
    const int j = c / C::NCH, ch = c % C::NCH;
    if constexpr (PASS == 2) {
      // the first chunk of block j: every wave has stored its sum of block j-1 (before this
      // barrier); wave 0 combines them
      if (ch == 0 && j > 0 && w == 0 && lane == 0) {
        float tot = 0.f;
#pragma unroll
        for (int ww = 0; ww < C::NW; ++ww) tot += s_part[((j - 1) & 1) * C::NW + ww];
        a.mass[((b * a.Hq + hq) * a.nblk + i) * a.nblk + (j - 1)] = tot * (1.f / BS);
      }
    }
    const char *Ks = stages + (c % C::NSTAGE) * C::TILE_BYTES;
    float s[C::KC / 16][4];
#pragma unroll
    for (int m = 0; m < C::KC / 16; ++m) {
      f32x4 acc4 = f32x4{0.f, 0.f, 0.f, 0.f};
      const int row = 16 * m + p;
#pragma unroll
      for (int ks = 0; ks < D / 32; ++ks) {
        const s16x8 kf = *(const s16x8 *)(Ks + (row * C::CPR + ((4 * ks + g) ^ swz(row, C::CPR))) * 16);
        acc4 = Mfma16<T>::run(kf, qf[ks], acc4);
      }
      // lane (p, g) holds keys 16m + 4g + r of the chunk for query row qrow
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float v = round_to_t<T>(round_to_t<T>(acc4[r]) * a.scale);
        if (j == i && ch * C::KC + 16 * m + 4 * g + r > qrow) v = -INFINITY;  // key after the query
        s[m][r] = v;
      }
    }
    if constexpr (PASS == 1) {
      float cm = s[0][0];
#pragma unroll
      for (int m = 0; m < C::KC / 16; ++m)
#pragma unroll
        for (int r = 0; r < 4; ++r) cm = fmaxf(cm, s[m][r]);
      if (cm > mx) {
        sm *= __expf(mx - cm);  // 0 while mx = -inf
        mx = cm;
      }
      if (mx != -INFINITY) {
#pragma unroll
        for (int m = 0; m < C::KC / 16; ++m)
#pragma unroll
          for (int r = 0; r < 4; ++r) sm += __expf(s[m][r] - mx);
      }
    } else {
#pragma unroll
      for (int m = 0; m < C::KC / 16; ++m)
#pragma unroll
        for (int r = 0; r < 4; ++r) acc += __expf(s[m][r] - lse_row);
      if (ch == C::NCH - 1) {
        // block j done: the wave's sum (over its 16 rows and the block's keys) to LDS
        float x = acc;
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) x += __shfl_xor(x, off, 64);
        if (lane == 0) s_part[(j & 1) * C::NW + w] = x;
        acc = 0.f;
      }
    }
  }

  if constexpr (PASS == 1) {
    // a query row's keys are spread over the lanes p, p+16, p+32, p+48
    float M = fmaxf(mx, __shfl_xor(mx, 16, 64));
    M = fmaxf(M, __shfl_xor(M, 32, 64));
    float part = mx == -INFINITY ? 0.f : sm * __expf(mx - M);
    part += __shfl_xor(part, 16, 64);
    part += __shfl_xor(part, 32, 64);
    if (g == 0) a.lse[(b * a.Hq + hq) * a.L + (int64_t)i * BS + qrow] = M + __logf(part);
  } else {
    __syncthreads();  // every wave's sum of block i is in LDS
    const int64_t rowoff = ((b * a.Hq + hq) * a.nblk + i) * a.nblk;
    if (tid == 0) {
      float tot = 0.f;
#pragma unroll
      for (int ww = 0; ww < C::NW; ++ww) tot += s_part[(i & 1) * C::NW + ww];
      a.mass[rowoff + i] = tot * (1.f / BS);
    }
    for (int64_t jj = i + 1 + tid; jj < a.nblk; jj += C::NT) a.mass[rowoff + jj] = 0.f;  // above the diagonal
  }
}

template <typename T, int BS, int D> static int launch_mass(const MassArgs &a, hipStream_t s) {
  using C = MassCfg<T, BS, D>;
  const size_t lds = (size_t)C::NSTAGE * C::TILE_BYTES + 2 * C::NW * sizeof(float);
  {
    int e = lds_optin((const void *)mass_kernel<T, BS, D, 1>, lds, "hipFuncSetAttribute(mass)");
    if (!e) e = lds_optin((const void *)mass_kernel<T, BS, D, 2>, lds, "hipFuncSetAttribute(mass)");
    if (e) return e;
  }
  const unsigned nwg = (unsigned)(a.B * a.Hq * a.nblk);
  hipLaunchKernelGGL((mass_kernel<T, BS, D, 1>), dim3(nwg), dim3(C::NT), lds, s, a);
  int e = hip_check(hipGetLastError(), "mass_kernel launch (pass 1)");
  if (e) return e;
  hipLaunchKernelGGL((mass_kernel<T, BS, D, 2>), dim3(nwg), dim3(C::NT), lds, s, a);
  return hip_check(hipGetLastError(), "mass_kernel launch (pass 2)");
}

template <typename T, int BS> static int mass_d(const MassArgs &a, int64_t D, hipStream_t s) {
  switch (D) {
    case 64: return launch_mass<T, BS, 64>(a, s);
    case 128: return launch_mass<T, BS, 128>(a, s);
    case 256: return launch_mass<T, BS, 256>(a, s);
  }
  return fail(FBSA_EUNSUPPORTED, "fbsa_block_mass: head dim %lld not in {64,128,256}", (long long)D);
}

template <typename T> static int mass_bs(const MassArgs &a, int64_t bs, int64_t D, hipStream_t s) {
  switch (bs) {
    case 64: return mass_d<T, 64>(a, D, s);
    case 128: return mass_d<T, 128>(a, D, s);
  }
  return fail(FBSA_EUNSUPPORTED, "fbsa_block_mass: block size %lld not in {64,128}", (long long)bs);
}

int run_block_mass(const fbsa_attn_desc *d, const void *q, const void *k, float *mass, float *lse, hipStream_t s) {
  MassArgs a;
  a.q = q; a.k = k; a.mass = mass; a.lse = lse;
  a.B = d->B; a.Hq = d->Hq; a.Hkv = d->Hkv; a.L = d->L; a.nblk = d->nblk;
  for (int x = 0; x < 3; ++x) { a.sq[x] = d->sq[x]; a.sk[x] = d->sk[x]; }
  a.scale = d->scale;
  a.grp = (int)(d->Hq / d->Hkv);
  if (d->dtype == FBSA_BF16) return mass_bs<bf16>(a, d->bs, d->D, s);
  if (d->dtype == FBSA_F16) return mass_bs<f16>(a, d->bs, d->D, s);
  return fail(FBSA_EUNSUPPORTED, "fbsa_block_mass: 16-bit operands only (bf16, f16)");
}

}  // namespace fbsa
