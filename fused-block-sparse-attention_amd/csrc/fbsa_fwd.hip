// Fused block-sparse attention forward for gfx950 (CDNA4).
//
// One workgroup per (b, query head, query block i); one wave per 16 query
// rows. The selected key blocks are streamed in chunks of KC keys: K and V
// chunks go global -> LDS with direct-to-LDS 16-byte loads through an
// NSTAGE-deep ring (no VGPR staging), with a per-row XOR swizzle of 16-byte
// chunks. Each wave computes S^T = K Q^T on MFMA (K rows read with ds_read_b128,
// Q held in VGPRs), applies the mask rule and gate bias, runs the online
// softmax in the log2 domain (one query per lane column, 4 lanes per query),
// and accumulates O^T += V^T P^T on MFMA, with V^T fragments read by the
// transposing ds_read_b64_tr_b16. The epilogue divides by the row sum,
// optionally multiplies by sigmoid(out_gate), stores O and the natural-log LSE.
//
// Reference semantics: src/triton_kernel.py:20-74 (online softmax over an
// index list, slot-0 triu, future content blocks masked, gate after scale) and
// src/qwen_blocksparse.py:67-81 (token-causal, padding, duplicate masks).
#include "fbsa_common.h"
#include "fbsa_internal.h"

namespace fbsa {

enum { KIND_FULL = 0, KIND_DIAG = 1, KIND_ABS = 2, KIND_PAD = 3 };

// LDS bytes per workgroup for the K/V prefetch ring (sets the ring depth).
#ifndef FBSA_FWD_LDS_BUDGET
#define FBSA_FWD_LDS_BUDGET 32768
#endif

template <typename T, int BS, int D> struct FwdCfg {
  static constexpr int ES = sizeof(T);
  static constexpr int NW = BS / 16;
  static constexpr int NT = NW * 64;
  static constexpr int KC = BS < (D >= 256 ? 32 : 64) ? BS : (D >= 256 ? 32 : 64);
  static constexpr int NCH = BS / KC;
  static constexpr int CPR = D * ES / 16;
  static constexpr int TILE_BYTES = KC * D * ES;
  static constexpr int STAGE_BYTES = 2 * TILE_BYTES;
  static constexpr int LPT = STAGE_BYTES / (NT * 16);
  static constexpr int NS0 = FBSA_FWD_LDS_BUDGET / STAGE_BYTES;
  static constexpr int NSTAGE = NS0 < 1 ? 1 : (NS0 > 4 ? 4 : NS0);
  static_assert(LPT * NT * 16 == STAGE_BYTES, "stage must split evenly over threads");
  static_assert(TILE_BYTES % 1024 == 0, "tile must be whole wave-loads");
};

template <int N> __device__ __forceinline__ void wait_pending(int pending_chunks) {
  // wait until at most pending_chunks * LPT DMA loads are outstanding (N = LPT)
  switch (pending_chunks) {
    case 0: wait_vmcnt<0>(); break;
    case 1: wait_vmcnt<(N < 64 ? N : 63)>(); break;
    case 2: wait_vmcnt<(2 * N < 64 ? 2 * N : 63)>(); break;
    default: wait_vmcnt<(3 * N < 64 ? 3 * N : 63)>(); break;
  }
}

template <typename T, int BS, int D>
__global__ __launch_bounds__(BS * 4) void fwd_kernel(FwdArgs a) {
  using C = FwdCfg<T, BS, D>;
  constexpr bool F32 = sizeof(T) == 4;
  extern __shared__ __attribute__((aligned(16))) char smem[];
  char *stages = smem;
  int *s_blk = (int *)(smem + C::NSTAGE * C::STAGE_BYTES);
  int *s_kind = s_blk + a.kk;
  float *s_gate = (float *)(s_kind + a.kk);
  __shared__ int s_nvalid;

  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, g = lane >> 4, p = lane & 15;
  const int64_t total = a.B * a.Hq * a.nblk;
  int64_t t = xcd_remap(blockIdx.x, total);
  const int hin = (int)(t % a.grp); t /= a.grp;
  const int64_t i = t % a.nblk; t /= a.nblk;
  const int hk = (int)(t % a.Hkv);
  const int64_t b = t / a.Hkv;
  const int hq = hk * a.grp + hin;
  const int hs = a.hsel == 1 ? 0 : hk;

  // ---- 1. plan: compact list of valid slots with their mask kind and gate ----
  const int64_t rowoff = ((b * a.hsel + hs) * a.nblk + i) * a.kk;
  const int32_t *selrow = a.sel + rowoff;
  if (w == 0) {
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
      }
      nout += __popcll(m);
    }
    if (lane == 0) s_nvalid = nout;
  }

  // ---- 2. Q fragment (B operand of S^T = K Q^T) ----
  const int tq = w * 16 + p;  // query row within the block
  const T *qrow = (const T *)a.q + b * a.sq[0] + hq * a.sq[1] + (i * BS + tq) * a.sq[2];
  constexpr int QF = F32 ? D / 4 : D / 32;
  s16x8 qf16[F32 ? 1 : QF];
  float qf32[F32 ? QF : 1];
  if constexpr (F32) {
#pragma unroll
    for (int ks = 0; ks < QF; ++ks) qf32[ks] = ((const float *)qrow)[4 * ks + g];
  } else {
#pragma unroll
    for (int ks = 0; ks < QF; ++ks) qf16[ks] = *(const s16x8 *)(qrow + 32 * ks + 8 * g);
  }
  __syncthreads();
  const int nv = s_nvalid;
  const int nchunks = nv * C::NCH;

  const T *kbase = (const T *)a.k + b * a.sk[0] + hk * a.sk[1];
  const T *vbase = (const T *)a.v + b * a.sv[0] + hk * a.sv[1];
  auto issue = [&](int c) {
    const int slot = c / C::NCH, ch = c % C::NCH;
    const int64_t row0 = (int64_t)s_blk[slot] * BS + ch * C::KC;
    char *st = stages + (c % C::NSTAGE) * C::STAGE_BYTES;
#pragma unroll
    for (int n = 0; n < C::LPT; ++n) {
      const int wl = n * C::NW + w;  // wave-load index within the stage (1 KiB each)
      const int u = wl * 64 + lane;
      const int part = u / (C::KC * C::CPR);
      const int rem = u - part * (C::KC * C::CPR);
      const int row = rem / C::CPR, pos = rem % C::CPR;
      const int chunk = pos ^ swz(row, C::CPR);
      const T *src = part ? vbase + (row0 + row) * a.sv[2] : kbase + (row0 + row) * a.sk[2];
      g2lds16(src + chunk * (16 / C::ES), st + wl * 1024);
    }
  };

  float m_run = -INFINITY, l_run = 0.f;
  f32x4 oacc[D / 16];
#pragma unroll
  for (int mt = 0; mt < D / 16; ++mt) oacc[mt] = f32x4{0.f, 0.f, 0.f, 0.f};

#pragma unroll
  for (int c = 0; c < C::NSTAGE - 1; ++c)
    if (c < nchunks) issue(c);

  for (int c = 0; c < nchunks; ++c) {
    if (c + C::NSTAGE - 1 < nchunks) issue(c + C::NSTAGE - 1);
    const int ahead = nchunks - 1 - c;
    wait_pending<C::LPT>(ahead < C::NSTAGE - 1 ? ahead : C::NSTAGE - 1);
    lds_barrier();

    const char *Ks = stages + (c % C::NSTAGE) * C::STAGE_BYTES;
    const char *Vs = Ks + C::TILE_BYTES;
    const int slot = c / C::NCH, ch = c % C::NCH;
    const int kind = s_kind[slot];
    const float gt = s_gate[slot];
    const int64_t j = s_blk[slot];

    // S^T (KC keys x 16 queries of this wave)
    f32x4 sacc[C::KC / 16];
#pragma unroll
    for (int m = 0; m < C::KC / 16; ++m) {
      sacc[m] = f32x4{0.f, 0.f, 0.f, 0.f};
      const int row = 16 * m + p;
      if constexpr (F32) {
#pragma unroll
        for (int ks = 0; ks < QF; ++ks) {
          const float kf = *(const float *)(Ks + (row * C::CPR + (ks ^ swz(row, C::CPR))) * 16 + g * 4);
          sacc[m] = mfma_f32_16x16x4(kf, qf32[ks], sacc[m]);
        }
      } else {
#pragma unroll
        for (int ks = 0; ks < QF; ++ks) {
          const s16x8 kf = *(const s16x8 *)(Ks + (row * C::CPR + ((4 * ks + g) ^ swz(row, C::CPR))) * 16);
          sacc[m] = Mfma16<T>::run(kf, qf16[ks], sacc[m]);
        }
      }
    }

    // mask: key row u (within block j) is valid iff u <= lim (uniform branch
    // skips the compares for unmasked chunks, the common case)
    if (kind != KIND_FULL) {
      const int64_t lim64 = kind == KIND_DIAG ? (int64_t)tq
                            : kind == KIND_PAD  ? a.l_valid - j * BS - 1
                                                : ((i - j) * BS + tq < a.l_valid - j * BS - 1 ? (i - j) * BS + tq
                                                                                              : a.l_valid - j * BS - 1);
      const int lim = (int)(lim64 < -1 ? -1 : lim64) - ch * C::KC - 4 * g;  // compare against 16m + r
#pragma unroll
      for (int m = 0; m < C::KC / 16; ++m)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (16 * m + r > lim) sacc[m][r] = -INFINITY;
    }
    // online softmax in the log2 domain; scale and gate are folded into one
    // FMA per score: p = exp2(s * scale2 + (gate2 - m))
    float mloc = -INFINITY;
#pragma unroll
    for (int m = 0; m < C::KC / 16; ++m)
      mloc = fmaxf(mloc, fmaxf(fmaxf(sacc[m][0], sacc[m][1]), fmaxf(sacc[m][2], sacc[m][3])));
    mloc = fmaxf(mloc, shfl_xor_f(mloc, 16));
    mloc = fmaxf(mloc, shfl_xor_f(mloc, 32));
    const float mchunk = mloc * a.scale2 + gt;  // -inf when every key is masked
    const float m_new = fmaxf(m_run, mchunk);
    const float m_use = m_new == -INFINITY ? 0.f : m_new;
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
    const float off = gt - m_use;
    float sv[C::KC / 16][4];
    float psum = 0.f;
#pragma unroll
    for (int m = 0; m < C::KC / 16; ++m)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float e = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[m][r], a.scale2, off));
        sv[m][r] = e;
        psum += e;
      }
    l_run = __builtin_fmaf(l_run, alpha, psum);
    m_run = m_new;
    if (__ballot(alpha != 1.f)) {  // rescale only when some row max moved
#pragma unroll
      for (int mt = 0; mt < D / 16; ++mt)
#pragma unroll
        for (int r = 0; r < 4; ++r) oacc[mt][r] *= alpha;
    }

    // O^T += V^T P^T
    if constexpr (F32) {
#pragma unroll
      for (int mt = 0; mt < D / 16; ++mt)
#pragma unroll
        for (int m = 0; m < C::KC / 16; ++m)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int vrow = 16 * m + 4 * g + r;
            const float vf = *(const float *)(Vs + (vrow * C::CPR + ((4 * mt + (p >> 2)) ^ swz(vrow, C::CPR))) * 16 + (p & 3) * 4);
            oacc[mt] = mfma_f32_16x16x4(vf, sv[m][r], oacc[mt]);
          }
    } else if constexpr (C::KC >= 32) {
      s16x8 pf[C::KC / 32];
#pragma unroll
      for (int k2 = 0; k2 < C::KC / 32; ++k2) {
        float x[8];
#pragma unroll
        for (int r = 0; r < 4; ++r) { x[r] = sv[2 * k2][r]; x[4 + r] = sv[2 * k2 + 1][r]; }
        pf[k2] = pack8<T>(x);
      }
      s16x4 vlo[D / 16][C::KC / 32], vhi[D / 16][C::KC / 32];
#pragma unroll
      for (int mt = 0; mt < D / 16; ++mt) {
        const int cb = 2 * mt + ((p & 3) >> 1);  // logical 16-B chunk of d0 = 16mt + 4(p&3)
#pragma unroll
        for (int k2 = 0; k2 < C::KC / 32; ++k2) {
          const int ra = 32 * k2 + 4 * g + (p >> 2);
          const int rb = ra + 16;
          vlo[mt][k2] = lds_read_tr16(Vs + (ra * C::CPR + (cb ^ swz(ra, C::CPR))) * 16 + (p & 1) * 8);
          vhi[mt][k2] = lds_read_tr16(Vs + (rb * C::CPR + (cb ^ swz(rb, C::CPR))) * 16 + (p & 1) * 8);
        }
      }
      lds_wait_all();
#pragma unroll
      for (int mt = 0; mt < D / 16; ++mt)
#pragma unroll
        for (int k2 = 0; k2 < C::KC / 32; ++k2) {
          lds_ready(vlo[mt][k2]);
          lds_ready(vhi[mt][k2]);
          const s16x4 lo = vlo[mt][k2], hi = vhi[mt][k2];
          const s16x8 vf = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
          oacc[mt] = Mfma16<T>::run(vf, pf[k2], oacc[mt]);
        }
    } else {
      // KC == 16: one 16x16x16 MFMA per d tile
      s16x4 pf;
#pragma unroll
      for (int r = 0; r < 4; ++r) pf[r] = bits16<T>((T)sv[0][r]);
      s16x4 vf[D / 16];
#pragma unroll
      for (int mt = 0; mt < D / 16; ++mt) {
        const int cb = 2 * mt + ((p & 3) >> 1);
        const int ra = 4 * g + (p >> 2);
        vf[mt] = lds_read_tr16(Vs + (ra * C::CPR + (cb ^ swz(ra, C::CPR))) * 16 + (p & 1) * 8);
      }
      lds_wait_all();
#pragma unroll
      for (int mt = 0; mt < D / 16; ++mt) {
        lds_ready(vf[mt]);
        oacc[mt] = Mfma16<T>::run16(vf[mt], pf, oacc[mt]);
      }
    }
    lds_barrier();  // the next iteration's prefetch overwrites this stage
  }

  // ---- 4. epilogue ----
  float lt = l_run + shfl_xor_f(l_run, 16);
  lt += shfl_xor_f(lt, 32);
  const float inv = lt > 0.f ? 1.f / lt : 0.f;
  T *orow = (T *)a.o + b * a.so[0] + hq * a.so[1] + (i * BS + tq) * a.so[2];
  const T *ogrow = a.og ? (const T *)a.og + b * a.sog[0] + hq * a.sog[1] + (i * BS + tq) * a.sog[2] : nullptr;
#pragma unroll
  for (int mt = 0; mt < D / 16; ++mt) {
    const int d0 = 16 * mt + 4 * g;
    float y[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) y[r] = oacc[mt][r] * inv;
    if (ogrow) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float z = to_f32<T>(ogrow[d0 + r]);
        y[r] *= 1.f / (1.f + __expf(-z));
      }
    }
    if constexpr (F32) {
      *(f32x4 *)(orow + d0) = f32x4{y[0], y[1], y[2], y[3]};
    } else {
      s16x4 pk;
#pragma unroll
      for (int r = 0; r < 4; ++r) pk[r] = bits16<T>((T)y[r]);
      *(s16x4 *)(orow + d0) = pk;
    }
  }
  if (a.lse && g == 0) {
    const int64_t li = (b * a.Hq + hq) * a.L + i * BS + tq;
    a.lse[li] = lt > 0.f ? (m_run + __log2f(lt)) * kLn2 : -INFINITY;
  }
}

template <typename T, int BS, int D> static int launch_fwd(const FwdArgs &a, hipStream_t stream) {
  using C = FwdCfg<T, BS, D>;
  const size_t lds = (size_t)C::NSTAGE * C::STAGE_BYTES + (size_t)a.kk * 12;
  if (lds > 160 * 1024 - 64) return fail(FBSA_EUNSUPPORTED, "fbsa_fwd: kk=%lld needs %zu bytes of LDS", (long long)a.kk, lds);
  if (lds > 64 * 1024) {
    static size_t attr_bytes = 0;  // largest opt-in granted so far for this instantiation
    if (lds > attr_bytes) {
      int e = hip_check(hipFuncSetAttribute((const void *)fwd_kernel<T, BS, D>,
                                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds),
                        "hipFuncSetAttribute(fwd)");
      if (e) return e;
      attr_bytes = lds;
    }
  }
  const int64_t nwg = a.B * a.Hq * a.nblk;
  hipLaunchKernelGGL((fwd_kernel<T, BS, D>), dim3((unsigned)nwg), dim3(C::NT), lds, stream, a);
  return hip_check(hipGetLastError(), "fwd_kernel launch");
}

template <typename T, int BS> static int dispatch_d(const FwdArgs &a, int64_t D, hipStream_t s) {
  switch (D) {
    case 32: return launch_fwd<T, BS, 32>(a, s);
    case 64: return launch_fwd<T, BS, 64>(a, s);
    case 128: return launch_fwd<T, BS, 128>(a, s);
    case 256: return launch_fwd<T, BS, 256>(a, s);
  }
  return fail(FBSA_EUNSUPPORTED, "fbsa_fwd: head dim %lld not in {32,64,128,256}", (long long)D);
}

template <typename T> static int dispatch_bs(const FwdArgs &a, int64_t bs, int64_t D, hipStream_t s) {
  switch (bs) {
    case 16: return dispatch_d<T, 16>(a, D, s);
    case 32: return dispatch_d<T, 32>(a, D, s);
    case 64: return dispatch_d<T, 64>(a, D, s);
    case 128: return dispatch_d<T, 128>(a, D, s);
  }
  return fail(FBSA_EUNSUPPORTED, "fbsa_fwd: block size %lld not in {16,32,64,128}", (long long)bs);
}

int run_fwd(const fbsa_attn_desc *d, const FwdArgs &a, hipStream_t s) {
  switch (d->dtype) {
    case FBSA_BF16: return dispatch_bs<bf16>(a, d->bs, d->D, s);
    case FBSA_F16: return dispatch_bs<f16>(a, d->bs, d->D, s);
    case FBSA_F32: return dispatch_bs<float>(a, d->bs, d->D, s);
  }
  return fail(FBSA_EINVAL, "fbsa_fwd: bad dtype %d", d->dtype);
}

}  // namespace fbsa
