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
#include <stdlib.h>

#include "fbsa_common.h"
#include "fbsa_internal.h"

namespace fbsa {

enum { KIND_FULL = 0, KIND_DIAG = 1, KIND_ABS = 2, KIND_PAD = 3 };

// LDS bytes per workgroup for the K/V prefetch ring (sets the ring depth).
#ifndef FBSA_FWD_LDS_BUDGET
#define FBSA_FWD_LDS_BUDGET 32768
#endif

// QT: 16-query tiles per wave (each wave owns 16*QT query rows, so a WG has
// BS/(16*QT) waves). KCO / NSO override the key-chunk size and the ring depth
// (0 = derived).
template <typename T, int BS, int D, int QT = 1, int KCO = 0, int NSO = 0> struct FwdCfg {
  static constexpr int ES = sizeof(T);
  static constexpr int NW = BS / (16 * QT);
  static constexpr int NT = NW * 64;
  // keys per chunk: 64, 32 at d 256 (16-bit), 16 for fp32 at d >= 128 (registers)
  static constexpr int KCW = ES == 4 && D >= 128 ? 16 : (D >= 256 ? 32 : 64);
  static constexpr int KC0 = BS < KCW ? BS : KCW;
  static constexpr int KC = KCO ? KCO : KC0;
  static constexpr int NCH = BS / KC;
  static constexpr int CPR = D * ES / 16;
  static constexpr int TILE_BYTES = KC * D * ES;
  static constexpr int STAGE_BYTES = 2 * TILE_BYTES;
  static constexpr int LPT = STAGE_BYTES / (NT * 16);
  static constexpr int NS0 = FBSA_FWD_LDS_BUDGET / STAGE_BYTES;
  static constexpr int NSTAGE = NSO ? NSO : (NS0 < 2 ? 2 : (NS0 > 4 ? 4 : NS0));
  static_assert(NW >= 1, "block too small for the query tiling");
  static_assert(NSTAGE >= 2, "the single-barrier ring needs two stages");
  static_assert(LPT * NT * 16 == STAGE_BYTES, "stage must split evenly over threads");
  static_assert(TILE_BYTES % 1024 == 0, "tile must be whole wave-loads");
};

// K fragments requested all at once before the score MFMAs (16-bit types)
#ifndef FBSA_FWD_KFIRST
#define FBSA_FWD_KFIRST 1
#endif

// Walk a row's selected key blocks in ascending block index (lists of up to 64
// valid slots). The softmax does not depend on the order; the workgroups that
// run together on an XCD then read nearby key blocks at about the same time,
// so more of the gathered K/V tiles are L2 hits.
#ifndef FBSA_FWD_SORT
#define FBSA_FWD_SORT 1
#endif

template <int N> __device__ __forceinline__ void wait_pending(int pending_chunks) {
  // wait until at most pending_chunks * LPT DMA loads are outstanding (N = LPT)
  switch (pending_chunks) {
    case 0: wait_vmcnt<0>(); break;
    case 1: wait_vmcnt<(N < 64 ? N : 63)>(); break;
    case 2: wait_vmcnt<(2 * N < 64 ? 2 * N : 63)>(); break;
    case 3: wait_vmcnt<(3 * N < 64 ? 3 * N : 63)>(); break;
    case 4: wait_vmcnt<(4 * N < 64 ? 4 * N : 63)>(); break;
    default: wait_vmcnt<(5 * N < 64 ? 5 * N : 63)>(); break;
  }
}

template <typename T, int BS, int D, int QT = 1, int KCO = 0, int NSO = 0, bool DENSE = false>
__global__ __launch_bounds__(BS * 4 / QT) void fwd_kernel(FwdArgs a) {
  using C = FwdCfg<T, BS, D, QT, KCO, NSO>;
  constexpr bool F32 = sizeof(T) == 4;
  extern __shared__ __attribute__((aligned(16))) char smem[];
  char *stages = smem;
  int *s_blk = (int *)(smem + C::NSTAGE * C::STAGE_BYTES);
  int *s_kind = s_blk + a.kk;
  float *s_gate = (float *)(s_kind + a.kk);
  __shared__ int s_nvalid;

  const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63, g = lane >> 4, p = lane & 15;
  // launch order: consecutive query blocks round-robin over the XCDs
  // (measured faster for the gathered K/V than XCD-contiguous ranges), the
  // query heads of one KV group back to back on one XCD (they share the K/V
  // tiles)
  int hin;
  int64_t t = gqa_unit(blockIdx.x, (int64_t)gridDim.x / a.grp, a.grp, &hin);
  // (32-bit division: launch indices are below 2^31)
  const uint32_t t32 = (uint32_t)t;
  const int64_t i = a.i0 + t32 % (uint32_t)a.ni;
  const int hk = (int)(t32 / (uint32_t)a.ni % (uint32_t)a.Hkv);
  const int64_t b = t32 / (uint32_t)a.ni / (uint32_t)a.Hkv;
  const int hq = hk * a.grp + hin;
  const int hs = a.hsel == 1 ? 0 : hk;

  // ---- 1. plan: compact list of valid slots with their mask kind and gate ----
  // (dense: slot s is block s for the blocks below l_valid, and up to i when
  // causal; kinds follow from the block index, no table)
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
      }
      nout += __popcll(m);
    }
    if (lane == 0) s_nvalid = nout;
    if (FBSA_FWD_SORT && nout > 1 && nout <= 64) {
      // rank of each entry by (block, slot); equal blocks keep their slot order
      int j = 0x7fffffff, kind = 0;
      float gt = 0.f;
      if (lane < nout) { j = s_blk[lane]; kind = s_kind[lane]; gt = s_gate[lane]; }
      int rank = 0;
      for (int m = 0; m < nout; ++m) {
        const int jm = s_blk[m];
        rank += jm < j || (jm == j && m < lane);
      }
      __builtin_amdgcn_wave_barrier();
      if (lane < nout) { s_blk[rank] = j; s_kind[rank] = kind; s_gate[rank] = gt; }
    }
  }

  // ---- 2. Q fragments (B operands of S^T = K Q^T), one per query tile ----
  int tq[QT];  // query rows (within the block) of this lane's columns
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) tq[qt] = (w * QT + qt) * 16 + p;
  constexpr int QF = F32 ? D / 4 : D / 32;
  s16x8 qf16[QT][F32 ? 1 : QF];
  float qf32[QT][F32 ? QF : 1];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    const T *qrow = (const T *)a.q + b * a.sq[0] + hq * a.sq[1] + (i * BS + tq[qt]) * a.sq[2];
    if constexpr (F32) {
#pragma unroll
      for (int ks = 0; ks < QF; ++ks) qf32[qt][ks] = ((const float *)qrow)[4 * ks + g];
    } else {
#pragma unroll
      for (int ks = 0; ks < QF; ++ks) qf16[qt][ks] = *(const s16x8 *)(qrow + 32 * ks + 8 * g);
    }
  }

  // Direct-to-LDS copy plan: this thread's LPT 16-byte loads of a K/V chunk.
  // Which tensor a load reads is uniform across a wave (a tile is a whole
  // number of 1 KiB wave-loads); the per-lane byte offset from the chunk's first
  // row is fixed, so each issue is a scalar base plus a precomputed offset.
  int32_t doff[C::LPT];
#pragma unroll
  for (int n = 0; n < C::LPT; ++n) {
    const int wl = n * C::NW + w;
    const int u = wl * 64 + lane;
    const int part = u / (C::KC * C::CPR);
    const int rem = u - part * (C::KC * C::CPR);
    const int row = rem / C::CPR, pos = rem % C::CPR;
    const int chunk = pos ^ swz(row, C::CPR);
    doff[n] = (int32_t)(((int64_t)row * (part ? a.sv[2] : a.sk[2]) + chunk * (16 / C::ES)) * C::ES);
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

  const char *kbase = (const char *)((const T *)a.k + b * a.sk[0] + hk * a.sk[1]);
  const char *vbase = (const char *)((const T *)a.v + b * a.sv[0] + hk * a.sv[1]);
  const int64_t kstep = a.sk[2] * C::ES, vstep = a.sv[2] * C::ES;
  auto issue = [&](int c) {
    const int slot = c / C::NCH, ch = c % C::NCH;
    const int64_t row0 = (int64_t)__builtin_amdgcn_readfirstlane(blk_of(slot) * BS + ch * C::KC);
    const char *kb = kbase + row0 * kstep, *vb = vbase + row0 * vstep;
    char *st = stages + (c % C::NSTAGE) * C::STAGE_BYTES;
#pragma unroll
    for (int n = 0; n < C::LPT; ++n) {
      const bool part = (n * C::NW + w) * 64 >= C::KC * C::CPR;  // wave-uniform
      g2lds16_s(part ? vb : kb, (unsigned)doff[n], st + (n * C::NW + w) * 1024);
    }
  };

  // Online softmax in the log2 domain with a lazily moved reference max: the
  // accumulators are rescaled only when a score exceeds the reference by more
  // than TAU (so p <= 2^TAU); each lane checks its own scores and only when
  // one does is the per-query chunk max formed across lanes.
  constexpr float TAU = 8.f;
  // l_run: this lane's part of the row sum of P, summed in fp32 from the
  // unrounded exponentials (the LSE the backward recomputes P from is then not
  // perturbed by the rounding of P to the MFMA operand type)
  float m_run[QT], l_run[QT];
  f32x4 oacc[QT][D / 16];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    m_run[qt] = -INFINITY;
    l_run[qt] = 0.f;
#pragma unroll
    for (int mt = 0; mt < D / 16; ++mt) oacc[qt][mt] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

#pragma unroll
  for (int c = 0; c < C::NSTAGE - 1; ++c)
    if (c < nchunks) issue(c);
  // the register-operand loads above and the first stages have landed (issued
  // together, so their latencies overlap): the compiler then waits for nothing
  // inside the ring loop, where its own waits would also drain the prefetch
  wait_vmcnt<0>();


  // per-lane LDS bases of the operand reads (16-bit types): each read is a base
  // plus the stage address plus a compile-time offset
  constexpr int KL = QF < 4 ? QF : 4, VL = D / 16 < 8 ? D / 16 : 8;
  unsigned kbl[KL], vbl[VL];
#pragma unroll
  for (int l = 0; l < KL; ++l) kbl[l] = tile_kbase(l, g, p, C::CPR);
#pragma unroll
  for (int l = 0; l < VL; ++l) vbl[l] = tile_vbase(l, g, p, C::CPR);

  for (int c = 0; c < nchunks; ++c) {
    // chunk c has landed once at most min(ahead, NSTAGE-2) later chunks are in flight
    const int ahead = nchunks - 1 - c;
    wait_pending<C::LPT>(ahead < C::NSTAGE - 2 ? ahead : C::NSTAGE - 2);
    // one barrier per chunk: every wave has landed its part of chunk c and
    // finished reading chunk c-1, whose stage the prefetch below overwrites
    lds_barrier();
    if (c + C::NSTAGE - 1 < nchunks) issue(c + C::NSTAGE - 1);

    const char *Ks = stages + (c % C::NSTAGE) * C::STAGE_BYTES;
    const char *Vs = Ks + C::TILE_BYTES;
    const int slot = c / C::NCH, ch = c % C::NCH;
    const int kind = kind_of(slot);
    const float gt = DENSE ? 0.f : s_gate[slot];
    const int64_t j = blk_of(slot);

    // V^T fragments for the PV product, shared by the query tiles (16-bit types)
    constexpr int KV2 = C::KC >= 32 ? C::KC / 32 : 1;
    s16x4 vlo[F32 ? 1 : D / 16][KV2], vhi[F32 ? 1 : D / 16][KV2];
    auto read_v = [&]() {
      // d tile mt, rows 32 k2 + 4g + p/4 (+16): lane base vbl[mt % 8] plus the
      // stage address plus a constant
      const unsigned vs = (unsigned)(uintptr_t)Vs;
      static_for<(F32 ? 0 : D / 16)>([&](auto MT) {
        constexpr int mt = decltype(MT)::value;
        static_for<KV2>([&](auto K2) {
          constexpr int k2 = decltype(K2)::value;
          constexpr int off = (mt / 8) * 256 + k2 * 512 * C::CPR;
          vlo[mt][k2] = lds_read_tr16_at<off>(vs + vbl[mt % 8]);
          if constexpr (C::KC >= 32) vhi[mt][k2] = lds_read_tr16_at<off + 256 * C::CPR>(vs + vbl[mt % 8]);
        });
      });
    };

    // S^T (KC keys x 16 queries per tile); each K fragment feeds every tile
    f32x4 sacc[QT][C::KC / 16];
#pragma unroll
    for (int m = 0; m < C::KC / 16; ++m)
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) sacc[qt][m] = f32x4{0.f, 0.f, 0.f, 0.f};
    if constexpr (F32) {
#pragma unroll
      for (int m = 0; m < C::KC / 16; ++m) {
        const int row = 16 * m + p;
#pragma unroll
        for (int ks = 0; ks < QF; ++ks) {
          const float kf = *(const float *)(Ks + (row * C::CPR + (ks ^ swz(row, C::CPR))) * 16 + g * 4);
#pragma unroll
          for (int qt = 0; qt < QT; ++qt) sacc[qt][m] = mfma_f32_16x16x4(kf, qf32[qt][ks], sacc[qt][m]);
          // at d 256, loads are not hoisted more than 16 MFMAs ahead (registers)
          if constexpr (D >= 256) if (ks % 16 == 15) asm volatile("" ::: "memory");
        }
      }
    } else if constexpr (FBSA_FWD_KFIRST) {
      // every K fragment of the chunk is requested at once and each MFMA waits
      // only for its own (LDS reads complete in order); the V^T reads follow,
      // so their latency overlaps the MFMAs in flight and the softmax
      constexpr int NK = C::KC / 16 * QF;
      s16x8 kf[C::KC / 16][QF];
      const unsigned ksu = (unsigned)(uintptr_t)Ks;
      static_for<NK>([&](auto F) {
        constexpr int m = decltype(F)::value / QF, ks = decltype(F)::value % QF;
        kf[m][ks] = lds_read_b128_at<(ks / 4) * 256 + m * 256 * C::CPR>(ksu + kbl[ks % 4]);
      });
#pragma unroll
      for (int m = 0; m < C::KC / 16; ++m)
#pragma unroll
        for (int ks = 0; ks < QF; ++ks) {
          lds_wait_upto(NK - 1 - (m * QF + ks));
          lds_ready(kf[m][ks]);
#pragma unroll
          for (int qt = 0; qt < QT; ++qt) sacc[qt][m] = Mfma16<T>::run(kf[m][ks], qf16[qt][ks], sacc[qt][m]);
        }
      read_v();
    } else {
      // V^T requested first, so its LDS latency overlaps the score MFMAs
      read_v();
#pragma unroll
      for (int m = 0; m < C::KC / 16; ++m) {
        const int row = 16 * m + p;
#pragma unroll
        for (int ks = 0; ks < QF; ++ks) {
          const s16x8 kf = *(const s16x8 *)(Ks + (row * C::CPR + ((4 * ks + g) ^ swz(row, C::CPR))) * 16);
#pragma unroll
          for (int qt = 0; qt < QT; ++qt) sacc[qt][m] = Mfma16<T>::run(kf, qf16[qt][ks], sacc[qt][m]);
        }
      }
    }

    // mask: key row u (within block j) is valid iff u <= lim (uniform branch
    // skips the compares for unmasked chunks, the common case)
    if (kind != KIND_FULL) {
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) {
        const int64_t lim64 = kind == KIND_DIAG ? (int64_t)tq[qt]
                              : kind == KIND_PAD  ? a.l_valid - j * BS - 1
                                                  : ((i - j) * BS + tq[qt] < a.l_valid - j * BS - 1
                                                         ? (i - j) * BS + tq[qt]
                                                         : a.l_valid - j * BS - 1);
        const int lim = (int)(lim64 < -1 ? -1 : lim64) - ch * C::KC - 4 * g;  // compare against 16m + r
#pragma unroll
        for (int m = 0; m < C::KC / 16; ++m)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (16 * m + r > lim) sacc[qt][m][r] = -INFINITY;
      }
    }

    // lazy reference max
    float lmax[QT];
    bool need = false;
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
      float mx = fmaxf(fmaxf(sacc[qt][0][0], sacc[qt][0][1]), fmaxf(sacc[qt][0][2], sacc[qt][0][3]));
#pragma unroll
      for (int m = 1; m < C::KC / 16; ++m)
        mx = fmaxf(fmaxf(mx, fmaxf(sacc[qt][m][0], sacc[qt][m][1])), fmaxf(sacc[qt][m][2], sacc[qt][m][3]));
      lmax[qt] = mx * a.scale2 + gt;  // -inf when every key of the lane is masked
      need |= lmax[qt] > m_run[qt] + TAU;
    }
    if (__ballot(need)) {
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) {
        float mc = fmaxf(lmax[qt], shfl_xor_f(lmax[qt], 16));
        mc = fmaxf(mc, shfl_xor_f(mc, 32));            // the query's chunk max, same on its 4 lanes
        if (mc > m_run[qt] + TAU) {
          const float alpha = __builtin_amdgcn_exp2f(m_run[qt] - mc);  // 0 when m_run = -inf
          l_run[qt] *= alpha;
#pragma unroll
          for (int mt = 0; mt < D / 16; ++mt)
#pragma unroll
            for (int r = 0; r < 4; ++r) oacc[qt][mt][r] *= alpha;
          m_run[qt] = mc;
        }
      }
    }

#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
      const float off = gt - (m_run[qt] == -INFINITY ? 0.f : m_run[qt]);
      float sv[C::KC / 16][4];
#pragma unroll
      for (int m = 0; m < C::KC / 16; ++m)
#pragma unroll
        for (int r = 0; r < 4; ++r) sv[m][r] = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[qt][m][r], a.scale2, off));

      // row sums of the unrounded P (this lane's keys), then O^T += V^T P^T
      {
        float psum = 0.f;
#pragma unroll
        for (int m = 0; m < C::KC / 16; ++m)
#pragma unroll
          for (int r = 0; r < 4; ++r) psum += sv[m][r];
        l_run[qt] += psum;
      }
      if constexpr (F32) {
#pragma unroll
        for (int mt = 0; mt < D / 16; ++mt)
#pragma unroll
          for (int m = 0; m < C::KC / 16; ++m)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const int vrow = 16 * m + 4 * g + r;
              const float vf = *(const float *)(Vs + (vrow * C::CPR + ((4 * mt + (p >> 2)) ^ swz(vrow, C::CPR))) * 16 + (p & 3) * 4);
              oacc[qt][mt] = mfma_f32_16x16x4(vf, sv[m][r], oacc[qt][mt]);
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
        if (qt == 0) lds_wait_all();
#pragma unroll
        for (int mt = 0; mt < D / 16; ++mt)
#pragma unroll
          for (int k2 = 0; k2 < C::KC / 32; ++k2) {
            lds_ready(vlo[mt][k2]);
            lds_ready(vhi[mt][k2]);
            const s16x4 lo = vlo[mt][k2], hi = vhi[mt][k2];
            const s16x8 vf = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            oacc[qt][mt] = Mfma16<T>::run(vf, pf[k2], oacc[qt][mt]);
          }
      } else {
        // KC == 16: one 16x16x16 MFMA per d tile
        s16x4 pf;
#pragma unroll
        for (int r = 0; r < 4; ++r) pf[r] = bits16<T>((T)sv[0][r]);
        if (qt == 0) lds_wait_all();
#pragma unroll
        for (int mt = 0; mt < D / 16; ++mt) {
          lds_ready(vlo[mt][0]);
          oacc[qt][mt] = Mfma16<T>::run16(vlo[mt][0], pf, oacc[qt][mt]);
        }
      }
    }
  }

  // ---- 4. epilogue ----
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    // the query's four lanes (g = 0..3) hold its row sum in parts
    float lt = l_run[qt] + shfl_xor_f(l_run[qt], 16);
    lt += shfl_xor_f(lt, 32);
    const float inv = lt > 0.f ? 1.f / lt : 0.f;
    T *orow = (T *)a.o + b * a.so[0] + hq * a.so[1] + (i * BS + tq[qt]) * a.so[2];
    const T *ogrow = a.og ? (const T *)a.og + b * a.sog[0] + hq * a.sog[1] + (i * BS + tq[qt]) * a.sog[2] : nullptr;
#pragma unroll
    for (int mt = 0; mt < D / 16; ++mt) {
      const int d0 = 16 * mt + 4 * g;
      float y[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) y[r] = oacc[qt][mt][r] * inv;
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
      const int64_t li = (b * a.Hq + hq) * a.L + i * BS + tq[qt];
      a.lse[li] = lt > 0.f ? (m_run[qt] + __log2f(lt)) * kLn2 : -INFINITY;
    }
  }
}

template <typename T, int BS, int D, int QT = 1, int KCO = 0, int NSO = 0, bool DENSE = false>
static int launch_fwd_as(const FwdArgs &a, hipStream_t stream) {
  using C = FwdCfg<T, BS, D, QT, KCO, NSO>;
  const size_t lds = (size_t)C::NSTAGE * C::STAGE_BYTES + (DENSE ? 0 : (size_t)a.kk * 12);
  if (lds > 160 * 1024 - 64) return fail(FBSA_EUNSUPPORTED, "fbsa_fwd: kk=%lld needs %zu bytes of LDS", (long long)a.kk, lds);
  {
    const int e = lds_optin((const void *)fwd_kernel<T, BS, D, QT, KCO, NSO, DENSE>, lds, "hipFuncSetAttribute(fwd)");
    if (e) return e;
  }
  const int64_t nwg = a.B * a.Hq * a.ni;
  if (nwg == 0) return FBSA_OK;
  hipLaunchKernelGGL((fwd_kernel<T, BS, D, QT, KCO, NSO, DENSE>), dim3((unsigned)nwg), dim3(C::NT), lds, stream, a);
  return hip_check(hipGetLastError(), "fwd_kernel launch");
}

// the dense (list-less) form is its own instantiation, so the list path's code
// is unchanged by it
template <typename T, int BS, int D, int QT = 1, int KCO = 0, int NSO = 0>
static int launch_fwd(const FwdArgs &a, hipStream_t stream) {
  return a.dense ? launch_fwd_as<T, BS, D, QT, KCO, NSO, true>(a, stream)
                 : launch_fwd_as<T, BS, D, QT, KCO, NSO, false>(a, stream);
}

// query tiles per wave at d = 256 (16-bit types, blocks of 64 or more rows)
#ifndef FBSA_FWD_QT256
#define FBSA_FWD_QT256 1
#endif
#ifndef FBSA_FWD_NS256
#define FBSA_FWD_NS256 0
#endif

template <typename T, int BS> static int dispatch_d(const FwdArgs &a, int64_t D, hipStream_t s) {
  constexpr int QT256 = (sizeof(T) == 2 && BS >= 64) ? FBSA_FWD_QT256 : 1;
  constexpr int NS256 = (sizeof(T) == 2 && BS >= 64) ? FBSA_FWD_NS256 : 0;
  switch (D) {
    case 32: return launch_fwd<T, BS, 32>(a, s);
    case 64: return launch_fwd<T, BS, 64>(a, s);
    case 128: return launch_fwd<T, BS, 128>(a, s);
    case 256: return launch_fwd<T, BS, 256, QT256, 0, NS256>(a, s);
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
