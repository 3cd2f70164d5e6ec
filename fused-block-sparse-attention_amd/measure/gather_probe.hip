// Random block-gather bandwidth probe for MI355X (gfx950).
//
// Measures how fast workgroups can read randomly chosen blocks of a device
// buffer, as the block-sparse forward reads its selected K/V tiles, for a
// range of footprints (the size of the region the blocks are drawn from):
// within the L2s, within the 256 MB Infinity Cache, and beyond. Also replays
// the forward's own access pattern at configuration 3 (8 heads x 4096 query
// blocks, each reading its own block and 16 blocks drawn uniformly from the
// strictly earlier ones, K and V tiles of 8 KB each) without any compute, which
// is the gather-only time the forward kernel cannot beat with this data.
//
// Every block index is drawn on the host inside the buffer, so every load is in
// bounds. Each thread keeps 16 loads of 16 bytes in flight; the loaded words are
// folded into one value per workgroup (written out, so no load is dead).
//
// Usage: measure/gather_probe    (prints one table; built by `make measure`)
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>

#include <algorithm>
#include <random>
#include <vector>

#define CHECK(x)                                                                              \
  do {                                                                                        \
    hipError_t e_ = (x);                                                                      \
    if (e_ != hipSuccess) {                                                                   \
      fprintf(stderr, "%s:%d %s: %s\n", __FILE__, __LINE__, #x, hipGetErrorString(e_));       \
      exit(1);                                                                                \
    }                                                                                         \
  } while (0)

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int kBlockBytes = 8192;                          // one K or V tile (64 rows x 64 bf16)
constexpr int kU4PerBlock = kBlockBytes / 16;              // 512 16-byte words
constexpr int kLoadsPerBlock = kU4PerBlock / kThreads;     // 2 per thread
constexpr int kBlocksInFlight = 8;                         // 16 loads of 16 bytes per thread

// Each workgroup reads nb blocks: block b of workgroup w starts at word
// idx[w * nb + b] * kU4PerBlock of buf (K) and, with two_tensors, the same
// block of buf2 (V).
template <bool NT>
__global__ __launch_bounds__(kThreads) void gather_kernel(const u32x4 *__restrict__ buf, const u32x4 *__restrict__ buf2,
                                                        const uint32_t *__restrict__ idx, int nb, int two_tensors,
                                                        uint32_t *__restrict__ out) {
  const uint32_t *my = idx + (size_t)blockIdx.x * nb;
  uint32_t acc = 0;
  const int t = threadIdx.x;
  for (int b0 = 0; b0 < nb; b0 += kBlocksInFlight) {
    u32x4 v[kBlocksInFlight * kLoadsPerBlock];
    const int n = min(kBlocksInFlight, nb - b0);
#pragma unroll
    for (int u = 0; u < kBlocksInFlight; ++u) {
      if (u < n) {
        const u32x4 *base = (two_tensors && (u & 1) ? buf2 : buf) + (size_t)my[b0 + u] * kU4PerBlock;
#pragma unroll
        for (int l = 0; l < kLoadsPerBlock; ++l) {
          if constexpr (NT)
            v[u * kLoadsPerBlock + l] = __builtin_nontemporal_load(base + l * kThreads + t);
          else
            v[u * kLoadsPerBlock + l] = base[l * kThreads + t];
        }
      }
    }
#pragma unroll
    for (int u = 0; u < kBlocksInFlight; ++u)
      if (u < n)
#pragma unroll
        for (int l = 0; l < kLoadsPerBlock; ++l) {
          const u32x4 x = v[u * kLoadsPerBlock + l];
          acc ^= x.x ^ x.y ^ x.z ^ x.w;
        }
  }
  out[(size_t)blockIdx.x * kThreads + t] = acc;
}

struct Result {
  double ms, tbs;
};

static Result run(const u32x4 *buf, const u32x4 *buf2, const std::vector<uint32_t> &h_idx, int nb, int two, bool nt,
                  uint32_t *d_out, uint32_t *d_idx) {
  const int nwg = (int)(h_idx.size() / nb);
  CHECK(hipMemcpy(d_idx, h_idx.data(), h_idx.size() * 4, hipMemcpyHostToDevice));
  hipEvent_t e0, e1;
  CHECK(hipEventCreate(&e0));
  CHECK(hipEventCreate(&e1));
  auto launch = [&]() {
    if (nt)
      hipLaunchKernelGGL(gather_kernel<true>, dim3(nwg), dim3(kThreads), 0, 0, buf, buf2, d_idx, nb, two, d_out);
    else
      hipLaunchKernelGGL(gather_kernel<false>, dim3(nwg), dim3(kThreads), 0, 0, buf, buf2, d_idx, nb, two, d_out);
  };
  for (int i = 0; i < 3; ++i) launch();
  CHECK(hipGetLastError());
  const int reps = 10;
  CHECK(hipEventRecord(e0, 0));
  for (int i = 0; i < reps; ++i) launch();
  CHECK(hipEventRecord(e1, 0));
  CHECK(hipEventSynchronize(e1));
  float ms = 0;
  CHECK(hipEventElapsedTime(&ms, e0, e1));
  CHECK(hipEventDestroy(e0));
  CHECK(hipEventDestroy(e1));
  const double bytes = (double)h_idx.size() * kBlockBytes;
  return {ms / reps, bytes / (ms / reps * 1e-3) / 1e12};
}

int main() {
  const size_t max_bytes = (size_t)2 << 30;  // 2 GiB
  u32x4 *buf = nullptr, *buf2 = nullptr;
  CHECK(hipMalloc(&buf, max_bytes));
  CHECK(hipMalloc(&buf2, (size_t)256 << 20));
  CHECK(hipMemset(buf, 1, max_bytes));
  CHECK(hipMemset(buf2, 2, (size_t)256 << 20));
  const int nwg = 32768, nb = 32;           // 32768 workgroups x 32 blocks of 8 KB = 8.6 GB per launch
  uint32_t *d_out = nullptr, *d_idx = nullptr;
  CHECK(hipMalloc(&d_out, (size_t)nwg * kThreads * 4));
  CHECK(hipMalloc(&d_idx, (size_t)8 * 4096 * 34 * 4 > (size_t)nwg * nb * 4 ? (size_t)8 * 4096 * 34 * 4
                                                                           : (size_t)nwg * nb * 4));
  std::mt19937_64 rng(12345);
  std::vector<uint32_t> idx((size_t)nwg * nb);

  printf("# random 8 KB block gathers, %d workgroups x %d blocks per launch (%.2f GB), 16 x 16-byte loads in flight "
         "per thread; average of 10 launches after 3 warm-up launches\n",
         nwg, nb, (double)nwg * nb * kBlockBytes / 1e9);
  printf("%-44s %10s %10s %10s\n", "pattern", "footprint", "ms", "TB/s");
  const size_t fps_mb[] = {2, 4, 8, 16, 32, 64, 128, 192, 256, 384, 512, 1024, 2048};
  for (int nt = 0; nt < 2; ++nt) {
    for (size_t fmb : fps_mb) {
      const uint32_t nblocks = (uint32_t)((fmb << 20) / kBlockBytes);
      std::uniform_int_distribution<uint32_t> U(0, nblocks - 1);
      for (auto &x : idx) x = U(rng);
      Result r = run(buf, buf, idx, nb, 0, nt, d_out, d_idx);
      char name[64];
      snprintf(name, sizeof name, "uniform random%s", nt ? ", nontemporal loads" : "");
      printf("%-44s %7zu MB %10.3f %10.2f\n", name, fmb, r.ms, r.tbs);
    }
  }
  // per-XCD regions: workgroup w runs on XCD w % 8 (round-robin dispatch) and
  // draws its blocks from region w % 8 only (8 disjoint regions)
  for (size_t fmb : {16, 32, 64, 256, 1024}) {
    const uint32_t nblocks = (uint32_t)((fmb << 20) / kBlockBytes);
    const uint32_t per = nblocks / 8;
    std::uniform_int_distribution<uint32_t> U(0, per - 1);
    for (int w = 0; w < nwg; ++w)
      for (int b = 0; b < nb; ++b) idx[(size_t)w * nb + b] = (uint32_t)(w % 8) * per + U(rng);
    Result r = run(buf, buf, idx, nb, 0, false, d_out, d_idx);
    printf("%-44s %7zu MB %10.3f %10.2f\n", "uniform within the XCD's eighth", fmb, r.ms, r.tbs);
  }
  // sequential blocks (each workgroup reads nb consecutive blocks)
  {
    const uint32_t nblocks = (uint32_t)(max_bytes / kBlockBytes);
    for (int w = 0; w < nwg; ++w)
      for (int b = 0; b < nb; ++b) idx[(size_t)w * nb + b] = ((uint32_t)w * nb + b) % nblocks;
    Result r = run(buf, buf, idx, nb, 0, false, d_out, d_idx);
    printf("%-44s %7zu MB %10.3f %10.2f\n", "sequential", (size_t)2048, r.ms, r.tbs);
  }
  // the forward's access pattern at configuration 3: 8 heads x 4096 query
  // blocks, each reading 17 blocks (own + 16 uniform from the strictly earlier
  // ones; the first 16 query blocks re-read their own) as a K tile (buf) and a V
  // tile (buf2); tiles of head h at block j live at (h * 4096 + j) * 8 KB.
  // Workgroup order: head-major, consecutive query blocks round-robin over the
  // XCDs (the forward's launch order), or one head per XCD.
  for (int order = 0; order < 2; ++order) {
    const int H = 8, NQ = 4096, KK = 17;
    std::vector<uint32_t> fidx((size_t)H * NQ * KK * 2);
    for (int w = 0; w < H * NQ; ++w) {
      int h, i;
      if (order == 0) { h = w / NQ; i = w % NQ; }
      else { const int x = w % 8, r = w / 8; h = x; i = r; }   // workgroup w runs on XCD w % 8: head = XCD
      for (int s = 0; s < KK; ++s) {
        uint32_t j = (uint32_t)i;
        if (s > 0 && i > 0) j = std::uniform_int_distribution<uint32_t>(0, (uint32_t)i - 1)(rng);
        const uint32_t blk = (uint32_t)h * NQ + j;
        fidx[((size_t)w * KK + s) * 2 + 0] = blk;
        fidx[((size_t)w * KK + s) * 2 + 1] = blk;
      }
    }
    Result r = run(buf, buf2, fidx, KK * 2, 1, false, d_out, d_idx);
    printf("%-44s %7s %10.3f %10.2f\n",
           order == 0 ? "config-3 forward pattern, head-major" : "config-3 forward pattern, one head per XCD",
           "512 MB", r.ms, r.tbs);
  }
  CHECK(hipFree(buf));
  CHECK(hipFree(buf2));
  CHECK(hipFree(d_out));
  CHECK(hipFree(d_idx));
  return 0;
}
