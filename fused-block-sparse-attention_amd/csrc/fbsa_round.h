// Rounding and element loads shared by the selection kernels (gfx950).
#pragma once
#include "fbsa_common.h"

namespace fbsa {

// ---------------------------------------------------------------- rounding
// torch rounds a bf16/fp16 reduction twice: the exact value to the fp32
// accumulator, then fp32 -> dtype (both RNE). The fp32 step is kept opaque so
// the compiler cannot fold the pair into one double -> 16-bit rounding, which
// differs when the fp32 value lands exactly on a 16-bit midpoint.
__device__ __forceinline__ float rne_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return __uint_as_float(0x7FC00000u);  // NaN
  u += 0x7FFFu + ((u >> 16) & 1u);
  return __uint_as_float(u & 0xFFFF0000u);
}
template <typename T> __device__ __forceinline__ float round_dt_f(float f) {
  if constexpr (sizeof(T) == 4) return f;
  else if constexpr (__is_same(T, bf16)) return rne_bf16(f);
  else {
    asm volatile("" : "+v"(f));
    return (float)(T)f;
  }
}
template <typename T> __device__ __forceinline__ float round_dt(double x) {
  float f = (float)x;  // RNE to fp32
  asm volatile("" : "+v"(f));
  return round_dt_f<T>(f);
}

// 16-bit pattern -> fp32 (exact)
template <typename T> __device__ __forceinline__ float half_bits_to_f32(uint32_t h);
template <> __device__ __forceinline__ float half_bits_to_f32<bf16>(uint32_t h) { return __uint_as_float(h << 16); }
template <> __device__ __forceinline__ float half_bits_to_f32<f16>(uint32_t h) {
  const unsigned short hs = (unsigned short)h;
  _Float16 x;
  __builtin_memcpy(&x, &hs, 2);
  return (float)x;
}

// 8 consecutive elements (16 bytes) -> fp64
template <typename T> __device__ __forceinline__ void load8(const T *p, double *v) {
  const uint4 r = *(const uint4 *)p;
  const uint32_t w[4] = {r.x, r.y, r.z, r.w};
  if constexpr (sizeof(T) == 4) {
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = (double)__uint_as_float(w[e]);
    const uint4 r2 = *(const uint4 *)(p + 4);
    const uint32_t w2[4] = {r2.x, r2.y, r2.z, r2.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) v[4 + e] = (double)__uint_as_float(w2[e]);
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[2 * e] = (double)half_bits_to_f32<T>(w[e] & 0xFFFFu);
      v[2 * e + 1] = (double)half_bits_to_f32<T>(w[e] >> 16);
    }
  }
}

}  // namespace fbsa
