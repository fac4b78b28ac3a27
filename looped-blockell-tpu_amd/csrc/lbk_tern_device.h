// lbk_tern_device.h — device helpers shared by the ternary kernels: 2-bit unpacking
// and the per-row fixed-point form of the block scales.
#pragma once

#include "lbk_device.h"

namespace lbk {

// code -> int8 table for v_perm: bytes [0]=0x00 [1]=0x01 [2]=0x00 [3]=0xff
constexpr uint32_t kTernLut = 0xFF000100u;

__device__ __forceinline__ uint32_t unpack4(uint32_t word, int q) {
  return __builtin_amdgcn_perm(0u, kTernLut, (word >> (2 * q)) & 0x03030303u);
}

// ---------------------------------------------------------------------------
// fixed-point form of one block row's scales
// ---------------------------------------------------------------------------
struct RowFix {
  int e;        // exponent: scale = m * 2^-e
  float mult;   // 2^-e as float
};

template <int B>
__device__ __forceinline__ RowFix row_fixed_point(const float* __restrict__ s, const int32_t* __restrict__ col,
                                                  int K, int C) {
  float smax = 0.f;
  int ka = 0;
  for (int k = 0; k < K; ++k) {
    const int c = col[k];
    if (c >= 0 && c < C) {
      smax = fmaxf(smax, fabsf(s[k]));
      ++ka;
    }
  }
  RowFix f{0, 1.0f};
  // no live block, all-zero, NaN or infinite scales: leave the row unscaled (m = rint(s))
  if (ka == 0 || !(smax > 0.f) || !(smax < INFINITY)) return f;
  int64_t lim = (int64_t)2147483647 / ((int64_t)ka * B * 128);
  if (lim < 1) lim = 1;
  const float mmax = (float)(lim < 65535 ? lim : 65535);
  int e = ilogbf(mmax) - ilogbf(smax);  // within +-1 of the answer; both loops are bounded
  for (int it = 0; it < 4 && ldexpf(smax, e) > mmax; ++it) --e;
  for (int it = 0; it < 4 && ldexpf(smax, e + 1) <= mmax; ++it) ++e;
  f.e = e;
  f.mult = ldexpf(1.0f, -e);
  return f;
}

}  // namespace lbk
