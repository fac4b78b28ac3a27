// lbk_format.hip — storage-format bridges for Block-ELL weights (gfx950).
//
// Copy and integer work; every result is a pure function of the inputs (no atomics).
//   fmt_from_dense_kernel<T>  dense [out, in] (row-major, leading dimension ld) -> tiles
//                             values[r, k] = [B_in, B_out] block (r, col[r, k]) transposed
//                             through LDS (zero tile for a column outside [0, C)); one
//                             workgroup per slot
//   fmt_to_dense_kernel<T>    tiles -> dense: one workgroup per dense block (r, c) copies the
//                             last slot of row r whose column is c (the reference's scatter
//                             order: later slots overwrite earlier ones) or writes zeros
//   fmt_topk_kernel<T>        per block row: Frobenius norm of every block (16-byte loads,
//                             fixed-order fp32 sums) into LDS, then the K largest (stable:
//                             ties by column), written in ascending column order
//   fmt_ternary_check_kernel  counts 2-bit fields holding the unused code 0b10 in packed
//                             ternary words (a file check before the words reach a kernel)
// T is uint16_t (bf16) or uint32_t (fp32): the copies move bits, only the norms read values.
#include "lbk_device.h"
#include "lbk_internal.h"

namespace lbk {

template <typename T>
__device__ __forceinline__ float fmt_as_float(T v) {
  if constexpr (sizeof(T) == 2) return __uint_as_float((uint32_t)v << 16);
  else return __uint_as_float(v);
}

// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void fmt_from_dense_kernel(const T* __restrict__ dense, int64_t ld, int C, int K,
                                                             int lgB, const int32_t* __restrict__ col,
                                                             T* __restrict__ values) {
  __shared__ T tile[64 * 65];
  const int k = (int)blockIdx.x, r = (int)blockIdx.y, tid = threadIdx.x;
  const int B = 1 << lgB, BB = B * B;
  const int c = col[(int64_t)r * K + k];
  T* out = values + ((int64_t)r * K + k) * BB;
  if (c < 0 || c >= C) {
    for (int e = tid; e < BB; e += 256) out[e] = (T)0;
    return;
  }
  const T* src = dense + (int64_t)r * B * ld + (int64_t)c * B;
  for (int e = tid; e < BB; e += 256) {            // dense row D (output index), column d
    const int D = e >> lgB, d = e & (B - 1);
    tile[D * 65 + d] = src[(int64_t)D * ld + d];
  }
  __syncthreads();
  for (int e = tid; e < BB; e += 256) {            // tile row d (input index), column D
    const int d = e >> lgB, D = e & (B - 1);
    out[e] = tile[D * 65 + d];
  }
}

// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void fmt_to_dense_kernel(const T* __restrict__ values,
                                                           const int32_t* __restrict__ col, int K, int lgB,
                                                           T* __restrict__ dense, int64_t ld) {
  __shared__ T tile[64 * 65];
  __shared__ int last_s;
  const int c = (int)blockIdx.x, r = (int)blockIdx.y, tid = threadIdx.x, lane = tid & 63;
  const int B = 1 << lgB, BB = B * B;
  if (tid < 64) {
    int last = -1;
    for (int k0 = 0; k0 < K; k0 += 64) {
      const int k = k0 + lane;
      const uint64_t m = __ballot(k < K && col[(int64_t)r * K + k] == c);
      if (m) last = k0 + 63 - __builtin_clzll(m);
    }
    if (tid == 0) last_s = last;
  }
  __syncthreads();
  const int k = last_s;
  T* dst = dense + (int64_t)r * B * ld + (int64_t)c * B;
  if (k < 0) {
    for (int e = tid; e < BB; e += 256) dst[(int64_t)(e >> lgB) * ld + (e & (B - 1))] = (T)0;
    return;
  }
  const T* src = values + ((int64_t)r * K + k) * BB;
  for (int e = tid; e < BB; e += 256) {            // tile row d, column D
    const int d = e >> lgB, D = e & (B - 1);
    tile[D * 65 + d] = src[e];
  }
  __syncthreads();
  for (int e = tid; e < BB; e += 256) {            // dense row D, column d
    const int D = e >> lgB, d = e & (B - 1);
    dst[(int64_t)D * ld + d] = tile[D * 65 + d];
  }
}

// ---------------------------------------------------------------------------
// a block is before another if its norm is larger, or equal with a smaller column; NaN last
__device__ __forceinline__ bool fmt_before(float a, int ia, float b, int ib) {
  const bool na = a != a, nb = b != b;
  if (na || nb) return !na && nb ? true : (na && nb ? ia < ib : false);
  return a > b || (a == b && ia < ib);
}

// TT = 2^lgT lanes (<= 64, one wave's aligned group) share a block for its norm and a column
// for its rank; a pass covers 1024 / TT blocks (columns)
template <typename T>
__global__ __launch_bounds__(1024) void fmt_topk_kernel(const T* __restrict__ dense, int64_t ld, int C, int lgB,
                                                        int K, int lgT, int32_t* __restrict__ col_out) {
  extern __shared__ float fmt_lds[];                 // C norms, then 16 wave counts
  float* nrm = fmt_lds;
  int* wcnt = reinterpret_cast<int*>(fmt_lds + C);
  const int r = (int)blockIdx.x, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int B = 1 << lgB, TT = 1 << lgT, j = tid & (TT - 1), per = 1024 >> lgT;
  constexpr int EPC = 16 / sizeof(T);                // elements per 16-byte chunk
  const int cpr = B / EPC, nch = B * cpr;            // chunks per block row, per block
  const T* rowp = dense + (int64_t)r * B * ld;
  // norms: lane j of a group sums chunks q = j, j + TT, ... of its block in order, then a fixed
  // butterfly over the group
  for (int c0 = 0; c0 < C; c0 += per) {
    const int c = c0 + (tid >> lgT);
    float s = 0.f;
    if (c < C) {
#pragma unroll 4
      for (int q = j; q < nch; q += TT) {
        const int row = q / cpr, ch = q - row * cpr;
        const u32x4 v4 = *reinterpret_cast<const u32x4*>(rowp + (int64_t)row * ld + (int64_t)c * B + ch * EPC);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if constexpr (sizeof(T) == 2) {
            const float a = __uint_as_float(v4[i] << 16), b = __uint_as_float(v4[i] & 0xffff0000u);
            s += a * a;
            s += b * b;
          } else {
            const float a = __uint_as_float(v4[i]);
            s += a * a;
          }
        }
      }
    }
    for (int o = TT >> 1; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
    if (c < C && j == 0) nrm[c] = __builtin_sqrtf(s);
  }
  __syncthreads();
  // selection (rank < K, ranks split over the group's lanes), then compaction in column order
  int base = 0;
  for (int c0 = 0; c0 < C; c0 += per) {
    const int c = c0 + (tid >> lgT);
    int rank = 0;
    if (c < C) {
      const float x = nrm[c];
      for (int d = j; d < C; d += TT) rank += fmt_before(nrm[d], d, x, c);
    }
    for (int o = TT >> 1; o > 0; o >>= 1) rank += __shfl_xor(rank, o, 64);
    const bool sel = c < C && j == 0 && rank < K;
    const uint64_t m = __ballot(sel);
    if (lane == 0) wcnt[w] = __builtin_popcountll(m);
    __syncthreads();
    int off = base, tot = 0;
#pragma unroll
    for (int ww = 0; ww < 16; ++ww) {
      if (ww < w) off += wcnt[ww];
      tot += wcnt[ww];
    }
    const int rk = __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0));
    if (sel) col_out[(int64_t)r * K + off + rk] = c;
    base += tot;
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// one workgroup (the check runs once per loaded file): fixed-order per-thread counts, then a
// butterfly per wave and the 16 wave totals in order
__global__ __launch_bounds__(1024) void fmt_ternary_check_kernel(const uint32_t* __restrict__ words, int64_t n,
                                                                 int32_t* __restrict__ bad) {
  __shared__ int wsum[16];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  int cnt = 0;
  for (int64_t i = tid; i < n; i += 1024) {
    const uint32_t x = words[i];
    // a field is 0b10 when its high bit is set and its low bit clear
    cnt += __builtin_popcount((x >> 1) & ~x & 0x55555555u);
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) cnt += __shfl_xor(cnt, o, 64);
  if (lane == 0) wsum[w] = cnt;
  __syncthreads();
  if (tid == 0) {
    int t = 0;
    for (int i = 0; i < 16; ++i) t += wsum[i];
    bad[0] = t;
  }
}

// ---------------------------------------------------------------------------
static int lg_tile(int B) { return B == 16 ? 4 : (B == 32 ? 5 : (B == 64 ? 6 : -1)); }

int launch_fmt_from_dense(const void* dense, int64_t ld, int elem_bytes, int R, int C, int B, const int32_t* col,
                          int K, void* values, hipStream_t st) {
  const int lgB = lg_tile(B);
  if (lgB < 0 || R > 65535) return -2;
  if ((int64_t)R * K == 0) return 0;
  const dim3 grid((unsigned)K, (unsigned)R);
  if (elem_bytes == 2)
    hipLaunchKernelGGL(fmt_from_dense_kernel<uint16_t>, grid, dim3(256), 0, st, static_cast<const uint16_t*>(dense),
                       ld, C, K, lgB, col, static_cast<uint16_t*>(values));
  else
    hipLaunchKernelGGL(fmt_from_dense_kernel<uint32_t>, grid, dim3(256), 0, st, static_cast<const uint32_t*>(dense),
                       ld, C, K, lgB, col, static_cast<uint32_t*>(values));
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_fmt_to_dense(const void* values, const int32_t* col, int R, int K, int B, int C, int elem_bytes,
                        void* dense, int64_t ld, hipStream_t st) {
  const int lgB = lg_tile(B);
  if (lgB < 0 || R > 65535) return -2;
  if ((int64_t)R * C == 0) return 0;
  const dim3 grid((unsigned)C, (unsigned)R);
  if (elem_bytes == 2)
    hipLaunchKernelGGL(fmt_to_dense_kernel<uint16_t>, grid, dim3(256), 0, st, static_cast<const uint16_t*>(values),
                       col, K, lgB, static_cast<uint16_t*>(dense), ld);
  else
    hipLaunchKernelGGL(fmt_to_dense_kernel<uint32_t>, grid, dim3(256), 0, st, static_cast<const uint32_t*>(values),
                       col, K, lgB, static_cast<uint32_t*>(dense), ld);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_fmt_topk(const void* dense, int64_t ld, int elem_bytes, int R, int C, int B, int K, int32_t* col_out,
                    hipStream_t st) {
  const int lgB = lg_tile(B);
  if (lgB < 0 || C < 1 || C > 16384 || K < 1 || K > C) return -2;
  if (R == 0) return 0;
  const size_t lds = (size_t)C * 4 + 64;
  int lgT = 0;                                       // lanes per block: 1024 / C, at most 64
  while (lgT < 6 && ((int64_t)C << (lgT + 1)) <= 1024) ++lgT;
  if (elem_bytes == 2) {
    auto kern = fmt_topk_kernel<uint16_t>;
    if (lds > 65536 && hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess)
      return -1;
    hipLaunchKernelGGL(kern, dim3((unsigned)R), dim3(1024), lds, st, static_cast<const uint16_t*>(dense), ld, C, lgB,
                       K, lgT, col_out);
  } else {
    auto kern = fmt_topk_kernel<uint32_t>;
    if (lds > 65536 && hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess)
      return -1;
    hipLaunchKernelGGL(kern, dim3((unsigned)R), dim3(1024), lds, st, static_cast<const uint32_t*>(dense), ld, C, lgB,
                       K, lgT, col_out);
  }
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_fmt_ternary_check(const uint32_t* words, int64_t n, int32_t* bad, hipStream_t st) {
  hipLaunchKernelGGL(fmt_ternary_check_kernel, dim3(1), dim3(1024), 0, st, words, n, bad);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace lbk
