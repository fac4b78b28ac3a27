// lbk_topo.hip — prune-time topology transforms of Block-ELL weights (gfx950).
//
// Integer and copy work only, all of it deterministic (no order-dependent sums):
//   topo_count_kernel     alive slots per row and their maximum (one workgroup)
//   topo_compact_kernel   per row: alive slots first, both groups in slot order (a
//                         ballot rank per 64-slot chunk), the first K_new slots copied;
//                         a workgroup per 8 source slots of a row
//   topo_importance_kernel  d_ff tile-column importance: integer counts in LDS
//   topo_perm_kernel      stable descending order of the importance by rank counting
//                         (up to 64 lanes per entry, partial ranks summed by shuffles)
//   topo_apply_kernel     a d_ff permutation: column indices remapped through the
//                         inverse permutation, or rows gathered
//   topo_kactive_kernel   macro-block columns that cover the largest alive column
//   topo_gather_kernel    rows of any tensor gathered through a permutation (byte copies,
//                         16 bytes per lane when rows and pointers allow)
//   topo_ccount_kernel    transposed (CSC) index: slots per column block in LDS, then the
//                         exclusive scan -> col_ptr (one workgroup)
//   topo_cfill_kernel     one workgroup per column block writes its slots r*K + k in
//                         ascending order (ballot compaction) at col_ptr[c]
#include "lbk_device.h"
#include "lbk_internal.h"

namespace lbk {

// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void topo_count_kernel(const uint8_t* __restrict__ alive, int R, int K,
                                                         int32_t* __restrict__ counts, int32_t* __restrict__ mx) {
  __shared__ int red[256];
  int m = 0;
  for (int r = threadIdx.x; r < R; r += 256) {
    int n = 0;
    for (int k = 0; k < K; ++k) n += alive[(int64_t)r * K + k] != 0;
    counts[r] = n;
    m = n > m ? n : m;
  }
  red[threadIdx.x] = m;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if ((int)threadIdx.x < s) red[threadIdx.x] = red[threadIdx.x] > red[threadIdx.x + s] ? red[threadIdx.x] : red[threadIdx.x + s];
    __syncthreads();
  }
  if (threadIdx.x == 0) mx[0] = red[0];
}

int launch_topo_count(const uint8_t* alive, int R, int K, int32_t* counts, int32_t* mx, hipStream_t st) {
  hipLaunchKernelGGL(topo_count_kernel, dim3(1), dim3(256), 0, st, alive, R, K, counts, mx);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

// ---------------------------------------------------------------------------
// A workgroup owns COMPACT_SLOTS source slots of one row.  Slot k's destination is (alive ?
// rank among alive : n_alive + rank among dead); wave 0 finds it by a ballot scan of the row's
// flags, then the whole workgroup copies the slots whose destination is below K_new.
constexpr int COMPACT_SLOTS = 8;

__global__ __launch_bounds__(256) void topo_compact_kernel(const uint16_t* __restrict__ values,
                                                           const int32_t* __restrict__ col,
                                                           const uint8_t* __restrict__ alive, int R, int K, int B,
                                                           int K_new, uint16_t* __restrict__ ov,
                                                           int32_t* __restrict__ oc, uint8_t* __restrict__ oa) {
  __shared__ int dst_s[COMPACT_SLOTS];
  const int r = (int)blockIdx.x, k0 = (int)blockIdx.y * COMPACT_SLOTS;
  const int tid = threadIdx.x, lane = tid & 63;
  const uint8_t* arow = alive + (int64_t)r * K;
  if (tid < 64) {
    int nalive = 0;
    for (int c0 = 0; c0 < K; c0 += 64)
      nalive += __builtin_popcountll(__ballot(c0 + lane < K && arow[c0 + lane] != 0));
    const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    int seen_a = 0, seen_d = 0;
    for (int c0 = 0; c0 < K && c0 < k0 + COMPACT_SLOTS; c0 += 64) {
      const int k = c0 + lane;
      const bool in = k < K;
      const bool al = in && arow[k] != 0;
      const uint64_t ma = __ballot(al), md = __ballot(in && !al);
      const int dest = al ? seen_a + __builtin_popcountll(ma & below)
                          : nalive + seen_d + __builtin_popcountll(md & below);
      if (in && k >= k0 && k < k0 + COMPACT_SLOTS) dst_s[k - k0] = dest;
      seen_a += __builtin_popcountll(ma);
      seen_d += __builtin_popcountll(md);
    }
  }
  __syncthreads();
  const int ns = (K - k0) < COMPACT_SLOTS ? (K - k0) : COMPACT_SLOTS;
  if (tid < ns) {
    const int d = dst_s[tid];
    if (d < K_new) {
      oc[(int64_t)r * K_new + d] = col[(int64_t)r * K + k0 + tid];
      oa[(int64_t)r * K_new + d] = arow[k0 + tid] != 0 ? 1 : 0;
    }
  }
  // tiles: ns tiles of per 16-byte chunks (per is a power of two) spread over the workgroup
  const int per = B * B / 8;
  const int lg = __builtin_ctz((unsigned)per);
  const u32x4* src = reinterpret_cast<const u32x4*>(values) + ((int64_t)r * K + k0) * per;
  u32x4* dst = reinterpret_cast<u32x4*>(ov) + (int64_t)r * K_new * per;
  for (int q = tid; q < ns * per; q += 256) {
    const int j = q >> lg, e = q & (per - 1);
    const int d = dst_s[j];
    if (d < K_new) dst[(int64_t)d * per + e] = src[(int64_t)j * per + e];
  }
}

int launch_topo_compact(const uint16_t* values, const int32_t* col, const uint8_t* alive, int R, int K, int B,
                        int K_new, uint16_t* ov, int32_t* oc, uint8_t* oa, hipStream_t st) {
  if (R == 0) return 0;
  const int gy = (K + COMPACT_SLOTS - 1) / COMPACT_SLOTS;
  if (gy > 65535) return -2;
  hipLaunchKernelGGL(topo_compact_kernel, dim3((unsigned)R, (unsigned)gy), dim3(256), 0, st, values, col, alive, R,
                     K, B, K_new, ov, oc, oa);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

// ---------------------------------------------------------------------------
// importance[c] = alive fc1 slots with column c (negative columns skipped, columns >= C_ff
// counted at C_ff - 1) + alive slots of fc2 row c (rows beyond C_ff ignored)
__global__ __launch_bounds__(1024) void topo_importance_kernel(const int32_t* __restrict__ c1,
                                                               const uint8_t* __restrict__ a1, int64_t n1,
                                                               const uint8_t* __restrict__ a2, int R2, int K2,
                                                               int C_ff, float* __restrict__ imp) {
  extern __shared__ int cnt[];
  for (int c = threadIdx.x; c < C_ff; c += 1024) cnt[c] = 0;
  __syncthreads();
  for (int64_t e = threadIdx.x; e < n1; e += 1024) {
    const int c = c1[e];
    if (c >= 0 && a1[e]) atomicAdd(&cnt[c < C_ff ? c : C_ff - 1], 1);   // LDS atomic, integer
  }
  __syncthreads();
  const int rows = R2 < C_ff ? R2 : C_ff;
  for (int c = threadIdx.x; c < C_ff; c += 1024) {
    int n = cnt[c];
    if (c < rows)
      for (int k = 0; k < K2; ++k) n += a2[(int64_t)c * K2 + k] != 0;
    imp[c] = (float)n;
  }
}

int launch_topo_importance(const int32_t* c1, const uint8_t* a1, int64_t n1, const uint8_t* a2, int R2, int K2,
                           int C_ff, float* imp, hipStream_t st) {
  if (C_ff <= 0 || C_ff > 16384) return -2;
  hipLaunchKernelGGL(topo_importance_kernel, dim3(1), dim3(1024), (size_t)C_ff * 4, st, c1, a1, n1, a2, R2, K2,
                     C_ff, imp);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

// ---------------------------------------------------------------------------
// perm = stable argsort of -importance: c goes to position #{c' before c}, where c' is before c
// if its importance is larger, or equal with a smaller index; NaN importances go last in
// index order (numpy's order for argsort(-importance))
__device__ __forceinline__ bool topo_before(float a, int ia, float b, int ib) {
  const bool na = a != a, nb = b != b;
  if (na || nb) return !na && nb ? true : (na && nb ? ia < ib : false);
  return a > b || (a == b && ia < ib);
}

// T lanes (a power of two <= 64, within one wave) share one c: lane j compares it with
// d = j, j + T, ... and the partial ranks are summed by shuffles.  The importance is read from
// global memory; all c-groups of a wave read the same d, so each load is a broadcast.
__global__ __launch_bounds__(256) void topo_perm_kernel(const float* __restrict__ imp, int C, int lgT,
                                                        int32_t* __restrict__ perm) {
  const int T = 1 << lgT;
  const int tid = threadIdx.x, j = tid & (T - 1);
  const int c = (int)blockIdx.x * (256 >> lgT) + (tid >> lgT);
  const bool ok = c < C;
  const float x = ok ? imp[c] : 0.f;
  int rank = 0;
  if (ok)
    for (int d = j; d < C; d += T) rank += topo_before(imp[d], d, x, c);
  for (int o = T >> 1; o > 0; o >>= 1) rank += __shfl_xor(rank, o, 64);
  if (ok && j == 0) perm[rank] = c;
}

int launch_topo_perm(const float* imp, int C, int32_t* perm, hipStream_t st) {
  if (C <= 0 || C > 16384) return -2;
  // about 64K threads in all, at most 64 per c
  int lgT = 0;
  while (lgT < 6 && ((int64_t)C << lgT) < 65536) ++lgT;
  const int per_block = 256 >> lgT;
  hipLaunchKernelGGL(topo_perm_kernel, dim3((unsigned)((C + per_block - 1) / per_block)), dim3(256), 0, st, imp, C,
                     lgT, perm);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

// ---------------------------------------------------------------------------
// column mode: out_col = col < 0 ? -1 : inv[min(col, C_ff - 1)], values and flags copied;
// row mode (R == C_ff): output row i = input row perm[i].  Permutation entries outside
// [0, C_ff) are clamped into it (a permutation never has them).
__global__ __launch_bounds__(256) void topo_apply_kernel(const uint16_t* __restrict__ values,
                                                         const int32_t* __restrict__ col,
                                                         const uint8_t* __restrict__ alive, int R, int K, int B,
                                                         const int32_t* __restrict__ perm, int C_ff, int column,
                                                         uint16_t* __restrict__ ov, int32_t* __restrict__ oc,
                                                         uint8_t* __restrict__ oa) {
  extern __shared__ int inv[];
  const int r = (int)blockIdx.x;
  const int64_t tb = (int64_t)B * B;
  if (column) {
    for (int c = threadIdx.x; c < C_ff; c += 256) inv[c] = 0;
    __syncthreads();
    for (int i = threadIdx.x; i < C_ff; i += 256) {
      int p = perm[i];
      p = p < 0 ? 0 : (p >= C_ff ? C_ff - 1 : p);
      inv[p] = i;
    }
    __syncthreads();
  }
  int src = r;
  if (!column) {
    const int p = perm[r];
    src = p < 0 ? 0 : (p >= R ? R - 1 : p);
  }
  for (int k = threadIdx.x; k < K; k += 256) {
    const int c = col[(int64_t)src * K + k];
    oc[(int64_t)r * K + k] = column ? (c < 0 ? -1 : inv[c < C_ff ? c : C_ff - 1]) : c;
    if (oa) oa[(int64_t)r * K + k] = alive[(int64_t)src * K + k];
  }
  if (!ov) return;   // column mode may leave the tiles where they are
  const u32x4* s = reinterpret_cast<const u32x4*>(values + (int64_t)src * K * tb);
  u32x4* d = reinterpret_cast<u32x4*>(ov + (int64_t)r * K * tb);
  for (int64_t q = threadIdx.x; q < K * tb / 8; q += 256) d[q] = s[q];
}

int launch_topo_apply(const uint16_t* values, const int32_t* col, const uint8_t* alive, int R, int K, int B,
                      const int32_t* perm, int C_ff, int column, uint16_t* ov, int32_t* oc, uint8_t* oa,
                      hipStream_t st) {
  if (R == 0) return 0;
  if (C_ff <= 0 || C_ff > 16384) return -2;
  hipLaunchKernelGGL(topo_apply_kernel, dim3((unsigned)R), dim3(256), column ? (size_t)C_ff * 4 : 0, st, values, col,
                     alive, R, K, B, perm, C_ff, column, ov, oc, oa);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void topo_kactive_kernel(const int32_t* __restrict__ col,
                                                           const uint8_t* __restrict__ alive, int64_t n, int tpm,
                                                           int32_t* __restrict__ out) {
  __shared__ int red[256];
  int m = -1;
  for (int64_t e = threadIdx.x; e < n; e += 256)
    if (alive[e]) m = col[e] > m ? col[e] : m;
  red[threadIdx.x] = m;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if ((int)threadIdx.x < s) red[threadIdx.x] = red[threadIdx.x] > red[threadIdx.x + s] ? red[threadIdx.x] : red[threadIdx.x + s];
    __syncthreads();
  }
  if (threadIdx.x == 0) out[0] = red[0] < 0 ? 0 : (red[0] + tpm) / tpm;   // ceil((max + 1) / tpm)
}

int launch_topo_kactive(const int32_t* col, const uint8_t* alive, int64_t n, int tpm, int32_t* out, hipStream_t st) {
  if (tpm <= 0) return -2;
  hipLaunchKernelGGL(topo_kactive_kernel, dim3(1), dim3(256), 0, st, col, alive, n, tpm, out);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

// ---------------------------------------------------------------------------
// dst row i = src row perm[i] (perm entries clamped into [0, n_src)), row_bytes each
__global__ __launch_bounds__(256) void topo_gather_kernel(const unsigned char* __restrict__ src, int64_t row_bytes,
                                                          const int32_t* __restrict__ perm, int n_src,
                                                          unsigned char* __restrict__ dst, int vec16) {
  const int i = (int)blockIdx.x;
  int p = perm[i];
  p = p < 0 ? 0 : (p >= n_src ? n_src - 1 : p);
  const unsigned char* s = src + (int64_t)p * row_bytes;
  unsigned char* d = dst + (int64_t)i * row_bytes;
  if (vec16) {
    const u32x4* s4 = reinterpret_cast<const u32x4*>(s);
    u32x4* d4 = reinterpret_cast<u32x4*>(d);
    for (int64_t q = threadIdx.x; q < row_bytes / 16; q += 256) d4[q] = s4[q];
  } else {
    for (int64_t q = threadIdx.x; q < row_bytes; q += 256) d[q] = s[q];
  }
}

int launch_topo_gather(const void* src, int64_t row_bytes, const int32_t* perm, int n_src, int n_dst, void* dst,
                       hipStream_t st) {
  if (n_dst == 0 || row_bytes == 0) return 0;
  const int vec16 = (row_bytes % 16 == 0 && (reinterpret_cast<uintptr_t>(src) % 16) == 0 &&
                     (reinterpret_cast<uintptr_t>(dst) % 16) == 0) ? 1 : 0;
  hipLaunchKernelGGL(topo_gather_kernel, dim3((unsigned)n_dst), dim3(256), 0, st,
                     static_cast<const unsigned char*>(src), row_bytes, perm, n_src,
                     static_cast<unsigned char*>(dst), vec16);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

// ---------------------------------------------------------------------------
// transposed index: col_ptr[c] .. col_ptr[c + 1] - 1 hold the slots e = r*K + k with
// col[e] == c in ascending e; slots with columns outside [0, C) are left out
__global__ __launch_bounds__(1024) void topo_ccount_kernel(const int32_t* __restrict__ col, int64_t n, int C,
                                                           int32_t* __restrict__ col_ptr) {
  extern __shared__ int hist[];   // C counts, then 16 wave totals
  int* wtot = hist + C;
  for (int c = threadIdx.x; c < C; c += 1024) hist[c] = 0;
  __syncthreads();
  for (int64_t e = threadIdx.x; e < n; e += 1024) {
    const int c = col[e];
    if (c >= 0 && c < C) atomicAdd(&hist[c], 1);   // LDS atomic, integer: order-free
  }
  __syncthreads();
  // exclusive scan over C in chunks of 1024: per-wave inclusive scan by shuffles
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  int carry = 0;
  for (int c0 = 0; c0 < C; c0 += 1024) {
    const int c = c0 + (int)threadIdx.x;
    const int v = c < C ? hist[c] : 0;
    int x = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int y = __shfl_up(x, o, 64);
      if (lane >= o) x += y;
    }
    if (lane == 63) wtot[w] = x;
    __syncthreads();
    int before = carry, all = 0;
#pragma unroll
    for (int ww = 0; ww < 16; ++ww) {
      if (ww < w) before += wtot[ww];
      all += wtot[ww];
    }
    if (c < C) col_ptr[c] = before + x - v;
    carry += all;
    __syncthreads();
  }
  if (threadIdx.x == 0) col_ptr[C] = carry;
}

__global__ __launch_bounds__(256) void topo_cfill_kernel(const int32_t* __restrict__ col, int n,
                                                         const int32_t* __restrict__ col_ptr,
                                                         int32_t* __restrict__ entries) {
  const int c = (int)blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  __shared__ int wsum[4];
  int base = col_ptr[c];
  for (int e0 = 0; e0 < n; e0 += 256) {
    const int e = e0 + tid;
    const bool hit = e < n && col[e] == c;
    const uint64_t m = __ballot(hit);
    const int rank = __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0));
    if (lane == 0) wsum[w] = __builtin_popcountll(m);
    __syncthreads();
    int off = base, tot = 0;
#pragma unroll
    for (int ww = 0; ww < 4; ++ww) {
      if (ww < w) off += wsum[ww];
      tot += wsum[ww];
    }
    if (hit) entries[off + rank] = e;
    base += tot;
    __syncthreads();
  }
}

int launch_topo_csc(const int32_t* col, int R, int K, int C, int32_t* col_ptr, int32_t* entries, hipStream_t st) {
  if (C <= 0 || C > 16384) return -2;
  const int64_t n = (int64_t)R * K;
  const size_t lds = ((size_t)C + 16) * 4;
  if (lds > 65536 && hipFuncSetAttribute(reinterpret_cast<const void*>(topo_ccount_kernel),
                                         hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess)
    return -1;
  hipLaunchKernelGGL(topo_ccount_kernel, dim3(1), dim3(1024), lds, st, col, n, C, col_ptr);
  if (hipGetLastError() != hipSuccess) return -1;
  if (n == 0) return 0;
  hipLaunchKernelGGL(topo_cfill_kernel, dim3((unsigned)C), dim3(256), 0, st, col, (int)n, col_ptr, entries);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace lbk
