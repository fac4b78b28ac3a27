// lbk_bf16.hip — bf16 Block-ELL kernels for gfx950 (MFMA 16x16x32 bf16, fp32 accumulate).
//
// The general-purpose family lives here (the fused single-launch FFN is in
// lbk_panel.hip):
//
//  * rowblock_kernel<B, MODE>: one workgroup = 64 tokens x one block row r.
//    Each of the 4 waves owns 16 tokens; A fragments come straight from global
//    memory (16-byte loads of the gathered column block), weight fragments from
//    transposing loads.  Works for any geometry (B in {16,32,64}, any K, dead
//    slots, ragged N).  MODE selects the epilogue: plain product (+bias),
//    gate/up with SiLU*mul (+ biases, + optional pre-activation outputs), or down
//    projection (+ bias, + residual).
//
#include "lbk_device.h"
#include "lbk_internal.h"

namespace lbk {

constexpr int MODE_LINEAR = 0;
constexpr int MODE_GATEUP = 1;
constexpr int MODE_DOWN = 2;

// ---------------------------------------------------------------------------
// rowblock kernel
// ---------------------------------------------------------------------------
template <int B, int MODE>
__global__ __launch_bounds__(256) void rowblock_kernel(
    const uint16_t* __restrict__ x, int64_t N, int64_t ldx, int C,
    const uint16_t* __restrict__ v0, const int32_t* __restrict__ c0, int K0,
    const uint16_t* __restrict__ v1, const int32_t* __restrict__ c1, int K1,
    // resid and y may be the same buffer (the general looped path updates its state in place;
    // each element is read before the thread that reads it writes it), so neither is restrict
    const float* __restrict__ bias, const float* __restrict__ bias1, const uint16_t* resid, int64_t ldr,
    uint16_t* y, int64_t ldy, uint16_t* __restrict__ aux0, uint16_t* __restrict__ aux1,
    int64_t ldaux) {
  constexpr int NKS = TileShape<B>::NKS, CW = TileShape<B>::CW;
  constexpr int NL = (MODE == MODE_GATEUP) ? 2 : 1;
  const int lane = threadIdx.x & 63;
  const int w = uniform(threadIdx.x >> 6);
  const int r = blockIdx.y;
  const int64_t t0 = (int64_t)blockIdx.x * 64 + 16 * w;
  const int i = lane & 15, g = lane >> 4;
  const int64_t my_tok = t0 + i;
  const bool tok_ok = my_tok < N;
  const uint16_t* xrow = x + (tok_ok ? my_tok : 0) * ldx;

  f32x4 acc[NL][CW];
#pragma unroll
  for (int l = 0; l < NL; ++l)
#pragma unroll
    for (int m = 0; m < CW; ++m) acc[l][m] = f32x4{0.f, 0.f, 0.f, 0.f};

#pragma unroll
  for (int l = 0; l < NL; ++l) {
    const uint16_t* vals = (l == 0) ? v0 : v1;
    const int32_t* cols = (l == 0) ? c0 : c1;
    const int K = (l == 0) ? K0 : K1;
    for (int k = 0; k < K; ++k) {
      const int col = uniform(cols[(int64_t)r * K + k]);
      if (col < 0 || col >= C) continue;  // dead slot (or out-of-range index): contributes nothing
      WRaw<B> raw;
      load_wraw<B>(vals + ((int64_t)r * K + k) * B * B, lane, raw);
      u32x4 a[NKS];
#pragma unroll
      for (int s = 0; s < NKS; ++s)
        a[s] = tok_ok ? load_afrag<B>(xrow + (int64_t)col * B, s, g) : u32x4{0, 0, 0, 0};
      u32x4 f[NKS][CW];
      wraw_to_frag<B>(raw, f);
#pragma unroll
      for (int s = 0; s < NKS; ++s)
#pragma unroll
        for (int m = 0; m < CW; ++m) acc[l][m] = mfma_bf16(a[s], f[s][m], acc[l][m]);
    }
  }

  // Epilogue: lane (j = i, g) owns rows 4g+v, output columns CW*j .. CW*j+CW-1.
  const int j = i;
  const int64_t ocol = (int64_t)r * B + CW * j;
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int64_t t = t0 + 4 * g + v;
    if (t >= N) continue;
    float o[CW];
    if constexpr (MODE == MODE_GATEUP) {
      float gv[CW], uv[CW];
#pragma unroll
      for (int m = 0; m < CW; ++m) {
        gv[m] = acc[0][m][v] + (bias ? bias[ocol + m] : 0.f);
        uv[m] = acc[1][m][v] + (bias1 ? bias1[ocol + m] : 0.f);
        o[m] = silu_f(gv[m]) * uv[m];
      }
      if (aux0) store_bf16<CW>(aux0 + t * ldaux + ocol, gv);
      if (aux1) store_bf16<CW>(aux1 + t * ldaux + ocol, uv);
    } else {
#pragma unroll
      for (int m = 0; m < CW; ++m) o[m] = acc[0][m][v];
      if (bias) {
#pragma unroll
        for (int m = 0; m < CW; ++m) o[m] += bias[ocol + m];
      }
      if constexpr (MODE == MODE_DOWN) {
        if (resid) {
          float rv[CW];
          load_bf16<CW>(resid + t * ldr + ocol, rv);
#pragma unroll
          for (int m = 0; m < CW; ++m) o[m] += rv[m];
        }
      }
    }
    store_bf16<CW>(y + t * ldy + ocol, o);
  }
}

// ---------------------------------------------------------------------------
// RMSNorm and diagonal injection (elementwise / row kernels)
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void rmsnorm_kernel(const uint16_t* __restrict__ x, int64_t N, int d,
                                                      const float* __restrict__ scale, float eps,
                                                      uint16_t* __restrict__ out) {
  // one wave per row
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= N) return;
  const uint16_t* xr = x + row * d;
  float s = 0.f;
  for (int c = lane; c < d; c += 64) {
    const float v = bf2f(xr[c]);
    s += v * v;
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) s += __shfl_xor(s, o, 64);
  const float rs = 1.0f / sqrtf(s / (float)d + eps);
  uint16_t* orow = out + row * d;
  for (int c = lane; c < d; c += 64) orow[c] = f2bf(bf2f(xr[c]) * rs * scale[c]);
}

// RMSNorm of fp32 rows into bf16 (the looped block's normalisation on the decode kernels' path):
// one wave per row; lane l holds columns 8 l + 512 j .. + 7 and sums their squares in the order
// of the gate/up kernel's normalising panel fill, so both produce the same bf16 rows.
// d % 8 == 0; x, scale and out 16-byte aligned.
__global__ __launch_bounds__(256) void rmsnorm_f32_kernel(const float* __restrict__ x, int64_t N, int d,
                                                          const float* __restrict__ scale, float eps,
                                                          uint16_t* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= N) return;
  const float* xr = x + row * d;
  float ss = 0.f;
  for (int col = 8 * lane; col < d; col += 512) {
    const f32x4 v0 = *reinterpret_cast<const f32x4*>(xr + col), v1 = *reinterpret_cast<const f32x4*>(xr + col + 4);
#pragma unroll
    for (int q = 0; q < 4; ++q) ss += v0[q] * v0[q];
#pragma unroll
    for (int q = 0; q < 4; ++q) ss += v1[q] * v1[q];
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o, 64);
  const float rs = 1.0f / sqrtf(ss / (float)d + eps);
  for (int col = 8 * lane; col < d; col += 512) {
    const f32x4 v0 = *reinterpret_cast<const f32x4*>(xr + col), v1 = *reinterpret_cast<const f32x4*>(xr + col + 4);
    const f32x4 s0 = *reinterpret_cast<const f32x4*>(scale + col), s1 = *reinterpret_cast<const f32x4*>(scale + col + 4);
    *reinterpret_cast<u32x4*>(out + row * d + col) =
        u32x4{pack2_bf16(v0[0] * rs * s0[0], v0[1] * rs * s0[1]), pack2_bf16(v0[2] * rs * s0[2], v0[3] * rs * s0[3]),
              pack2_bf16(v1[0] * rs * s1[0], v1[1] * rs * s1[1]), pack2_bf16(v1[2] * rs * s1[2], v1[3] * rs * s1[3])};
  }
}

// Backward of out = x * rs * scale, rs = 1 / sqrt(mean(x^2) + eps), per row of length d:
//   dx     = rs * scale * dy - x * rs^3 * mean(scale * dy * x)
//   dscale = sum over rows of dy * x * rs
// A workgroup owns RMS_BWD_ROWS consecutive rows: its four waves first reduce each row's
// sum of squares and sum(scale * dy * x) (rows w, w + 4, ...), then every thread walks its
// columns c = tid, tid + 256, ... over the rows, writing dx and keeping its dscale partial,
// stored per workgroup ([gridDim, d] fp32) and summed over the workgroups in a fixed order by
// rmsnorm_dscale_kernel: deterministic.
constexpr int RMS_BWD_ROWS = 64;

__global__ __launch_bounds__(256) void rmsnorm_bwd_kernel(const uint16_t* __restrict__ x,
                                                          const uint16_t* __restrict__ dy, int64_t N, int d,
                                                          const float* __restrict__ scale, float eps,
                                                          uint16_t* __restrict__ dx, float* __restrict__ part) {
  __shared__ float s_rs[RMS_BWD_ROWS], s_coef[RMS_BWD_ROWS];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int64_t r0 = (int64_t)blockIdx.x * RMS_BWD_ROWS;
  const int nrows = (int)(N - r0 < RMS_BWD_ROWS ? N - r0 : RMS_BWD_ROWS);
  for (int rr = w; rr < nrows; rr += 4) {
    const uint16_t* xr = x + (r0 + rr) * d;
    const uint16_t* gr = dy + (r0 + rr) * d;
    float ss = 0.f, dot = 0.f;
    for (int c = lane; c < d; c += 64) {
      const float xv = bf2f(xr[c]);
      ss += xv * xv;
      dot += scale[c] * bf2f(gr[c]) * xv;
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
      ss += __shfl_xor(ss, o, 64);
      dot += __shfl_xor(dot, o, 64);
    }
    if (lane == 0) {
      const float rs = 1.0f / sqrtf(ss / (float)d + eps);
      s_rs[rr] = rs;
      s_coef[rr] = rs * rs * rs * (dot / (float)d);
    }
  }
  __syncthreads();
  for (int c = tid; c < d; c += 256) {
    const float sc = scale[c];
    float ds = 0.f;
    for (int rr = 0; rr < nrows; ++rr) {
      const int64_t off = (r0 + rr) * d + c;
      const float xv = bf2f(x[off]), gv = bf2f(dy[off]);
      const float rs = s_rs[rr];
      dx[off] = f2bf(rs * sc * gv - xv * s_coef[rr]);
      ds += gv * xv * rs;
    }
    part[(int64_t)blockIdx.x * d + c] = ds;
  }
}

__global__ __launch_bounds__(256) void rmsnorm_dscale_kernel(const float* __restrict__ part, int nblk, int d,
                                                             float* __restrict__ dscale) {
  const int c = blockIdx.x * 256 + threadIdx.x;
  if (c >= d) return;
  float s = 0.f;
  for (int b = 0; b < nblk; ++b) s += part[(int64_t)b * d + c];
  dscale[c] = s;
}

// Column sums of a bf16 matrix [N, C] (row stride lda) in fp32 (bias gradients): workgroup b
// sums rows [64 b, 64 b + 64) of its columns c = tid, tid + 256, ... into part[b, c], then
// rmsnorm_dscale_kernel sums the workgroups in order: deterministic.
__global__ __launch_bounds__(256) void colsum_part_kernel(const uint16_t* __restrict__ a, int64_t N, int C,
                                                          int64_t lda, float* __restrict__ part) {
  const int64_t r0 = (int64_t)blockIdx.x * RMS_BWD_ROWS;
  const int nrows = (int)(N - r0 < RMS_BWD_ROWS ? N - r0 : RMS_BWD_ROWS);
  for (int c = threadIdx.x; c < C; c += 256) {
    float s = 0.f;
    for (int rr = 0; rr < nrows; ++rr) s += bf2f(a[(r0 + rr) * lda + c]);
    part[(int64_t)blockIdx.x * C + c] = s;
  }
}

size_t colsum_bytes(int64_t N, int C) { return (size_t)((N + RMS_BWD_ROWS - 1) / RMS_BWD_ROWS) * (size_t)C * 4; }

int launch_colsum(const uint16_t* a, int64_t N, int C, int64_t lda, float* part, float* out, hipStream_t st) {
  const int64_t nblk = (N + RMS_BWD_ROWS - 1) / RMS_BWD_ROWS;
  if (nblk > 0x7fffffff || C <= 0) return -2;
  if (nblk > 0) {
    hipLaunchKernelGGL(colsum_part_kernel, dim3((unsigned)nblk), dim3(256), 0, st, a, N, C, lda, part);
    if (hipGetLastError() != hipSuccess) return -1;
  }
  hipLaunchKernelGGL(rmsnorm_dscale_kernel, dim3((unsigned)((C + 255) / 256)), dim3(256), 0, st, part, (int)nblk, C,
                     out);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

size_t rmsnorm_bwd_bytes(int64_t N, int d) {
  return (size_t)((N + RMS_BWD_ROWS - 1) / RMS_BWD_ROWS) * (size_t)d * 4;
}

int launch_rmsnorm_bwd(const uint16_t* x, const uint16_t* dy, int64_t N, int d, const float* scale, float eps,
                       uint16_t* dx, float* dscale, float* part, hipStream_t st) {
  const int64_t nblk = (N + RMS_BWD_ROWS - 1) / RMS_BWD_ROWS;
  if (nblk > 0x7fffffff) return -2;
  if (nblk > 0) {
    hipLaunchKernelGGL(rmsnorm_bwd_kernel, dim3((unsigned)nblk), dim3(256), 0, st, x, dy, N, d, scale, eps, dx, part);
    if (hipGetLastError() != hipSuccess) return -1;
  }
  hipLaunchKernelGGL(rmsnorm_dscale_kernel, dim3((unsigned)((d + 255) / 256)), dim3(256), 0, st, part, (int)nblk, d,
                     dscale);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

// out may alias h (lbk_diagonal_injection_bf16 allows it): neither is restrict
__global__ __launch_bounds__(256) void injection_kernel(const uint16_t* h, const uint16_t* __restrict__ e,
                                                        const float* __restrict__ log_A, const float* __restrict__ log_dt,
                                                        int64_t total, int d, uint16_t* out) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= total) return;
  const int c = (int)(idx % d);
  const float ld = log_dt[c];
  // softplus(x) = log1p(exp(x)), evaluated stably for large x
  const float dt = ld > 20.f ? ld : log1pf(expf(ld));
  const float decay = expf(-dt * expf(log_A[c]));
  out[idx] = f2bf(decay * bf2f(h[idx]) + dt * bf2f(e[idx]));
}

// Backward of the injection, one workgroup per 64 rows: dh = decay * g, de = dt * g (either may
// be skipped), and per column the partial sums over the block's rows of g * h and g * e, which
// injection_param_grad_kernel adds in a fixed order into the parameter gradients.
__global__ __launch_bounds__(256) void injection_bwd_kernel(const uint16_t* __restrict__ g,
                                                            const uint16_t* __restrict__ h,
                                                            const uint16_t* __restrict__ e,
                                                            const float* __restrict__ log_A,
                                                            const float* __restrict__ log_dt, int64_t N, int d,
                                                            uint16_t* __restrict__ dh, uint16_t* __restrict__ de,
                                                            float* __restrict__ part) {
  const int64_t r0 = (int64_t)blockIdx.x * RMS_BWD_ROWS;
  const int nrows = (int)(N - r0 < RMS_BWD_ROWS ? N - r0 : RMS_BWD_ROWS);
  for (int c = threadIdx.x; c < d; c += 256) {
    const float ld = log_dt[c];
    const float dt = ld > 20.f ? ld : log1pf(expf(ld));
    const float decay = expf(-dt * expf(log_A[c]));
    float sgh = 0.f, sge = 0.f;
    for (int rr = 0; rr < nrows; ++rr) {
      const int64_t idx = (r0 + rr) * d + c;
      const float gv = bf2f(g[idx]);
      sgh += gv * bf2f(h[idx]);
      sge += gv * bf2f(e[idx]);
      if (dh) dh[idx] = f2bf(decay * gv);
      if (de) de[idx] = f2bf(dt * gv);
    }
    part[((int64_t)blockIdx.x * 2) * d + c] = sgh;
    part[((int64_t)blockIdx.x * 2 + 1) * d + c] = sge;
  }
}

// d log_A = -S_gh * decay * dt * A, d log_dt = (S_ge - S_gh * decay * A) * sigmoid(log_dt), with the
// column sums S over the nblk row blocks added in block order
__global__ __launch_bounds__(256) void injection_param_grad_kernel(const float* __restrict__ part, int nblk, int d,
                                                                   const float* __restrict__ log_A,
                                                                   const float* __restrict__ log_dt,
                                                                   float* __restrict__ d_log_A,
                                                                   float* __restrict__ d_log_dt) {
  const int c = blockIdx.x * 256 + threadIdx.x;
  if (c >= d) return;
  float sgh = 0.f, sge = 0.f;
  for (int b = 0; b < nblk; ++b) {
    sgh += part[((int64_t)b * 2) * d + c];
    sge += part[((int64_t)b * 2 + 1) * d + c];
  }
  const float ld = log_dt[c];
  const float dt = ld > 20.f ? ld : log1pf(expf(ld));
  const float A = expf(log_A[c]);
  const float decay = expf(-dt * A);
  const float sig = 1.0f / (1.0f + expf(-ld));
  if (d_log_A) d_log_A[c] = -sgh * decay * dt * A;
  if (d_log_dt) d_log_dt[c] = (sge - sgh * decay * A) * sig;
}

// ---------------------------------------------------------------------------
// host launchers
// ---------------------------------------------------------------------------
template <int B, int MODE>
static int launch_rowblock_t(const RowblockLaunch& a, hipStream_t st) {
  dim3 grid((unsigned)((a.N + 63) / 64), (unsigned)a.R);
  hipLaunchKernelGGL((rowblock_kernel<B, MODE>), grid, dim3(256), 0, st, a.x, a.N, a.ldx, a.C, a.v0, a.c0, a.K0,
                     a.v1, a.c1, a.K1, a.bias, a.bias1, a.resid, a.ldr, a.y, a.ldy, a.aux0, a.aux1, a.ldaux);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_rowblock(int B, int mode, const RowblockLaunch& a, hipStream_t st) {
  if (a.N == 0 || a.R == 0) return 0;
  if (a.R > 65535 || (a.N + 63) / 64 > 0x7fffffff) return -3;  // grid limits
#define LBK_RB(BB)                                                         \
  if (B == BB) {                                                           \
    if (mode == MODE_LINEAR) return launch_rowblock_t<BB, MODE_LINEAR>(a, st); \
    if (mode == MODE_GATEUP) return launch_rowblock_t<BB, MODE_GATEUP>(a, st); \
    if (mode == MODE_DOWN) return launch_rowblock_t<BB, MODE_DOWN>(a, st);     \
  }
  LBK_RB(16)
  LBK_RB(32)
  LBK_RB(64)
#undef LBK_RB
  return -2;
}

int launch_rmsnorm_f32(const float* x, int64_t N, int d, const float* scale, float eps, uint16_t* out,
                       hipStream_t st) {
  if (N == 0) return 0;
  if (d % 8) return -2;
  hipLaunchKernelGGL(rmsnorm_f32_kernel, dim3((unsigned)((N + 3) / 4)), dim3(256), 0, st, x, N, d, scale, eps, out);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_rmsnorm(const uint16_t* x, int64_t N, int d, const float* scale, float eps, uint16_t* out,
                   hipStream_t st) {
  if (N == 0) return 0;
  hipLaunchKernelGGL(rmsnorm_kernel, dim3((unsigned)((N + 3) / 4)), dim3(256), 0, st, x, N, d, scale, eps, out);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

size_t injection_bwd_bytes(int64_t N, int d) {
  return (size_t)((N + RMS_BWD_ROWS - 1) / RMS_BWD_ROWS) * 2 * (size_t)d * 4;
}

int launch_injection_bwd(const uint16_t* g, const uint16_t* h, const uint16_t* e, const float* log_A,
                         const float* log_dt, int64_t N, int d, uint16_t* dh, uint16_t* de, float* d_log_A,
                         float* d_log_dt, float* part, hipStream_t st) {
  const int64_t nblk = (N + RMS_BWD_ROWS - 1) / RMS_BWD_ROWS;
  if (nblk > 0x7fffffff || d <= 0) return -2;
  if (nblk > 0) {
    hipLaunchKernelGGL(injection_bwd_kernel, dim3((unsigned)nblk), dim3(256), 0, st, g, h, e, log_A, log_dt, N, d,
                       dh, de, part);
    if (hipGetLastError() != hipSuccess) return -1;
  }
  if (d_log_A || d_log_dt)
    hipLaunchKernelGGL(injection_param_grad_kernel, dim3((unsigned)((d + 255) / 256)), dim3(256), 0, st, part,
                       (int)nblk, d, log_A, log_dt, d_log_A, d_log_dt);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_injection(const uint16_t* h, const uint16_t* e, const float* log_A, const float* log_dt, int64_t N,
                     int d, uint16_t* out, hipStream_t st) {
  const int64_t total = N * d;
  if (total == 0) return 0;
  hipLaunchKernelGGL(injection_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, h, e, log_A,
                     log_dt, total, d, out);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

// ---------------------------------------------------------------------------
// bf16 tiles [R*K, B, B] ([B_in, B_out] each) -> fragment-major packed tiles
// (layout described with PackedTile in lbk_device.h), one thread per dword.
// Tiles of dead slots (col < 0 or col >= C) are written as zeros, and one
// extra zero tile follows the R*K tiles, so kernels can point padding and dead
// positions at zero weights instead of masking them.
// ---------------------------------------------------------------------------
template <int B>
__device__ __forceinline__ void pack_bf16_dword(const uint16_t* __restrict__ values, const int32_t* __restrict__ col,
                                                int64_t ntiles, int C, int64_t ndw, uint32_t* __restrict__ packed,
                                                int64_t idx, int gu_layout) {
  constexpr int CW = TileShape<B>::CW;
  constexpr int PER_TILE = PackedTile<B>::U32X4 * 4;   // dwords per packed tile
  if (idx >= ndw) return;
  const int64_t tile = idx / PER_TILE;
  if (tile >= ntiles || col[tile] < 0 || col[tile] >= C) {
    packed[idx] = 0u;
    return;
  }
  constexpr int LANES = PackedTile<B>::LANES;
  int r = (int)(idx - tile * PER_TILE);
  const int u = r & 3;
  r >>= 2;
  const int l = r % LANES;
  r /= LANES;
  const int m = r % CW;
  const int ks = r / CW;
  const int j = l & 15, g = l >> 4;
  const int k = 32 * ks + 8 * g + 2 * u;
  // gate/up layout (B = 32): column 8 (j / 4) + 4 m + j % 4, so that the product with the
  // tile as the A operand leaves 8 consecutive columns of one token in each lane
  const int c = (B == 32 && gu_layout) ? 8 * (j >> 2) + 4 * m + (j & 3) : CW * j + m;
  const uint16_t* w = values + tile * B * B;
  packed[idx] = (uint32_t)w[k * B + c] | ((uint32_t)w[(k + 1) * B + c] << 16);
}

template <int B>
__global__ __launch_bounds__(256) void pack_bf16_kernel(const uint16_t* __restrict__ values,
                                                        const int32_t* __restrict__ col, int64_t ntiles, int C,
                                                        int64_t ndw, uint32_t* __restrict__ packed) {
  pack_bf16_dword<B>(values, col, ntiles, C, ndw, packed, (int64_t)blockIdx.x * 256 + threadIdx.x, 0);
}

// several weights in one launch, one wave per tile (the R*K tiles of weight t and its zero
// tile are workgroups [first[t], first[t + 1])): the raw tile is read with 16-byte loads into
// LDS, then each lane gathers its fragment dwords from there and writes them as 16-byte chunks
// (chunk index (ks, m) is 64 consecutive u32x4 across the wave)
template <int B>
__global__ __launch_bounds__(64) void pack_bf16_multi_kernel(PackJobs jobs) {
  constexpr int CW = TileShape<B>::CW, NKS = TileShape<B>::NKS;
  constexpr int LANES = PackedTile<B>::LANES, U32X4 = PackedTile<B>::U32X4;
  constexpr int RAW = B * B / 8;                     // 16-byte chunks of a raw tile
  __shared__ __attribute__((aligned(16))) uint16_t s[B * B];
  int t = 0;
#pragma unroll
  for (int u = 1; u < PackJobs::kMax; ++u)
    if (u < jobs.n && (int64_t)blockIdx.x >= jobs.first[u]) t = u;
  const PackJob& J = jobs.job[t];
  const int64_t tile = (int64_t)blockIdx.x - jobs.first[t];
  const int lane = threadIdx.x;
  u32x4* out = reinterpret_cast<u32x4*>(J.packed) + tile * U32X4;
  const int c0 = tile < J.ntiles ? J.col[tile] : -1;
  if (c0 < 0 || c0 >= J.C) {                         // dead slot or the appended zero tile
    for (int q = lane; q < U32X4; q += 64) out[q] = u32x4{0, 0, 0, 0};
    return;
  }
  if ((reinterpret_cast<uintptr_t>(J.values) & 15u) == 0) {
    const u32x4* src = reinterpret_cast<const u32x4*>(J.values + tile * B * B);
    for (int q = lane; q < RAW; q += 64) reinterpret_cast<u32x4*>(s)[q] = src[q];
  } else {                                           // 8-byte aligned values (the ABI's minimum)
    const u32x2* src = reinterpret_cast<const u32x2*>(J.values + tile * B * B);
    for (int q = lane; q < 2 * RAW; q += 64) reinterpret_cast<u32x2*>(s)[q] = src[q];
  }
  __syncthreads();
  if (lane >= LANES) return;
  const int j = lane & 15, g = lane >> 4;
#pragma unroll
  for (int ks = 0; ks < NKS; ++ks)
#pragma unroll
    for (int m = 0; m < CW; ++m) {
      // gate/up layout (B = 32): column 8 (j / 4) + 4 m + j % 4, so that the product with the
      // tile as the A operand leaves 8 consecutive columns of one token in each lane
      const int c = (B == 32 && J.gu_layout) ? 8 * (j >> 2) + 4 * m + (j & 3) : CW * j + m;
      const int k0 = 32 * ks + 8 * g;
      u32x4 v;
#pragma unroll
      for (int u = 0; u < 4; ++u)
        v[u] = (uint32_t)s[(k0 + 2 * u) * B + c] | ((uint32_t)s[(k0 + 2 * u + 1) * B + c] << 16);
      out[(ks * CW + m) * LANES + lane] = v;
    }
}

size_t packed_bf16_bytes(int64_t ntiles, int B) {
  switch (B) {
    case 16: return (size_t)(ntiles + 1) * PackedTile<16>::U32X4 * 16;
    case 32: return (size_t)(ntiles + 1) * PackedTile<32>::U32X4 * 16;
    case 64: return (size_t)(ntiles + 1) * PackedTile<64>::U32X4 * 16;
    default: return 0;
  }
}

int launch_pack_bf16_multi(const PackJob* jobs, int n, int B, hipStream_t st) {
  if (n < 1 || n > PackJobs::kMax) return -2;
  PackJobs J{};
  J.n = n;
  int64_t blocks = 0;
  for (int t = 0; t < n; ++t) {
    J.job[t] = jobs[t];
    J.job[t].ndw = (int64_t)(packed_bf16_bytes(jobs[t].ntiles, B) / 4);
    J.first[t] = blocks;
    blocks += jobs[t].ntiles + 1;                    // one wave per tile, plus the zero tile
  }
  if (blocks == 0 || blocks > 0x7fffffff) return -2;
  const dim3 grid((unsigned)blocks);
  if (B == 16) hipLaunchKernelGGL(pack_bf16_multi_kernel<16>, grid, dim3(64), 0, st, J);
  else if (B == 32) hipLaunchKernelGGL(pack_bf16_multi_kernel<32>, grid, dim3(64), 0, st, J);
  else if (B == 64) hipLaunchKernelGGL(pack_bf16_multi_kernel<64>, grid, dim3(64), 0, st, J);
  else return -2;
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_pack_bf16(const uint16_t* values, const int32_t* col, int64_t ntiles, int C, int B, uint32_t* packed,
                     hipStream_t st) {
  const int64_t ndw = (int64_t)(packed_bf16_bytes(ntiles, B) / 4);
  if (ndw == 0) return -2;
  const unsigned grid = (unsigned)((ndw + 255) / 256);
  if (B == 16) hipLaunchKernelGGL(pack_bf16_kernel<16>, dim3(grid), dim3(256), 0, st, values, col, ntiles, C, ndw, packed);
  if (B == 32) hipLaunchKernelGGL(pack_bf16_kernel<32>, dim3(grid), dim3(256), 0, st, values, col, ntiles, C, ndw, packed);
  if (B == 64) hipLaunchKernelGGL(pack_bf16_kernel<64>, dim3(grid), dim3(256), 0, st, values, col, ntiles, C, ndw, packed);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

// ---------------------------------------------------------------------------
// looped core helpers: the injection's per-feature coefficients, per-token depths, the fp32 state
// set-up and the state update of core blocks run outside the split kernels (8 features per
// thread; d % 8 == 0 and 16-byte aligned rows)
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void core_prep_kernel(const float* __restrict__ log_A,
                                                        const float* __restrict__ log_dt, int d,
                                                        float* __restrict__ coef, const int32_t* __restrict__ depths,
                                                        int64_t seq_len, int64_t N, int32_t* __restrict__ tdepth) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (coef && i < d) {
    // the injection kernel's arithmetic: dt = softplus(log_dt), decay = exp(-dt * exp(log_A))
    const float ld = log_dt[i];
    const float dt = ld > 20.f ? ld : log1pf(expf(ld));
    coef[i] = expf(-dt * expf(log_A[i]));
    coef[d + i] = dt;
  }
  if (tdepth && i < N) tdepth[i] = depths[i / seq_len];
}

__global__ __launch_bounds__(256) void core_init_kernel(const uint16_t* __restrict__ h_in,
                                                        const uint16_t* __restrict__ e, const float* __restrict__ coef,
                                                        const int32_t* __restrict__ tdepth, int L, int64_t N, int d,
                                                        float* __restrict__ state) {
  const int64_t e0 = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 8;
  if (e0 >= N * d) return;
  const int64_t t = e0 / d;
  const int c = (int)(e0 - t * d);
  float s[8];
  unpack8_bf16(*reinterpret_cast<const u32x4*>(h_in + e0), s);
  if (e && L > 0 && (!tdepth || tdepth[t] > 0)) inject8(s, e, coef, e0, c, d);
  *reinterpret_cast<f32x4*>(state + e0) = f32x4{s[0], s[1], s[2], s[3]};
  *reinterpret_cast<f32x4*>(state + e0 + 4) = f32x4{s[4], s[5], s[6], s[7]};
}

__global__ __launch_bounds__(256) void core_update_kernel(float* __restrict__ state, const uint16_t* __restrict__ y,
                                                          const int32_t* __restrict__ tdepth, int it,
                                                          const uint16_t* __restrict__ e,
                                                          const float* __restrict__ coef, int64_t N, int d,
                                                          uint16_t* __restrict__ out) {
  const int64_t e0 = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 8;
  if (e0 >= N * d) return;
  const int64_t t = e0 / d;
  const int c = (int)(e0 - t * d);
  const f32x4 v0 = *reinterpret_cast<const f32x4*>(state + e0), v1 = *reinterpret_cast<const f32x4*>(state + e0 + 4);
  float s[8] = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
  const int dep = tdepth ? tdepth[t] : 0x7fffffff;
  if (it < dep) {
    float yf[8];
    unpack8_bf16(*reinterpret_cast<const u32x4*>(y + e0), yf);
#pragma unroll
    for (int q = 0; q < 8; ++q) s[q] += yf[q];
    if (e && it + 1 < dep) inject8(s, e, coef, e0, c, d);
    *reinterpret_cast<f32x4*>(state + e0) = f32x4{s[0], s[1], s[2], s[3]};
    *reinterpret_cast<f32x4*>(state + e0 + 4) = f32x4{s[4], s[5], s[6], s[7]};
  }
  if (out)
    *reinterpret_cast<u32x4*>(out + e0) = u32x4{pack2_bf16(s[0], s[1]), pack2_bf16(s[2], s[3]),
                                                pack2_bf16(s[4], s[5]), pack2_bf16(s[6], s[7])};
}

int launch_core_prep(const float* log_A, const float* log_dt, int d, float* coef, const int32_t* depths,
                     int64_t seq_len, int64_t N, int32_t* tdepth, hipStream_t st) {
  if (!coef && !tdepth) return 0;
  if (tdepth && seq_len < 1) return -2;
  const int64_t nc = coef ? (int64_t)d : 0, nt = tdepth ? N : 0;
  const int64_t n = nc > nt ? nc : nt;
  if (n <= 0) return 0;
  hipLaunchKernelGGL(core_prep_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, log_A, log_dt, d, coef,
                     depths, seq_len, N, tdepth);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_core_init(const uint16_t* h_in, const uint16_t* e, const float* coef, const int32_t* tdepth, int L,
                     int64_t N, int d, float* state, hipStream_t st) {
  if (N == 0) return 0;
  if (d % 8) return -2;
  const int64_t n8 = N * d / 8;
  hipLaunchKernelGGL(core_init_kernel, dim3((unsigned)((n8 + 255) / 256)), dim3(256), 0, st, h_in, e, coef, tdepth, L,
                     N, d, state);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_core_update(float* state, const uint16_t* y, const int32_t* tdepth, int it, const uint16_t* e,
                       const float* coef, int64_t N, int d, uint16_t* out, hipStream_t st) {
  if (N == 0) return 0;
  if (d % 8) return -2;
  const int64_t n8 = N * d / 8;
  hipLaunchKernelGGL(core_update_kernel, dim3((unsigned)((n8 + 255) / 256)), dim3(256), 0, st, state, y, tdepth, it,
                     e, coef, N, d, out);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace lbk
