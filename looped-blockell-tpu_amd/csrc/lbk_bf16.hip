// lbk_bf16.hip — bf16 Block-ELL kernels for gfx950 (MFMA 16x16x32 bf16, fp32 accumulate).
//
// Two families:
//
//  * rowblock_kernel<B, MODE>: one workgroup = 64 tokens x one block row r.
//    Each of the 4 waves owns 16 tokens; A fragments come straight from global
//    memory (16-byte loads of the gathered column block), weight fragments from
//    transposing loads.  Works for any geometry (B in {16,32,64}, any K, dead
//    slots, ragged N).  MODE selects the epilogue: plain product (+bias),
//    gate/up with SiLU*mul (+ optional pre-activation outputs), or down
//    projection (+ residual).
//
//  * panel_kernel<B, RPW, NORM>: one workgroup owns a 64-token tile for the whole
//    FFN.  The tile's input row panel [64, d_model] sits in LDS and is reused by
//    every gate/up block row; each round the 4 waves produce 4 d_ff blocks of h
//    into LDS, and every wave folds them into its RPW down-projection block rows
//    whose fp32 accumulators live in registers (the column->(row, slot) map of
//    the down weight is built once per workgroup in LDS).  h never leaves the
//    CU.  With NORM the workgroup loops L times over
//    h <- h + SwiGLU(RMSNorm(h)): the carried state stays in the fp32 down
//    accumulators, RMSNorm is computed from them and written back into the LDS
//    panel, so between iterations nothing goes to HBM except weight reads.
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
    const float* __restrict__ bias, const uint16_t* __restrict__ resid, int64_t ldr,
    uint16_t* __restrict__ y, int64_t ldy, uint16_t* __restrict__ aux0, uint16_t* __restrict__ aux1,
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
        gv[m] = acc[0][m][v];
        uv[m] = acc[1][m][v];
        o[m] = silu_f(gv[m]) * uv[m];
      }
      if (aux0) store_bf16<CW>(aux0 + t * ldaux + ocol, gv);
      if (aux1) store_bf16<CW>(aux1 + t * ldaux + ocol, uv);
    } else {
#pragma unroll
      for (int m = 0; m < CW; ++m) o[m] = acc[0][m][v];
      if constexpr (MODE == MODE_LINEAR) {
        if (bias) {
#pragma unroll
          for (int m = 0; m < CW; ++m) o[m] += bias[ocol + m];
        }
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
// panel kernel
// ---------------------------------------------------------------------------
constexpr int PANEL_TOK = 64;  // tokens per workgroup (4 M-tiles of 16)
constexpr int PANEL_MT = 4;



__host__ __device__ constexpr int panel_xstride(int d_model) { return d_model + 8; }
template <int B>
__host__ __device__ constexpr int panel_hstride() { return B + 8; }

// LDS bytes for one workgroup of panel_kernel.
size_t panel_lds_bytes(int B, int d_model, int R_ff, int R_m) {
  size_t x = (size_t)PANEL_TOK * panel_xstride(d_model) * 2;
  size_t h = (size_t)4 * PANEL_TOK * (B + 8) * 2;
  size_t csc = (((size_t)R_ff * R_m) + 15) & ~(size_t)15;
  size_t red = 4 * PANEL_TOK * 4;
  return x + h + csc + red;
}

template <int B, int RPW, bool NORM>
__global__ __launch_bounds__(256, 1) void panel_kernel(PanelArgs p) {
  constexpr int CW = TileShape<B>::CW;
  static_assert(TileShape<B>::NKS == 1, "panel kernel handles B <= 32");
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int d_model = p.d_model;
  const int xs = panel_xstride(d_model);
  constexpr int hs = panel_hstride<B>();
  uint16_t* xpanel = reinterpret_cast<uint16_t*>(smem);
  uint16_t* hslot = xpanel + PANEL_TOK * xs;
  int8_t* csc = reinterpret_cast<int8_t*>(hslot + 4 * PANEL_TOK * hs);
  float* red = reinterpret_cast<float*>(csc + ((((size_t)p.R_ff * p.R_m) + 15) & ~(size_t)15));

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = uniform(tid >> 6);
  const int i = lane & 15, g = lane >> 4;
  const int64_t t0 = (int64_t)blockIdx.x * PANEL_TOK;
  const int cin = d_model / B;

  // ---- column -> slot map of the down weight: csc[c * R_m + r_m] = k or -1
  const int ncsc = p.R_ff * p.R_m;
  for (int e = tid; e < ncsc; e += 256) csc[e] = -1;
  __syncthreads();
  for (int e = tid; e < p.R_m * p.Kd; e += 256) {
    const int rm = e / p.Kd, k = e - rm * p.Kd;
    const int c = p.cd[e];
    if (c >= 0 && c < p.R_ff) csc[c * p.R_m + rm] = (int8_t)k;
  }

  // ---- down accumulators: acc[rho][mt][m] for block rows r_m = w*RPW + rho
  f32x4 acc[RPW][PANEL_MT][CW];
#pragma unroll
  for (int rho = 0; rho < RPW; ++rho)
#pragma unroll
    for (int mt = 0; mt < PANEL_MT; ++mt)
#pragma unroll
      for (int m = 0; m < CW; ++m) acc[rho][mt][m] = f32x4{0.f, 0.f, 0.f, 0.f};

  if (NORM || p.add_residual) {
#pragma unroll
    for (int rho = 0; rho < RPW; ++rho) {
      const int rm = w * RPW + rho;
      if (rm >= p.R_m) continue;
#pragma unroll
      for (int mt = 0; mt < PANEL_MT; ++mt)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int64_t t = t0 + 16 * mt + 4 * g + v;
          if (t >= p.N) continue;
          float xv[CW];
          load_bf16<CW>(p.x + t * d_model + rm * B + CW * i, xv);
#pragma unroll
          for (int m = 0; m < CW; ++m) acc[rho][mt][m][v] = xv[m];
        }
    }
  }

  const int iters = NORM ? p.L : 1;
  for (int it = 0; it < iters; ++it) {
    // ---- fill the input panel
    if constexpr (!NORM) {
      const int c8 = d_model / 8;
      for (int e = tid; e < PANEL_TOK * c8; e += 256) {
        const int row = e / c8, cc = e - row * c8;
        const int64_t t = t0 + row;
        u32x4 v = {0, 0, 0, 0};
        if (t < p.N) v = *reinterpret_cast<const u32x4*>(p.x + t * d_model + 8 * cc);
        *reinterpret_cast<u32x4*>(xpanel + row * xs + 8 * cc) = v;
      }
    } else {
      // sum of squares per token over this lane's columns, reduced over the 16 lanes j
      float ss[PANEL_MT][4];
#pragma unroll
      for (int mt = 0; mt < PANEL_MT; ++mt)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          float s = 0.f;
#pragma unroll
          for (int rho = 0; rho < RPW; ++rho)
#pragma unroll
            for (int m = 0; m < CW; ++m) s += acc[rho][mt][m][v] * acc[rho][mt][m][v];
          s += __shfl_xor(s, 1, 16);
          s += __shfl_xor(s, 2, 16);
          s += __shfl_xor(s, 4, 16);
          s += __shfl_xor(s, 8, 16);
          ss[mt][v] = s;
        }
      if (i == 0) {
#pragma unroll
        for (int mt = 0; mt < PANEL_MT; ++mt)
#pragma unroll
          for (int v = 0; v < 4; ++v) red[w * PANEL_TOK + 16 * mt + 4 * g + v] = ss[mt][v];
      }
      __syncthreads();
      float rs[PANEL_MT][4];
#pragma unroll
      for (int mt = 0; mt < PANEL_MT; ++mt)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int row = 16 * mt + 4 * g + v;
          const float tot = red[row] + red[PANEL_TOK + row] + red[2 * PANEL_TOK + row] + red[3 * PANEL_TOK + row];
          rs[mt][v] = 1.0f / sqrtf(tot / (float)d_model + p.eps);
        }
#pragma unroll
      for (int rho = 0; rho < RPW; ++rho) {
        const int rm = w * RPW + rho;
        if (rm >= p.R_m) continue;
        float sc[CW];
#pragma unroll
        for (int m = 0; m < CW; ++m) sc[m] = p.norm_scale[rm * B + CW * i + m];
#pragma unroll
        for (int mt = 0; mt < PANEL_MT; ++mt)
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            float o[CW];
#pragma unroll
            for (int m = 0; m < CW; ++m) o[m] = acc[rho][mt][m][v] * rs[mt][v] * sc[m];
            store_bf16<CW>(xpanel + (16 * mt + 4 * g + v) * xs + rm * B + CW * i, o);
          }
      }
    }
    __syncthreads();

    // ---- rounds of 4 d_ff block rows
    const int nrounds = (p.R_ff + 3) / 4;
    for (int q = 0; q < nrounds; ++q) {
      const int r = 4 * q + w;
      if (r < p.R_ff) {
        f32x4 ag[PANEL_MT][CW], au[PANEL_MT][CW];
#pragma unroll
        for (int mt = 0; mt < PANEL_MT; ++mt)
#pragma unroll
          for (int m = 0; m < CW; ++m) {
            ag[mt][m] = f32x4{0.f, 0.f, 0.f, 0.f};
            au[mt][m] = f32x4{0.f, 0.f, 0.f, 0.f};
          }
        const int kmax = p.Kg > p.Ku ? p.Kg : p.Ku;
        for (int k = 0; k < kmax; ++k) {
          int colg = (k < p.Kg) ? uniform(p.cg[(int64_t)r * p.Kg + k]) : -1;
          int colu = (k < p.Ku) ? uniform(p.cu[(int64_t)r * p.Ku + k]) : -1;
          if (colg >= cin) colg = -1;  // out-of-range index: contributes nothing
          if (colu >= cin) colu = -1;
          WRaw<B> rg, ru;
          if (colg >= 0) load_wraw<B>(p.vg + ((int64_t)r * p.Kg + k) * B * B, lane, rg);
          if (colu >= 0) load_wraw<B>(p.vu + ((int64_t)r * p.Ku + k) * B * B, lane, ru);
          if (colg >= 0) {
            u32x4 f[1][CW];
            wraw_to_frag<B>(rg, f);
#pragma unroll
            for (int mt = 0; mt < PANEL_MT; ++mt) {
              const u32x4 a = load_afrag<B>(xpanel + (16 * mt + i) * xs + colg * B, 0, g);
#pragma unroll
              for (int m = 0; m < CW; ++m) ag[mt][m] = mfma_bf16(a, f[0][m], ag[mt][m]);
            }
          }
          if (colu >= 0) {
            u32x4 f[1][CW];
            wraw_to_frag<B>(ru, f);
#pragma unroll
            for (int mt = 0; mt < PANEL_MT; ++mt) {
              const u32x4 a = load_afrag<B>(xpanel + (16 * mt + i) * xs + colu * B, 0, g);
#pragma unroll
              for (int m = 0; m < CW; ++m) au[mt][m] = mfma_bf16(a, f[0][m], au[mt][m]);
            }
          }
        }
        // h = silu(g) * u -> LDS slot w (bf16)
        uint16_t* hw = hslot + w * PANEL_TOK * hs;
#pragma unroll
        for (int mt = 0; mt < PANEL_MT; ++mt)
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            float o[CW];
#pragma unroll
            for (int m = 0; m < CW; ++m) o[m] = silu_f(ag[mt][m][v]) * au[mt][m][v];
            store_bf16<CW>(hw + (16 * mt + 4 * g + v) * hs + CW * i, o);
          }
      }
      __syncthreads();
      // ---- fold the 4 fresh h blocks into this wave's down rows
#pragma unroll 1
      for (int s = 0; s < 4; ++s) {
        const int c = 4 * q + s;
        if (c >= p.R_ff) break;
        const uint16_t* hsrc = hslot + s * PANEL_TOK * hs;
#pragma unroll
        for (int rho = 0; rho < RPW; ++rho) {
          const int rm = w * RPW + rho;
          if (rm >= p.R_m) continue;
          const int k = uniform(csc[c * p.R_m + rm]);
          if (k < 0) continue;
          WRaw<B> rd;
          load_wraw<B>(p.vd + ((int64_t)rm * p.Kd + k) * B * B, lane, rd);
          u32x4 f[1][CW];
          wraw_to_frag<B>(rd, f);
#pragma unroll
          for (int mt = 0; mt < PANEL_MT; ++mt) {
            const u32x4 a = load_afrag<B>(hsrc + (16 * mt + i) * hs, 0, g);
#pragma unroll
            for (int m = 0; m < CW; ++m) acc[rho][mt][m] = mfma_bf16(a, f[0][m], acc[rho][mt][m]);
          }
        }
      }
      __syncthreads();
    }
  }

  // ---- epilogue: out = acc (already holds the residual / carried state)
#pragma unroll
  for (int rho = 0; rho < RPW; ++rho) {
    const int rm = w * RPW + rho;
    if (rm >= p.R_m) continue;
#pragma unroll
    for (int mt = 0; mt < PANEL_MT; ++mt)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int64_t t = t0 + 16 * mt + 4 * g + v;
        if (t >= p.N) continue;
        float o[CW];
#pragma unroll
        for (int m = 0; m < CW; ++m) o[m] = acc[rho][mt][m][v];
        store_bf16<CW>(p.out + t * d_model + rm * B + CW * i, o);
      }
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

__global__ __launch_bounds__(256) void injection_kernel(const uint16_t* __restrict__ h, const uint16_t* __restrict__ e,
                                                        const float* __restrict__ log_A, const float* __restrict__ log_dt,
                                                        int64_t total, int d, uint16_t* __restrict__ out) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= total) return;
  const int c = (int)(idx % d);
  const float ld = log_dt[c];
  // softplus(x) = log1p(exp(x)), evaluated stably for large x
  const float dt = ld > 20.f ? ld : log1pf(expf(ld));
  const float decay = expf(-dt * expf(log_A[c]));
  out[idx] = f2bf(decay * bf2f(h[idx]) + dt * bf2f(e[idx]));
}

// ---------------------------------------------------------------------------
// host launchers
// ---------------------------------------------------------------------------
template <int B, int MODE>
static int launch_rowblock_t(const RowblockLaunch& a, hipStream_t st) {
  dim3 grid((unsigned)((a.N + 63) / 64), (unsigned)a.R);
  hipLaunchKernelGGL((rowblock_kernel<B, MODE>), grid, dim3(256), 0, st, a.x, a.N, a.ldx, a.C, a.v0, a.c0, a.K0,
                     a.v1, a.c1, a.K1, a.bias, a.resid, a.ldr, a.y, a.ldy, a.aux0, a.aux1, a.ldaux);
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

int panel_rpw(int R_m) {
  for (int rpw : {1, 2, 4, 8})
    if (4 * rpw >= R_m) return rpw;
  return -1;
}

template <int B, int RPW, bool NORM>
static int launch_panel_t(const PanelArgs& p, size_t lds, hipStream_t st) {
  auto kern = panel_kernel<B, RPW, NORM>;
  static bool configured = false;  // attribute set once per process (idempotent)
  if (!configured) {
    if (hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, 163840) != hipSuccess)
      return -1;
    configured = true;
  }
  dim3 grid((unsigned)((p.N + PANEL_TOK - 1) / PANEL_TOK));
  hipLaunchKernelGGL(kern, grid, dim3(256), lds, st, p);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_panel(int B, bool norm, const PanelArgs& p, hipStream_t st) {
  if (p.N == 0) return 0;
  const int rpw = panel_rpw(p.R_m);
  const size_t lds = panel_lds_bytes(B, p.d_model, p.R_ff, p.R_m);
#define LBK_PN(BB, RR)                                                  \
  if (B == BB && rpw == RR) {                                           \
    return norm ? launch_panel_t<BB, RR, true>(p, lds, st)              \
                : launch_panel_t<BB, RR, false>(p, lds, st);            \
  }
  LBK_PN(16, 1) LBK_PN(16, 2) LBK_PN(16, 4) LBK_PN(16, 8)
  LBK_PN(32, 1) LBK_PN(32, 2) LBK_PN(32, 4) LBK_PN(32, 8)
#undef LBK_PN
  return -2;
}

bool panel_supported(int B, int d_model, int R_ff, int R_m, int Kd) {
  if (B != 16 && B != 32) return false;
  if (panel_rpw(R_m) < 0) return false;
  if (R_m * B != d_model) return false;
  if (Kd > 127) return false;
  if (d_model % 8) return false;
  return panel_lds_bytes(B, d_model, R_ff, R_m) <= 163840;
}

int launch_rmsnorm(const uint16_t* x, int64_t N, int d, const float* scale, float eps, uint16_t* out,
                   hipStream_t st) {
  if (N == 0) return 0;
  hipLaunchKernelGGL(rmsnorm_kernel, dim3((unsigned)((N + 3) / 4)), dim3(256), 0, st, x, N, d, scale, eps, out);
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

}  // namespace lbk
