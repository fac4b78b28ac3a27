// lbk_tsplit.hip — ternary SwiGLU FFN with int8 MFMA, B = 64 (gfx950).
//
// Arithmetic (the same as the row-block kernels of lbk_ternary.hip): for block
// row r the fp32 block scales are used in the fixed point m[r,k] * 2^-e[r]
// (row_fixed_point: m up to 16 bits, sum_k m * P inside int32), each block's
// int32 partial P comes from an int8 MFMA chain started at zero, and
// acc += m * P is one 24-bit integer multiply-add per element; the output is
// y = f32(f32(acc) * 2^-e[r]) * sx[token].
//
//   tprep_kernel  per call: packed tiles [R,K,64,4] -> fragment-major words
//                 (lane l of a wave reads its 4 words with one dwordx4), m per
//                 tile (zero for dead slots and for one appended zero tile),
//                 and 2^-e[r] per row.
//   tgu_kernel    gate/up + SiLU*mul: a workgroup owns 64 tokens (int8 x panel
//                 in LDS, XOR-swizzled) and one of H slices of the block rows;
//                 each wave streams rows r through a ring of (gate, up) tile
//                 pairs (same structure as the bf16 gu_kernel).  h goes out
//                 as bf16 with the per-token max |h| of this slice.
//   tdn_kernel    down + residual: a workgroup owns 16 tokens; it reads their h
//                 rows, quantises them per token (absmax over the H slices,
//                 128/absmax scale, round-half-even, clamp) straight into an int8
//                 LDS panel of the full d_ff width, then each wave streams its
//                 down rows through a ring of tiles.
#include "lbk_device.h"
#include "lbk_internal.h"
#include "lbk_tern_device.h"

namespace lbk {

namespace {

// ring depths (tile slots prefetched ahead): a gate/up slot is a (gate, up) tile pair, 32
// MFMAs; a down slot is one tile, 4 MFMAs
constexpr int TG_RING = 2;
constexpr int TD_RING = 8;

__device__ __forceinline__ u32x4 lds16t(const unsigned char* base, uint32_t off) {
  return *reinterpret_cast<const u32x4*>(base + off);
}

// panel layout (as in the bf16 kernels): token row 16*mt + i at row slot i*MT + mt,
// 16-byte chunk c at chunk c ^ i
template <int MT>
__device__ __forceinline__ uint32_t tpanel_addr(int row, int chunk, int rowb) {
  const int i = row & 15, mt = row >> 4;
  return (uint32_t)((i * MT + mt) * rowb + ((chunk ^ i) << 4));
}

// 16 int8 weights {-1, 0, +1} of one fragment (16 two-bit codes)
__device__ __forceinline__ i32x4 tunpack(uint32_t w) {
  return i32x4{(int)unpack4(w, 0), (int)unpack4(w, 1), (int)unpack4(w, 2), (int)unpack4(w, 3)};
}

}  // namespace

// ---------------------------------------------------------------------------
// weight preparation
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(64) void tprep_kernel(const uint32_t* __restrict__ packed, const float* __restrict__ s,
                                                   const int32_t* __restrict__ col, int R, int K, int C,
                                                   u32x4* __restrict__ tw, int32_t* __restrict__ mval,
                                                   float* __restrict__ rmul) {
  const int64_t t = blockIdx.x;
  const int l = threadIdx.x, j = l & 15, g = l >> 4;
  const int64_t ntiles = (int64_t)R * K;
  bool alive = false;
  if (t < ntiles) {
    const int c = col[t];
    alive = c >= 0 && c < C;
  }
  u32x4 v = {0, 0, 0, 0};
  if (alive) {
    const uint32_t* tile = packed + t * (64 * 4);
#pragma unroll
    for (int n = 0; n < 4; ++n) v[n] = tile[(4 * j + n) * 4 + g];   // output column 4j + n, inputs 16g..16g+15
  }
  tw[t * 64 + l] = v;
  if (l == 0) {
    int m = 0;
    if (t < ntiles) {
      const int r = (int)(t / K);
      const RowFix fx = row_fixed_point<64>(s + (int64_t)r * K, col + (int64_t)r * K, K, C);
      if (alive) m = (int)rintf(ldexpf(s[t], fx.e));
      if (t == (int64_t)r * K) rmul[r] = fx.mult;
    }
    mval[t] = m;
  }
}

// ---------------------------------------------------------------------------
// gate/up
// ---------------------------------------------------------------------------
struct TSlot {
  u32x4 wg, wu;      // fragment words of the gate and up tiles
  int mg, mu;        // their fixed-point scales
  int cg, cu;        // input column blocks (dead -> 0, weights are zero)
};

template <int MT>
__global__ __launch_bounds__(512, 1) void tgu_kernel(TGUArgs a) {
  constexpr int TM = 16 * MT;
  constexpr int ROWB = 2048;   // int8 panel row stride: d_model <= 2048
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = uniform(tid >> 6);
  const int i = lane & 15, g = lane >> 4;
  const int tb = (int)blockIdx.x / a.H, half = (int)blockIdx.x - tb * a.H;
  const int64_t t0 = (int64_t)tb * TM;
  const int d_model = a.d_model;
  const int cin = d_model / 64;
  const int64_t d_ff = (int64_t)a.R_ff * 64;
  const int K = a.K;
  const int RH = (a.R_ff + a.H - 1) / a.H;
  const int r_lo = half * RH, r_hi = (r_lo + RH) < a.R_ff ? (r_lo + RH) : a.R_ff;
  const int64_t ztile = (int64_t)a.R_ff * K;
  int2* ctab = reinterpret_cast<int2*>(smem + (size_t)TM * ROWB);
  float* hred = reinterpret_cast<float*>(smem);   // reused after the loop: [8 waves][TM]
  __shared__ float s_sx[TM];

  // ---- column table of this slice
  for (int e = tid; e < (r_hi - r_lo) * K; e += 512) {
    const int64_t ge = (int64_t)r_lo * K + e;
    int cg = a.cg[ge], cu = a.cu[ge];
    cg = (cg >= 0 && cg < cin) ? cg : 0;
    cu = (cu >= 0 && cu < cin) ? cu : 0;
    ctab[e] = make_int2(cg, cu);
  }

  const int nrows = r_hi > r_lo + w ? (r_hi - r_lo - w + 7) / 8 : 0;
  const int KP = (K + TG_RING - 1) / TG_RING * TG_RING;
  int rn = 0, rk = 0;
  auto fetch_w = [&](TSlot& S) {
    const bool live = rn < nrows && rk < K;
    const int r = r_lo + w + 8 * rn;
    const int64_t e = live ? (int64_t)r * K + rk : ztile;
    S.wg = a.twg[e * 64 + lane];
    S.wu = a.twu[e * 64 + lane];
    S.mg = a.mg[e];
    S.mu = a.mu[e];
    S.cg = live ? (r - r_lo) * K + rk : -1;
  };
  auto fetch_c = [&](TSlot& S) {
    const int2 c = ctab[S.cg >= 0 ? S.cg : 0];
    S.cg = c.x;
    S.cu = c.y;
    if (++rk == KP) {
      rk = 0;
      ++rn;
    }
  };
  TSlot P[TG_RING];
  auto prefetch_ring = [&]() {
    int sn = 0, sk = 0;
#pragma unroll
    for (int sl = 0; sl < TG_RING; ++sl) {
      rn = sn;
      rk = sk;
      fetch_w(P[sl]);
      if (++sk == KP) {
        sk = 0;
        ++sn;
      }
    }
    rn = 0;
    rk = 0;
  };

  // ---- sx of the block's tokens, the int8 x panel, then the ring's first weights: every load is
  // unconditional (clamped addresses, zero selected afterwards) so that each store below waits
  // only for its own load
  const int64_t tsx = t0 + (tid & 63);
  const float sxv = a.sx[tsx < a.N ? tsx : a.N - 1];
  {
    constexpr int CPR = ROWB / 16;
    constexpr int PIT = TM * CPR / 512;
    const int cpr = d_model / 16;
    u32x4 pv[PIT];
#pragma unroll
    for (int it = 0; it < PIT; ++it) {
      const int e = tid + 512 * it;
      const int row = e / CPR, cc = e % CPR;
      const int64_t t = t0 + row;
      const u32x4 v = *reinterpret_cast<const u32x4*>(a.xq + (t < a.N ? t : a.N - 1) * d_model +
                                                      16 * (cc < cpr ? cc : cpr - 1));
      pv[it] = (cc < cpr && t < a.N) ? v : u32x4{0, 0, 0, 0};
    }
    prefetch_ring();
    if (w == 0) s_sx[tid] = tsx < a.N ? sxv : 0.f;
#pragma unroll
    for (int it = 0; it < PIT; ++it) {
      const int e = tid + 512 * it;
      *reinterpret_cast<u32x4*>(smem + tpanel_addr<MT>(e / CPR, e % CPR, ROWB)) = pv[it];
    }
  }
  float hmax[MT][4];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int v = 0; v < 4; ++v) hmax[mt][v] = 0.f;
  __syncthreads();

  if (nrows > 0) {
#pragma unroll
    for (int sl = 0; sl < TG_RING; ++sl) fetch_c(P[sl]);
    const uint32_t lbase = (uint32_t)(i * MT * ROWB);
    i32x4 ag[MT][4], au[MT][4];
    // a (gate, up) tile pair as 16 steps (tile, 16-column group n, token-tile half): a step's two
    // MFMAs give block partials P, whose acc += m * P runs in the next step beside that step's
    // MFMAs.  Scheduling fences between steps bound the live partials to two steps and the
    // activation fragments to one tile (the up fragments are read during the gate's last group).
    static_assert(MT == 4, "two token tiles per step");
    auto compute = [&](const TSlot& S) {
      const int mg = uniform(S.mg), mu = uniform(S.mu);
      const uint32_t ag0 = lbase + (((uniform(S.cg) * 4 + g) ^ i) << 4);
      const uint32_t au0 = lbase + (((uniform(S.cu) * 4 + g) ^ i) << 4);
      i32x4 av[MT], avu[MT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) av[mt] = __builtin_bit_cast(i32x4, lds16t(smem, ag0 + mt * ROWB));
      i32x4 Pp[2], f;
#pragma unroll
      for (int q = 0; q < 17; ++q) {
        i32x4 Pn[2];
        if (q < 16) {
          const bool up = q >= 8;
          const int n = (q >> 1) & 3, hh = q & 1;
          if (q == 6) {
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) avu[mt] = __builtin_bit_cast(i32x4, lds16t(smem, au0 + mt * ROWB));
          }
          if (q == 8) {
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) av[mt] = avu[mt];
          }
          if (hh == 0) f = tunpack(up ? S.wu[n] : S.wg[n]);
#pragma unroll
          for (int u = 0; u < 2; ++u) Pn[u] = mfma_i8_k64(av[2 * hh + u], f, i32x4{0, 0, 0, 0});
        }
        if (q > 0) {
          const int pq = q - 1;
          const int n = (pq >> 1) & 3, hh = pq & 1;
          // the empty asm keeps each tile's multiply-add a v_mad_i32_i24 (no reassociation)
#pragma unroll
          for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
              if (pq < 8) {
                int acc = __mul24(Pp[u][v], mg) + ag[2 * hh + u][n][v];
                asm("" : "+v"(acc));
                ag[2 * hh + u][n][v] = acc;
              } else {
                int acc = __mul24(Pp[u][v], mu) + au[2 * hh + u][n][v];
                asm("" : "+v"(acc));
                au[2 * hh + u][n][v] = acc;
              }
            }
        }
#pragma unroll
        for (int u = 0; u < 2; ++u) Pp[u] = Pn[u];
        __builtin_amdgcn_sched_barrier(0);
      }
    };
    __builtin_amdgcn_sched_barrier(0);
    for (int n = 0; n < nrows; ++n) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          ag[mt][q] = i32x4{0, 0, 0, 0};
          au[mt][q] = i32x4{0, 0, 0, 0};
        }
      for (int k = 0; k < KP; k += TG_RING) {
#pragma unroll
        for (int sl = 0; sl < TG_RING; ++sl) {
          compute(P[sl]);
          fetch_w(P[sl]);
          fetch_c(P[sl]);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
      // epilogue of row r: g, u = acc * (2^-e * sx); h = silu(g) * u (bf16)
      const int r = r_lo + w + 8 * n;
      const float fg = a.rmg[r], fu = a.rmu[r];
      const int64_t col0 = (int64_t)r * 64 + 4 * i;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int64_t t = t0 + 16 * mt + 4 * g + v;
          const float sxv = s_sx[16 * mt + 4 * g + v];
          const float cg = fg * sxv, cu = fu * sxv;
          uint32_t hb[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const float gv = (float)ag[mt][q][v] * cg;
            const float uv = (float)au[mt][q][v] * cu;
            hb[q] = f2bf(silu_f(gv) * uv);
            hmax[mt][v] = fmaxf(hmax[mt][v], fabsf(bf2f(hb[q])));
          }
          if (t < a.N)
            *reinterpret_cast<u32x2*>(a.h + t * d_ff + col0) = u32x2{hb[0] | (hb[1] << 16), hb[2] | (hb[3] << 16)};
        }
    }
  }

  // ---- per-token max |h| of this slice: lanes of one g share tokens, then waves via LDS
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      float m = hmax[mt][v];
#pragma unroll
      for (int o = 1; o < 16; o <<= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
      hmax[mt][v] = m;
    }
  __syncthreads();   // the panel is no longer read
  if (i == 0) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int v = 0; v < 4; ++v) hred[w * TM + 16 * mt + 4 * g + v] = hmax[mt][v];
  }
  __syncthreads();
  if (tid < TM) {
    float m = hred[tid];
#pragma unroll
    for (int ww = 1; ww < 8; ++ww) m = fmaxf(m, hred[ww * TM + tid]);
    const int64_t t = t0 + tid;
    if (t < a.N) a.hmax[(int64_t)half * a.N + t] = m;
  }
}

// ---------------------------------------------------------------------------
// down (+ on-the-fly quantisation of h)
// ---------------------------------------------------------------------------
struct TDSlot {
  u32x4 wd;
  int m;
  int c;
};

__global__ __launch_bounds__(512, 1) void tdn_kernel(TDNArgs a) {
  constexpr int TM = 16;
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  __shared__ float s_scale[TM], s_sh[TM];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = uniform(tid >> 6);
  const int i = lane & 15, g = lane >> 4;
  const int64_t t0 = (int64_t)blockIdx.x * TM;
  const int d_ff = a.d_ff;
  const int rowb = d_ff;   // int8 panel row stride (a multiple of 256)
  const int Kd = a.Kd;
  const int64_t ztile = (int64_t)a.R_m * Kd;

  // ---- per-token absmax over the slices -> quantisation scale (as quantize_act_kernel)
  if (tid < TM) {
    const int64_t t = t0 + tid;
    float amax = 0.f;
    if (t < a.N)
      for (int hh = 0; hh < a.H; ++hh) amax = fmaxf(amax, a.hmax[(int64_t)hh * a.N + t]);
    amax = fmaxf(amax, 1e-8f);
    s_scale[tid] = __fdiv_rn(128.0f, amax);
    s_sh[tid] = amax * 0.0078125f;
    if (a.sh_out && t < a.N) a.sh_out[t] = amax * 0.0078125f;
  }

  // ---- ring of down tiles: wave w owns rows rm = w, w+8, ...
  const int nrows = (a.R_m - w + 7) / 8;
  const int KP = (Kd + TD_RING - 1) / TD_RING * TD_RING;
  int rn = 0, rk = 0;
  auto fetch = [&](TDSlot& S) {
    const bool live = rn < nrows && rk < Kd;
    const int rm = w + 8 * rn;
    const int64_t e = live ? (int64_t)rm * Kd + rk : ztile;
    S.wd = a.twd[e * 64 + lane];
    S.m = a.md[e];
    const int c = a.cd[live ? e : 0];
    S.c = (live && c >= 0 && c < a.C_d) ? c : 0;
    if (++rk == KP) {
      rk = 0;
      ++rn;
    }
  };
  TDSlot P[TD_RING];
#pragma unroll
  for (int sl = 0; sl < TD_RING; ++sl) fetch(P[sl]);
  __syncthreads();   // s_scale

  // ---- panel: the 16 h rows quantised to int8.  A unit is 16 values (32 bytes of h);
  // batches of 8 units per thread are loaded before any is converted.
  {
    constexpr int UB = 8;
    const int upr = d_ff / 16;          // units per row
    const int units = TM * upr;
    for (int base = tid; base < units; base += 512 * UB) {
      u32x4 hv[UB][2];
#pragma unroll
      for (int b = 0; b < UB; ++b) {
        int e = base + 512 * b;
        e = e < units ? e : units - 1;
        const int row = e / upr, cc = e - row * upr;
        int64_t t = t0 + row;
        t = t < a.N ? t : a.N - 1;
        const u32x4* hp = reinterpret_cast<const u32x4*>(a.h + t * (int64_t)d_ff + 16 * cc);
        hv[b][0] = hp[0];
        hv[b][1] = hp[1];
      }
#pragma unroll
      for (int b = 0; b < UB; ++b) {
        const int eb = base + 512 * b;
        const int e = eb < units ? eb : units - 1;   // a clamped unit rewrites the last unit's own bytes
        const int row = e / upr, cc = e - row * upr;
        const int64_t t = t0 + row;
        const float sc = s_scale[row];
        u32x4 q = {0, 0, 0, 0};
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const uint32_t wv = hv[b][u >> 2][u & 3];
          const float lo = fminf(fmaxf(rintf(__fmul_rn(bf_lo(wv), sc)), -128.f), 127.f);
          const float hi = fminf(fmaxf(rintf(__fmul_rn(bf_hi(wv), sc)), -128.f), 127.f);
          const uint32_t pair = ((uint32_t)((int)lo) & 0xffu) | (((uint32_t)((int)hi) & 0xffu) << 8);
          q[u >> 1] |= pair << (16 * (u & 1));
        }
        if (t >= a.N) q = u32x4{0, 0, 0, 0};
        if (a.hq_out && t < a.N && eb < units)
          *reinterpret_cast<u32x4*>(a.hq_out + t * (int64_t)d_ff + 16 * cc) = q;
        *reinterpret_cast<u32x4*>(smem + tpanel_addr<1>(row, cc, rowb)) = q;
      }
    }
  }
  __syncthreads();
  if (nrows <= 0) return;

  const uint32_t lbase = (uint32_t)(i * rowb);
  i32x4 acc[4];
  __builtin_amdgcn_sched_barrier(0);
  for (int n = 0; n < nrows; ++n) {
#pragma unroll
    for (int q = 0; q < 4; ++q) acc[q] = i32x4{0, 0, 0, 0};
    for (int k = 0; k < KP; k += TD_RING) {
#pragma unroll
      for (int sl = 0; sl < TD_RING; ++sl) {
        const int c = uniform(P[sl].c);
        const int m = uniform(P[sl].m);
        const i32x4 av = __builtin_bit_cast(i32x4, lds16t(smem, lbase + (((c * 4 + g) ^ i) << 4)));
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const i32x4 Pq = mfma_i8_k64(av, tunpack(P[sl].wd[q]), i32x4{0, 0, 0, 0});
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            int t = __mul24(Pq[v], m) + acc[q][v];
            asm("" : "+v"(t));
            acc[q][v] = t;
          }
        }
        fetch(P[sl]);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    // epilogue of down row rm: y = f32(f32(acc) * 2^-e) * sh (+ residual) -> bf16
    const int rm = w + 8 * n;
    const float fd = a.rmd[rm];
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int64_t t = t0 + 4 * g + v;
      if (t >= a.N) continue;
      const float shv = s_sh[4 * g + v];
      const int64_t off = t * a.d_model + (int64_t)rm * 64 + 4 * i;
      float o[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) o[q] = __fmul_rn(__fmul_rn((float)acc[q][v], fd), shv);
      if (a.resid) {
        float rv[4];
        load_bf16<4>(a.resid + off, rv);
#pragma unroll
        for (int q = 0; q < 4; ++q) o[q] += rv[q];
      }
      store_bf16<4>(a.out + off, o);
    }
  }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
size_t tprep_bytes(int64_t ntiles, int R) {
  // words (1 KB per tile, + zero tile) | m per tile | row multipliers, each 256-aligned
  auto al = [](size_t v) { return (v + 255) & ~(size_t)255; };
  return al((size_t)(ntiles + 1) * 1024) + al((size_t)(ntiles + 1) * 4) + al((size_t)R * 4);
}

int launch_tprep(const uint32_t* packed, const float* s, const int32_t* col, int R, int K, int C, void* out,
                 const u32x4** tw, const int32_t** mval, const float** rmul, hipStream_t st) {
  auto al = [](size_t v) { return (v + 255) & ~(size_t)255; };
  const int64_t nt = (int64_t)R * K;
  char* p = static_cast<char*>(out);
  u32x4* w = reinterpret_cast<u32x4*>(p);
  int32_t* m = reinterpret_cast<int32_t*>(p + al((size_t)(nt + 1) * 1024));
  float* f = reinterpret_cast<float*>(p + al((size_t)(nt + 1) * 1024) + al((size_t)(nt + 1) * 4));
  *tw = w;
  *mval = m;
  *rmul = f;
  hipLaunchKernelGGL(tprep_kernel, dim3((unsigned)(nt + 1)), dim3(64), 0, st, packed, s, col, R, K, C, w, m, f);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

bool tsplit_supported(int B, int d_model, int R_ff, int R_m, int Kg, int Ku, int Kd) {
  if (B != 64) return false;
  if (Kg != Ku || Kg < 1 || Kd < 1) return false;
  if (d_model % 256 || d_model > 2048) return false;     // int8 x panel rows of 2048 bytes
  const int64_t d_ff = (int64_t)R_ff * 64;
  if (d_ff % 256 || 16 * d_ff + 256 > 163840) return false;   // int8 h panel of 16 rows + scales
  if ((int64_t)64 * 2048 + (int64_t)R_ff * Kg * 8 + 256 > 163840) return false;   // panel + column table + sx
  (void)R_m;
  return true;
}

int tgu_slices(int64_t N) {
  const int64_t blocks = (N + 63) / 64;
  return blocks >= 256 ? 1 : (blocks >= 128 ? 2 : 4);
}

int launch_tgu(const TGUArgs& a, hipStream_t st) {
  if (a.N == 0) return 0;
  auto kern = tgu_kernel<4>;
  static bool configured = false;
  if (!configured) {
    if (hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, 163840 - 256) !=
        hipSuccess)
      return -1;
    configured = true;
  }
  const int RH = (a.R_ff + a.H - 1) / a.H;
  const size_t lds = (size_t)64 * 2048 + (size_t)RH * a.K * 8;
  const int64_t blocks = (a.N + 63) / 64;
  hipLaunchKernelGGL(kern, dim3((unsigned)(blocks * a.H)), dim3(512), lds, st, a);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_tdn(const TDNArgs& a, hipStream_t st) {
  if (a.N == 0) return 0;
  static bool configured = false;
  if (!configured) {
    if (hipFuncSetAttribute((const void*)tdn_kernel, hipFuncAttributeMaxDynamicSharedMemorySize, 163840 - 256) !=
        hipSuccess)
      return -1;
    configured = true;
  }
  const size_t lds = (size_t)16 * a.d_ff;
  hipLaunchKernelGGL(tdn_kernel, dim3((unsigned)((a.N + 15) / 16)), dim3(512), lds, st, a);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace lbk
