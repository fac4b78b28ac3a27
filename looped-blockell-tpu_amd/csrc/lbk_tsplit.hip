// lbk_tsplit.hip — ternary SwiGLU FFN with int8 MFMA, B = 64 (gfx950).
//
// Arithmetic (the same as the row-block kernels of lbk_ternary.hip): for block
// row r the fp32 block scales are used in the fixed point m[r,k] * 2^-e[r]
// (row_fixed_point: m up to 16 bits, sum_k m * P inside int32), each block's
// exact int32 partial P = x . t comes from int8 MFMAs, and acc += m * P is one
// 24-bit integer multiply-add per element; the output is
// y = f32(f32(acc) * 2^-e[r]) * sx[token].
//
// Weight encodings of the prepared tiles.  Gate and up: the MFMA B fragments as
// int8 t (4 KB per 64 x 64 tile, fragment-major: [tile][16-column group][lane] x 16
// bytes), so the gate/up kernel feeds its loads straight to the MFMA (each CU
// reads its share of tiles once per 64 tokens, well within what L2 delivers).
// Down: every weight as t + 1 in {0, 1, 2} (2 bits, 1 KB per tile), so a byte
// of weights is just (word >> 2q) & 0x03030303 (no table lookup), and the MFMA
// computes x . (t + 1) = P + sum(x) starting from C = -sum(x): the per-token
// sums of each 64-wide activation block are kept in LDS beside the activation
// panel (int32, exact).  The down kernel reuses each tile for only 16 tokens,
// so its weights stay in the 2-bit form (a quarter of the bytes through L2).
//
//   tprep_kernel  per call or once per weight version, gate, up and down in one
//                 launch: packed tiles [R,K,64,4] -> the fragment-major forms
//                 above (dead slots and one appended tile encode t = 0), m per
//                 tile (zero for dead slots and the appended tile), and 2^-e[r]
//                 per row.
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

typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

// ring depths (tile slots prefetched ahead): a gate/up slot is a (gate, up) tile pair, 32
// MFMAs; a down slot is one tile, 4 MFMAs
constexpr int TG_RING = 2;

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

// 16 int8 weights t + 1 in {0, 1, 2} of one fragment (16 two-bit fields)
__device__ __forceinline__ i32x4 tunpack(uint32_t w) {
  return i32x4{(int)(w & 0x03030303u), (int)((w >> 2) & 0x03030303u), (int)((w >> 4) & 0x03030303u),
               (int)((w >> 6) & 0x03030303u)};
}

// 2-bit codes of the storage format (00 -> 0, 01 -> +1, 11 -> -1, 10 -> 0) -> t + 1
// (0 -> 01, +1 -> 10, -1 -> 00), field by field
__device__ __forceinline__ uint32_t recode_t1(uint32_t w) {
  const uint32_t b0 = w & 0x55555555u, b1 = (w >> 1) & 0x55555555u;
  return ((b0 & ~b1) << 1) | (~w & 0x55555555u);
}

// sum of the 16 int8 values of a 16-byte chunk
__device__ __forceinline__ int sum16_i8(const u32x4& v) {
  int s = 0;
#pragma unroll
  for (int d = 0; d < 4; ++d) s = __builtin_amdgcn_sdot4((int)v[d], 0x01010101, s, false);
  return s;
}

}  // namespace

// ---------------------------------------------------------------------------
// weight preparation
// ---------------------------------------------------------------------------
__device__ __forceinline__ void tprep_tile(const uint32_t* __restrict__ packed, const float* __restrict__ s,
                                           const int32_t* __restrict__ col, int R, int K, int C, bool int8,
                                           u32x4* __restrict__ tw, int32_t* __restrict__ mval,
                                           float* __restrict__ rmul, int64_t t) {
  const int l = threadIdx.x, j = l & 15, g = l >> 4;
  const int64_t ntiles = (int64_t)R * K;
  bool alive = false;
  if (t < ntiles) {
    const int c = col[t];
    alive = c >= 0 && c < C;
  }
  // storage words of column 4j + n, inputs 16g..16g+15 (dead: all codes 0, t = 0)
  uint32_t wv[4] = {0u, 0u, 0u, 0u};
  if (alive) {
    const uint32_t* tile = packed + t * (64 * 4);
#pragma unroll
    for (int n = 0; n < 4; ++n) wv[n] = tile[(4 * j + n) * 4 + g];
  }
  if (int8) {
    // group n: the 16 int8 weights of column 4j + n, byte 4q + b = input 16g + 4q + b
#pragma unroll
    for (int n = 0; n < 4; ++n)
      tw[(t * 4 + n) * 64 + l] = u32x4{unpack4(wv[n], 0), unpack4(wv[n], 1), unpack4(wv[n], 2), unpack4(wv[n], 3)};
  } else {
    tw[t * 64 + l] = u32x4{recode_t1(wv[0]), recode_t1(wv[1]), recode_t1(wv[2]), recode_t1(wv[3])};
  }
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

// the three weights of a forward in one launch: workgroup b prepares tile b - first[t] of
// weight t (each weight has R * K + 1 tiles, the last one the zero tile)
__global__ __launch_bounds__(64) void tprep_kernel(TPrepJobs jobs) {
  int t = 0;
#pragma unroll
  for (int u = 1; u < 3; ++u)
    if ((int64_t)blockIdx.x >= jobs.first[u]) t = u;
  const TPrepJob& J = jobs.job[t];
  tprep_tile(J.packed, J.s, J.col, J.R, J.K, J.C, J.int8, J.tw, J.mval, J.rmul, (int64_t)blockIdx.x - jobs.first[t]);
}

// ---------------------------------------------------------------------------
// gate/up
// ---------------------------------------------------------------------------
struct TSlot {
  u32x4 wg[4], wu[4];   // int8 fragments of the gate and up tiles, one per 16-column group
  int cg, cu;           // input column blocks (dead -> 0, weights are zero)
  int mg, mu;           // their fixed-point scales
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
  const int nrem = (int)(a.N - t0 < TM ? a.N - t0 : TM);   // tokens of this block that exist
  // LDS: x panel | slot table {cg, cu, mg, mu} of this slice | row table {2^-e_g, 2^-e_u} |
  // per-token epilogue factors.
  // Every per-slot and per-row value the loop needs is read from LDS: a scalar load in the
  // loop would make each slot wait for the latest one (scalar loads return out of order).
  int4* ctab = reinterpret_cast<int4*>(smem + (size_t)TM * ROWB);
  float2* rtab = reinterpret_cast<float2*>(smem + (size_t)TM * ROWB + (size_t)RH * K * 16);
  // per token: (-log2(e) * sx, 1 / sx^2) for the epilogue
  float2* s_tf = reinterpret_cast<float2*>(smem + (size_t)TM * ROWB + (size_t)RH * K * 16 + (size_t)RH * 8);
  float* hred = reinterpret_cast<float*>(smem);   // reused after the loop: [8 waves][TM]
  __shared__ float s_sx[TM];

  for (int e = tid; e < (r_hi - r_lo) * K; e += 512) {
    const int64_t ge = (int64_t)r_lo * K + e;
    int cg = a.cg[ge], cu = a.cu[ge];
    cg = (cg >= 0 && cg < cin) ? cg : 0;
    cu = (cu >= 0 && cu < cin) ? cu : 0;
    ctab[e] = make_int4(cg, cu, a.mg[ge], a.mu[ge]);
  }
  for (int e = tid; e < r_hi - r_lo; e += 512) rtab[e] = make_float2(a.rmg[r_lo + e], a.rmu[r_lo + e]);

  const int nrows = r_hi > r_lo + w ? (r_hi - r_lo - w + 7) / 8 : 0;
  const int KP = (K + TG_RING - 1) / TG_RING * TG_RING;
  int rn = 0, rk = 0;
  auto fetch_w = [&](TSlot& S) {
    const bool live = rn < nrows && rk < K;
    const int r = r_lo + w + 8 * rn;
    const int64_t e = live ? (int64_t)r * K + rk : ztile;
#pragma unroll
    for (int n = 0; n < 4; ++n) S.wg[n] = a.twg[(e * 4 + n) * 64 + lane];
#pragma unroll
    for (int n = 0; n < 4; ++n) S.wu[n] = a.twu[(e * 4 + n) * 64 + lane];
    S.cg = live ? (r - r_lo) * K + rk : -1;
  };
  auto fetch_c = [&](TSlot& S) {
    const int4 c = ctab[S.cg >= 0 ? S.cg : 0];   // padding slots: zero tiles, any entry
    S.cg = c.x;
    S.cu = c.y;
    S.mg = c.z;
    S.mu = c.w;
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
  const float sx_own = a.sx[tsx < a.N ? tsx : a.N - 1];
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
    if (w == 0) {
      const float sv = tsx < a.N ? sx_own : 0.f;
      s_sx[tid] = sv;
      s_tf[tid] = make_float2(sv * -1.4426950408889634f, __builtin_amdgcn_rcpf(sv * sv));
    }
#pragma unroll
    for (int it = 0; it < PIT; ++it) {
      const int e = tid + 512 * it;
      *reinterpret_cast<u32x4*>(smem + tpanel_addr<MT>(e / CPR, e % CPR, ROWB)) = pv[it];
    }
  }
  // running max |h| per token of this lane: bf16 bit patterns of |h| (non-negative, so integer
  // order is float order), two tokens (v, v + 1) per register
  u16x2 hmax[MT][2];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int v = 0; v < 2; ++v) hmax[mt][v] = u16x2{0, 0};
  __syncthreads();

  if (nrows > 0) {
#pragma unroll
    for (int sl = 0; sl < TG_RING; ++sl) fetch_c(P[sl]);
    const uint32_t lbase = (uint32_t)(i * MT * ROWB);
    i32x4 ag[MT][4], au[MT][4];
    // a (gate, up) tile pair as 16 steps (tile, 16-column group n, token-tile half): a step's two
    // MFMAs give block partials P (int8 t straight from the ring, C = 0), whose acc += m * P runs
    // in the next step beside that step's MFMAs.  Scheduling fences between steps bound the live
    // partials to two steps and the activation fragments to one tile (the up fragments are read
    // during the gate's last group).
    static_assert(MT == 4, "two token tiles per step");
    auto compute = [&](const TSlot& S) {
      const int mg = uniform(S.mg), mu = uniform(S.mu);
      const int cgc = uniform(S.cg), cuc = uniform(S.cu);
      const uint32_t ag0 = lbase + (((cgc * 4 + g) ^ i) << 4);
      const uint32_t au0 = lbase + (((cuc * 4 + g) ^ i) << 4);
      i32x4 av[MT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) av[mt] = __builtin_bit_cast(i32x4, lds16t(smem, ag0 + mt * ROWB));
      const i32x4 zero = {0, 0, 0, 0};
      i32x4 Pp[2];
#pragma unroll
      for (int q = 0; q < 17; ++q) {
        i32x4 Pn[2];
        if (q < 16) {
          const bool up = q >= 8;
          const int n = (q >> 1) & 3, hh = q & 1;
          // the up fragments replace the gate's one half at a time, a step before their use
          // (step 7 is the gate's last use of token tiles 0-1, step 8 of 2-3)
          if (q == 7 || q == 8) {
#pragma unroll
            for (int mt = 2 * (q - 7); mt < 2 * (q - 7) + 2; ++mt)
              av[mt] = __builtin_bit_cast(i32x4, lds16t(smem, au0 + mt * ROWB));
          }
          const i32x4 f = __builtin_bit_cast(i32x4, up ? S.wu[n] : S.wg[n]);
#pragma unroll
          for (int u = 0; u < 2; ++u) Pn[u] = mfma_i8_k64(av[2 * hh + u], f, zero);
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
      // epilogue of row r: with g = G * cg, u = U * cu (G, U the integer accumulators,
      // cg = 2^-e_g * sx, cu = 2^-e_u * sx),
      //   h = silu(g) * u = G * U / ((1 + 2^(G * k)) / (cg * cu)),  k = -log2(e) * cg,
      // where (1 + E) / C is one fma with 1 / C (clamped finite); h is rounded to bf16
      const int r = r_lo + w + 8 * n;
      const float2 fr = rtab[r - r_lo];
      const float fg = fr.x, fu = fr.y;
      // 32-bit element offsets from the token block's first row (< 64 * d_ff), token bounds as a
      // compare against the rows left: no 64-bit address per (mt, v) stays live across the loop
      uint32_t dffu = (uint32_t)d_ff;
      int nr = nrem;
      asm("" : "+s"(dffu), "+s"(nr));   // keeps offsets and bounds from being hoisted out of the row loop
      const uint32_t lane_off = (uint32_t)(4 * g) * dffu + (uint32_t)(r * 64 + 4 * i);
      const int64_t rb = t0 * d_ff;
      const float ifgu = __builtin_amdgcn_rcpf(fg * fu);   // a power of two
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int tl = 16 * mt + 4 * g + v;
          const bool tok = tl < nr;
          const uint32_t off = lane_off + (uint32_t)(16 * mt + v) * dffu;
          // with cg = 2^-e_g * sx, cu = 2^-e_u * sx: k = -log2(e) * cg, 1 / (cg * cu) =
          // 2^(e_g + e_u) / sx^2, from per-token factors and the row's power of two
          const float2 tf = s_tf[tl];
          const float k = fg * tf.x;
          const float ic = fminf(tf.y * ifgu, 1e38f);
          float hv[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const float G = (float)ag[mt][q][v], U = (float)au[mt][q][v];
            const float E = __builtin_amdgcn_exp2f(G * k);
            hv[q] = (G * U) * __builtin_amdgcn_rcpf(fmaf(E, ic, ic));
          }
          const uint32_t p01 = pack2_bf16(hv[0], hv[1]), p23 = pack2_bf16(hv[2], hv[3]);
          const u16x2 pm = __builtin_elementwise_max(__builtin_bit_cast(u16x2, p01 & 0x7fff7fffu),
                                                     __builtin_bit_cast(u16x2, p23 & 0x7fff7fffu));
          const unsigned short tm = pm[0] > pm[1] ? pm[0] : pm[1];
          hmax[mt][v >> 1] = __builtin_elementwise_max(hmax[mt][v >> 1],
                                                       (v & 1) ? u16x2{0, tm} : u16x2{tm, 0});
          if (tok) *reinterpret_cast<u32x2*>(a.h + rb + off) = u32x2{p01, p23};
          // optional export of the integer accumulators and the fp32 pre-activations
          if (a.acc_g && tok) {
            *reinterpret_cast<i32x4*>(a.acc_g + rb + off) = i32x4{ag[mt][0][v], ag[mt][1][v], ag[mt][2][v], ag[mt][3][v]};
            *reinterpret_cast<i32x4*>(a.acc_u + rb + off) = i32x4{au[mt][0][v], au[mt][1][v], au[mt][2][v], au[mt][3][v]};
          }
          if (a.g_pre && tok) {
            const float sxv = s_sx[tl];
            float gp[4], up[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              gp[q] = __fmul_rn(__fmul_rn((float)ag[mt][q][v], fg), sxv);
              up[q] = __fmul_rn(__fmul_rn((float)au[mt][q][v], fu), sxv);
            }
            *reinterpret_cast<float4*>(a.g_pre + rb + off) = make_float4(gp[0], gp[1], gp[2], gp[3]);
            *reinterpret_cast<float4*>(a.u_pre + rb + off) = make_float4(up[0], up[1], up[2], up[3]);
          }
        }
    }
  }

  // ---- per-token max |h| of this slice: lanes of one g share tokens, then waves via LDS
  float hm[MT][4];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      float m = bf2f(hmax[mt][v >> 1][v & 1]);
#pragma unroll
      for (int o = 1; o < 16; o <<= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
      hm[mt][v] = m;
    }
  __syncthreads();   // the panel is no longer read
  if (i == 0) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int v = 0; v < 4; ++v) hred[w * TM + 16 * mt + 4 * g + v] = hm[mt][v];
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
  int2 cm;   // input column block (dead -> 0), fixed-point scale
};

template <int NW, int RING, int UB>
__global__ __launch_bounds__(64 * NW, 1) void tdn_kernel(TDNArgs a) {
  constexpr int TM = 16;
  constexpr int NT = 64 * NW;
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  __shared__ float s_scale[TM], s_sh[TM];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = uniform(tid >> 6);
  const int i = lane & 15, g = lane >> 4;
  // workgroup -> (16-token block, row group grp of G: down rows grp, grp + G, ...)
  const int grp = (int)(blockIdx.x % (unsigned)a.G);
  const int64_t t0 = (int64_t)(blockIdx.x / (unsigned)a.G) * TM;
  const int d_ff = a.d_ff;
  const int rowb = d_ff;   // int8 panel row stride (a multiple of 256)
  const int Kd = a.Kd;
  const int64_t ztile = (int64_t)a.R_m * Kd;
  // LDS: int8 h panel | -sum(hq) per (input block, token) [C_d][TM] int32 | slot table {c, m} |
  // row table 2^-e (no scalar loads in the loop)
  int* rsum = reinterpret_cast<int*>(smem + (size_t)TM * d_ff);
  int2* dtab = reinterpret_cast<int2*>(smem + (size_t)TM * d_ff + (size_t)a.C_d * TM * 4);
  float* rtab = reinterpret_cast<float*>(smem + (size_t)TM * d_ff + (size_t)a.C_d * TM * 4 + (size_t)a.R_m * Kd * 8);
  for (int e = tid; e < a.R_m * Kd; e += NT) {
    const int c = a.cd[e];
    dtab[e] = make_int2((c >= 0 && c < a.C_d) ? c : 0, a.md[e]);
  }
  for (int e = tid; e < a.R_m; e += NT) rtab[e] = a.rmd[e];

  // ---- panel fill, part 1: this thread's first batch of h rows is requested before anything
  // else (the scales it needs come later).  A unit is 16 values (32 bytes of h) of one row.
  // With at least as many threads as units per row (upr), thread tid takes unit tid % upr of
  // the rows of row group tid / upr (NT / upr groups; one division per thread), otherwise units
  // tid, tid + NT, ... of every row; rows go in batches of UB whose loads are all issued before
  // any is converted.
  const int upr = d_ff / 16;          // units per row (a multiple of 16)
  const bool wide = upr > NT;
  const int rstep = wide ? 1 : NT / upr;
  const int rg = wide ? 0 : tid / upr;
  const int cc0 = wide ? tid : tid - rg * upr;
  const int ccstep = wide ? NT : upr;
  u32x4 hv[UB][2];
  auto load_batch = [&](int cc, int rb) {
#pragma unroll
    for (int b = 0; b < UB; ++b) {
      int64_t t = t0 + rb + b;
      t = t < a.N ? t : a.N - 1;
      const u32x4* hp = reinterpret_cast<const u32x4*>(a.h + t * (int64_t)d_ff + 16 * cc);
      hv[b][0] = hp[0];
      hv[b][1] = hp[1];
    }
  };
  // threads past the last whole row group (when upr does not divide NT) stay idle
  const bool filler = rg < rstep;
  const bool first = filler && cc0 < upr && rg * UB < TM;
  if (first) load_batch(cc0, rg * UB);

  // ---- per-token absmax over the slices -> quantisation scale (as quantize_act_kernel)
  if (tid < TM) {
    const int64_t t = t0 + tid;
    float amax = 0.f;
    if (t < a.N)
      for (int hh = 0; hh < a.H; ++hh) amax = fmaxf(amax, a.hmax[(int64_t)hh * a.N + t]);
    amax = fmaxf(amax, 1e-8f);
    s_scale[tid] = __fdiv_rn(128.0f, amax);
    s_sh[tid] = amax * 0.0078125f;
    if (a.sh_out && grp == 0 && t < a.N) a.sh_out[t] = amax * 0.0078125f;
  }

  // ---- ring of down tiles: wave w owns rows rm = grp + G (w + NW n)
  const int rows_g = (a.R_m - grp + a.G - 1) / a.G;
  const int nrows = (rows_g - w + NW - 1) / NW;
  const int KP = (Kd + RING - 1) / RING * RING;
  int rn = 0, rk = 0;
  auto fetch = [&](TDSlot& S) {
    const bool live = rn < nrows && rk < Kd;
    const int rm = grp + a.G * (w + NW * rn);
    const int64_t e = live ? (int64_t)rm * Kd + rk : ztile;
    S.wd = a.twd[e * 64 + lane];
    S.cm = make_int2(live ? (int)e : 0, 0);
    if (++rk == KP) {
      rk = 0;
      ++rn;
    }
  };
  TDSlot P[RING];
#pragma unroll
  for (int sl = 0; sl < RING; ++sl) fetch(P[sl]);
  __syncthreads();   // s_scale, dtab, rtab
  // slot metadata from LDS: for the prefetched slots here, for later ones one ring cycle ahead
  auto meta = [&](TDSlot& S) { S.cm = dtab[S.cm.x]; };   // padding slots: zero tiles, any entry
#pragma unroll
  for (int sl = 0; sl < RING; ++sl) meta(P[sl]);

  // ---- panel fill, part 2: the 16 h rows quantised to int8.  Quantisation per value: q =
  // clamp(rint(h * scale), -128, 127) computed as med3(h * scale, -128, 127) + 1.5 * 2^23 (the
  // add rounds to the nearest integer, ties to even, and leaves the int8 two's complement in
  // the low byte of the float); bytes of four values merged with two v_perm.
  {
    for (int cc = filler ? cc0 : upr; cc < upr; cc += ccstep) {
#pragma unroll 1
      for (int rb = rg * UB; rb < TM; rb += rstep * UB) {
        if (cc != cc0 || rb != rg * UB) load_batch(cc, rb);
#pragma unroll
        for (int b = 0; b < UB; ++b) {
          const int row = rb + b;
          const int64_t t = t0 + row;
          const float sc = s_scale[row];
          u32x4 q;
#pragma unroll
          for (int d = 0; d < 4; ++d) {
            // dword d of the result: values 4d .. 4d + 3 (bf16 pairs hv[.][d / 2][2 (d % 2)], + 1)
            const uint32_t w0 = hv[b][d >> 1][2 * (d & 1)], w1 = hv[b][d >> 1][2 * (d & 1) + 1];
            const float v0 = __builtin_amdgcn_fmed3f(__fmul_rn(bf_lo(w0), sc), -128.f, 127.f) + 12582912.0f;
            const float v1 = __builtin_amdgcn_fmed3f(__fmul_rn(bf_hi(w0), sc), -128.f, 127.f) + 12582912.0f;
            const float v2 = __builtin_amdgcn_fmed3f(__fmul_rn(bf_lo(w1), sc), -128.f, 127.f) + 12582912.0f;
            const float v3 = __builtin_amdgcn_fmed3f(__fmul_rn(bf_hi(w1), sc), -128.f, 127.f) + 12582912.0f;
            const uint32_t lo = __builtin_amdgcn_perm(__float_as_uint(v1), __float_as_uint(v0), 0x0c0c0400u);
            const uint32_t hi = __builtin_amdgcn_perm(__float_as_uint(v3), __float_as_uint(v2), 0x04000c0cu);
            q[d] = lo | hi;
          }
          if (t >= a.N) q = u32x4{0, 0, 0, 0};
          if (a.hq_out && grp == 0 && t < a.N) *reinterpret_cast<u32x4*>(a.hq_out + t * (int64_t)d_ff + 16 * cc) = q;
          // -sum(hq) of each 64-wide block: its 4 units sit in 4 adjacent lanes, all of which
          // take part (upr is a multiple of 16, so a 4-lane group is in or out as a whole)
          int sm = sum16_i8(q);
          sm += __shfl_xor(sm, 1, 64);
          sm += __shfl_xor(sm, 2, 64);
          if ((cc & 3) == 0) rsum[(cc >> 2) * TM + row] = -sm;
          *reinterpret_cast<u32x4*>(smem + tpanel_addr<1>(row, cc, rowb)) = q;
        }
      }
    }
  }
  __syncthreads();
  if (nrows <= 0) return;

  // Software pipeline over the slots of a row: slot s issues its LDS read one slot early, its
  // MFMAs (partials P) beside the multiply-adds of slot s - 1, which drain at the row's end.
  const uint32_t lbase = (uint32_t)(i * rowb);
  auto a_frag = [&](const TDSlot& S) {
    return __builtin_bit_cast(i32x4, lds16t(smem, lbase + (((uniform(S.cm.x) * 4 + g) ^ i) << 4)));
  };
  auto c_frag = [&](const TDSlot& S) {
    return *reinterpret_cast<const i32x4*>(rsum + uniform(S.cm.x) * TM + 4 * g);
  };
  auto madd = [&](i32x4 (&acc)[4], const i32x4 (&Pp)[4], int m) {
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        int t = __mul24(Pp[q][v], m) + acc[q][v];
        asm("" : "+v"(t));   // keeps each tile's multiply-add a v_mad_i32_i24 (no reassociation)
        acc[q][v] = t;
      }
  };
  i32x4 acc[4], Pp[4];
  int mp = 0;
  i32x4 av = a_frag(P[0]), cz = c_frag(P[0]);
  __builtin_amdgcn_sched_barrier(0);
  for (int n = 0; n < nrows; ++n) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      acc[q] = i32x4{0, 0, 0, 0};
      Pp[q] = i32x4{0, 0, 0, 0};
    }
    mp = 0;
    for (int k = 0; k < KP; k += RING) {
#pragma unroll
      for (int sl = 0; sl < RING; ++sl) {
        const int m = uniform(P[sl].cm.y);
        i32x4 Pn[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) Pn[q] = mfma_i8_k64(av, tunpack(P[sl].wd[q]), cz);
        madd(acc, Pp, mp);
#pragma unroll
        for (int q = 0; q < 4; ++q) Pp[q] = Pn[q];
        mp = m;
        fetch(P[sl]);
        meta(P[sl]);
        av = a_frag(P[(sl + 1) % RING]);   // the next slot in ring order
        cz = c_frag(P[(sl + 1) % RING]);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    madd(acc, Pp, mp);
    // epilogue of down row rm: y = f32(f32(acc) * 2^-e) * sh (+ residual) -> bf16
    const int rm = grp + a.G * (w + NW * n);
    const float fd = rtab[rm];
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int64_t t = t0 + 4 * g + v;
      if (t >= a.N) continue;
      const float shv = s_sh[4 * g + v];
      const int64_t off = t * a.d_model + (int64_t)rm * 64 + 4 * i;
      if (a.acc_d) *reinterpret_cast<i32x4*>(a.acc_d + off) = i32x4{acc[0][v], acc[1][v], acc[2][v], acc[3][v]};
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
size_t tprep_bytes(int64_t ntiles, int R, int which) {
  // tiles (+ zero tile) | m per tile | row multipliers, each 256-aligned
  auto al = [](size_t v) { return (v + 255) & ~(size_t)255; };
  return al((size_t)(ntiles + 1) * tprep_tile_bytes(which)) + al((size_t)(ntiles + 1) * 4) + al((size_t)R * 4);
}

int launch_tprep(const TPrepWeight (&w)[3], void* const (&out)[3], const u32x4* (&tw)[3],
                 const int32_t* (&mval)[3], const float* (&rmul)[3], hipStream_t st, bool run) {
  auto al = [](size_t v) { return (v + 255) & ~(size_t)255; };
  TPrepJobs J{};
  int64_t blocks = 0;
  for (int t = 0; t < 3; ++t) {
    const int64_t nt = (int64_t)w[t].R * w[t].K;
    const size_t tiles = al((size_t)(nt + 1) * tprep_tile_bytes(t));
    char* p = static_cast<char*>(out[t]);
    TPrepJob& j = J.job[t];
    j.packed = w[t].packed; j.s = w[t].s; j.col = w[t].col;
    j.R = w[t].R; j.K = w[t].K; j.C = w[t].C;
    j.int8 = tprep_tile_bytes(t) == 4096;
    j.tw = reinterpret_cast<u32x4*>(p);
    j.mval = reinterpret_cast<int32_t*>(p + tiles);
    j.rmul = reinterpret_cast<float*>(p + tiles + al((size_t)(nt + 1) * 4));
    tw[t] = j.tw;
    mval[t] = j.mval;
    rmul[t] = j.rmul;
    J.first[t] = blocks;
    blocks += nt + 1;
  }
  if (blocks > 0x7fffffff) return -2;
  if (!run) return 0;
  hipLaunchKernelGGL(tprep_kernel, dim3((unsigned)blocks), dim3(64), 0, st, J);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

// LDS bytes of the two kernels (dynamic part; each also has <= 256 bytes of static LDS)
static size_t tgu_lds(int RH, int K) {
  return (size_t)64 * 2048 + (size_t)RH * K * 16 + (size_t)RH * 8 + (size_t)64 * 8;
}
static size_t tdn_lds(int d_ff, int R_m, int Kd) {
  return (size_t)16 * d_ff + (size_t)(d_ff / 64) * 16 * 4 + (size_t)R_m * Kd * 8 + (size_t)R_m * 4;
}

bool tsplit_supported(int B, int d_model, int R_ff, int R_m, int Kg, int Ku, int Kd) {
  if (B != 64) return false;
  if (Kg != Ku || Kg < 1 || Kd < 1) return false;
  if (d_model % 256 || d_model > 2048) return false;   // int8 x panel rows of 2048 bytes
  const int64_t d_ff = (int64_t)R_ff * 64;
  if (d_ff % 256 || d_ff > 10240) return false;         // int8 h panel of 16 rows
  if (tgu_lds(R_ff, Kg) + 256 > 163840) return false;   // one slice (N >= 16384) holds every row
  if (tdn_lds((int)d_ff, R_m, Kd) + 256 > 163840) return false;
  return true;
}

// row slices per 64-token block: about 256 workgroups in all, at least 8 rows (one per wave) per
// slice
int tgu_slices(int64_t N, int R_ff) {
  const int64_t blocks = (N + 63) / 64;
  if (blocks >= 256) return 1;
  const int hmax = R_ff / 8 > 1 ? R_ff / 8 : 1;
  const int H = (int)((256 + blocks - 1) / blocks);
  return H < hmax ? H : hmax;
}

int launch_tgu(const TGUArgs& a, hipStream_t st) {
  if (a.N == 0) return 0;
  auto kern = tgu_kernel<4>;
  static std::atomic<uint64_t> configured{0};
  if (set_lds_limit_once((const void*)kern, 163840 - 256, configured)) return -1;
  const size_t lds = tgu_lds((a.R_ff + a.H - 1) / a.H, a.K);
  const int64_t blocks = (a.N + 63) / 64;
  hipLaunchKernelGGL(kern, dim3((unsigned)(blocks * a.H)), dim3(512), lds, st, a);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

// down kernel shape: TDN_WAVES waves (two down rows each at d_model 2048), a ring of TDN_RING
// tiles per wave, TDN_UB h rows per load batch of the panel fill.  Measured at d_model 2048,
// d_ff 8192, 8192 tokens (ternary forward from xq, kernel time): 16 waves, ring 4 142 us;
// 16 waves, ring 8 144 us; 8 waves (four rows each), ring 8 153 us.
constexpr int TDN_WAVES = 16, TDN_RING = 4, TDN_UB = 4;

int launch_tdn(const TDNArgs& a0, hipStream_t st) {
  if (a0.N == 0) return 0;
  auto kern = tdn_kernel<TDN_WAVES, TDN_RING, TDN_UB>;
  static std::atomic<uint64_t> configured{0};
  if (set_lds_limit_once((const void*)kern, 163840 - 256, configured)) return -1;
  const size_t lds = tdn_lds(a0.d_ff, a0.R_m, a0.Kd);
  // with fewer than 256 token blocks, the down rows are dealt to G row groups (each workgroup
  // quantises the block's h rows itself and runs every G-th row), at least 4 rows per group
  TDNArgs a = a0;
  const int64_t blocks = (a.N + 15) / 16;
  const int gmax = a.R_m / 4 > 1 ? a.R_m / 4 : 1;
  a.G = blocks >= 256 ? 1 : (int)std::min<int64_t>((256 + blocks - 1) / blocks, gmax);
  hipLaunchKernelGGL(kern, dim3((unsigned)(blocks * a.G)), dim3(64 * TDN_WAVES), lds, st, a);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace lbk
