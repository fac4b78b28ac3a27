// lbk_decode.hip — decode-shaped SwiGLU FFN (N <= 64 tokens, in one, two or four
// 16-token tiles), gfx950.
//
// With 16 tokens every weight byte feeds 16 MACs, so the forward is a stream of
// the weights through HBM: every CU should keep its share of the bytes in
// flight, with the loads of all of its tiles issued before any MFMA.  Two
// launches, with h (bf16) between them:
//
//   decode_gu_kernel  one workgroup per h row block r: waves 0-3 take the gate
//                     slots, waves 4-7 the up slots (at most 2 each), both tiles
//                     of a wave requested before its MFMAs (raw [B_in, B_out]
//                     tiles, transposed into MFMA fragments in registers); the
//                     partial sums meet in LDS and h = silu(g) * u is stored.
//   decode_dn_kernel  one workgroup per 16 output columns (16q .. 16q + 15) of a
//                     down row.  The B / 16 units of a row sit on one XCD
//                     (workgroups are dealt to the 8 XCDs round robin), so the
//                     lines of the row's tiles come from HBM once and each unit
//                     reads only its quarter of every line with 16-byte loads,
//                     transposed into B fragments through LDS; waves take the
//                     slots k = w, w + 8, ..., and the 8 partial sums meet in LDS
//                     in fixed order before the residual is added.  No
//                     cross-workgroup reduction: the result is deterministic.
//
// A single launch that hands h from the first phase to the second inside the
// kernel was measured slower on this part: a value written by one XCD becomes
// visible to device-coherent loads on another only after several microseconds,
// more than the ~2.5 us between two launches, whose boundary also makes h
// visible to plain loads.  With no per-call state in the workspace, both kernels
// can be captured into a graph.
#include "lbk_device.h"
#include "lbk_internal.h"

namespace lbk {

namespace {

constexpr int DEC_DS_MAX = 4;   // down slots per wave: Kd <= 8 * DEC_DS_MAX

template <int B>
__device__ __forceinline__ void mfma_tile(const u32x4 (&a)[TileShape<B>::NKS], const WRaw<B>& wt,
                                          f32x4 (&acc)[TileShape<B>::CW]) {
  constexpr int NKS = TileShape<B>::NKS, CW = TileShape<B>::CW;
  u32x4 f[NKS][CW];
  wraw_to_frag<B>(wt, f);
#pragma unroll
  for (int ks = 0; ks < NKS; ++ks)
#pragma unroll
    for (int m = 0; m < CW; ++m) acc[m] = mfma_bf16(a[ks], f[ks][m], acc[m]);
}

// A fragments of rows of an activation matrix (rows >= N are zero; row 0 is always readable)
template <int B>
__device__ __forceinline__ void load_a_rows(const uint16_t* base, int64_t ld, int N, int i, int g,
                                            u32x4 (&a)[TileShape<B>::NKS]) {
#pragma unroll
  for (int ks = 0; ks < TileShape<B>::NKS; ++ks) {
    const u32x4 v = load_afrag<B>(base + (int64_t)(i < N ? i : 0) * ld, ks, g);   // unconditional load
    a[ks] = (i < N) ? v : u32x4{0, 0, 0, 0};
  }
}

}  // namespace

// ---------------------------------------------------------------------------
// down-tile prefetch share of a gate/up workgroup
// ---------------------------------------------------------------------------
// The down kernel's workgroups for down row rm run on XCD rm % 8 (see decode_dn_kernel).
// The gate/up launch has 8 * S workgroups, S on each XCD (workgroup b on XCD b % 8); those
// of XCD x read the tiles of the down rows rm = x (mod 8) once, so that the down kernel
// finds them in the memory-side cache (and in the XCD's L2 where it is kept), and the
// down weights stream from HBM while the gate/up phase runs.  Work is balanced in tiles:
// a workgroup with a gate/up row (Kg + Ku tiles) takes fewer down tiles than one without.
// Returns the XOR of what was read (consumed by the caller so the loads stay).
template <int B, int PF>
__device__ __forceinline__ uint32_t prefetch_down_share(const DecodeArgs& a, int b, int S, int tid) {
  constexpr int CPT = B * B / 8;          // 16-byte chunks per tile
  constexpr int TPR = 512 / CPT;          // tiles covered by one 512-thread round
  const int x = b & 7, s = b >> 3;
  const int n_gu = a.R_ff > x ? min(S, (a.R_ff - x + 7) / 8) : 0;
  const int rows_x = a.R_m > x ? (a.R_m - x + 7) / 8 : 0;
  const int D = rows_x * a.Kd;                                  // down tiles read on this XCD
  const int gu_t = a.Kg + a.Ku;
  const int T = (n_gu * gu_t + D + S - 1) / S;                 // tiles per workgroup
  const int cg = T > gu_t ? T - gu_t : 0;                       // down share of a gate/up workgroup
  const int j0 = s < n_gu ? s * cg : n_gu * cg + (s - n_gu) * T;
  const int j1 = min(D, j0 + (s < n_gu ? cg : T));
  const bool any = j1 > j0;
  // the last workgroup of the XCD also reads the column indices of the XCD's down rows (first,
  // so that nothing waits for it behind the tiles)
  int cv = 0;
  if (s == S - 1 && tid < D) {
    const int rr = tid / a.Kd;
    cv = a.cd[(int64_t)(x + 8 * rr) * a.Kd + (tid - rr * a.Kd)];
  }
  // PF rounds, all requested before any is consumed and none under a branch (a share shorter
  // than PF re-reads its last tile, an empty one tile 0; a longer one is left to the down
  // kernel's own loads: this is only a prefetch)
  const int jt = tid / CPT, ch = tid % CPT;
  u32x4 v[PF];
  if constexpr (TPR == 1) {
    // one tile per round, a uniform walk over (row, slot) with no division inside
    int rr = any ? j0 / a.Kd : 0;
    int kk = any ? j0 - rr * a.Kd : 0;
#pragma unroll
    for (int u = 0; u < PF; ++u) {
      const int64_t e = any ? (int64_t)(x + 8 * rr) * a.Kd + kk : 0;
      v[u] = *reinterpret_cast<const u32x4*>(a.vd + e * B * B + 8 * ch);
      const bool adv = j0 + u + 1 < j1;
      const int kn = kk + 1 == a.Kd ? 0 : kk + 1;
      rr = adv && kn == 0 ? rr + 1 : rr;
      kk = adv ? kn : kk;
    }
  } else {
#pragma unroll
    for (int u = 0; u < PF; ++u) {
      int j = j0 + TPR * u + jt;
      j = j < j1 ? j : j1 - 1;
      const int rr = any ? j / a.Kd : 0;
      const int64_t e = any ? (int64_t)(x + 8 * rr) * a.Kd + (j - rr * a.Kd) : 0;
      v[u] = *reinterpret_cast<const u32x4*>(a.vd + e * B * B + 8 * ch);
    }
  }
  uint32_t acc = (uint32_t)cv;
#pragma unroll
  for (int u = 0; u < PF; ++u) acc ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
  return acc;
}

// workgroups of the gate/up launch per XCD: at least one per CU, a multiple of the 8 XCDs
__host__ __device__ inline int decode_gu_per_xcd(int R_ff) { return ((R_ff > 256 ? R_ff : 256) + 7) / 8; }

// ---------------------------------------------------------------------------
// gate/up: h row block r = blockIdx.x (workgroups r >= R_ff only prefetch)
// ---------------------------------------------------------------------------
template <int B, int MT>
__global__ __launch_bounds__(512, 1) void decode_gu_kernel(DecodeArgs a) {
  constexpr int CW = TileShape<B>::CW;
  constexpr int NKS = TileShape<B>::NKS;
  __shared__ f32x4 red[8][CW][64];   // one 16-token tile at a time
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = uniform(tid >> 6);
  const int i = lane & 15, g = lane >> 4;
  const int r = (int)blockIdx.x;
  if (r >= a.R_ff) {
    const uint32_t pf = prefetch_down_share<B, 16>(a, r, decode_gu_per_xcd(a.R_ff), tid);
    if (pf == 0x9e3779b9u && a.N < 0) a.h[0] = 0;               // never true: keeps the loads
    return;
  }
  const int C_in = a.d_model / B;
  const int64_t d_ff = (int64_t)a.R_ff * B;
  // waves 0-3: gate slots k = (w & 3) + 4j, waves 4-7: up slots, j < 2.  The same loads in
  // every wave (an unused slot reads the row's first tile): no load under a branch.
  const bool gate_wave = w < 4;
  const int Km = gate_wave ? a.Kg : a.Ku;
  const uint16_t* vm = gate_wave ? a.vg : a.vu;
  const int32_t* cm = gate_wave ? a.cg : a.cu;
  const int k0 = w & 3, k1 = k0 + 4;
  const bool use0 = k0 < Km, use1 = k1 < Km;
  const int64_t e0 = (int64_t)r * Km + (use0 ? k0 : 0), e1 = (int64_t)r * Km + (use1 ? k1 : 0);
  // Request order (a wave's loads return in order): the two column indices (one vector
  // load), this workgroup's tiles (their addresses need no index), the x fragments the indices
  // select (issued once the indices are back), then its share of the down tiles, which nothing
  // waits for until the end, so the MFMAs, the reduction and the h stores run while it streams.
  const int cl = cm[lane == 1 ? e1 : e0];
  asm volatile("" ::: "memory");
  WRaw<B> t0, t1;
  u32x4 a0[MT][NKS], a1[MT][NKS];
  load_wraw<B>(vm + e0 * B * B, lane, t0);
  load_wraw<B>(vm + e1 * B * B, lane, t1);
  asm volatile("" ::: "memory");
  const int c0 = use0 ? __builtin_amdgcn_readlane(cl, 0) : -1, c1 = use1 ? __builtin_amdgcn_readlane(cl, 1) : -1;
  const bool ok0 = c0 >= 0 && c0 < C_in, ok1 = c1 >= 0 && c1 < C_in;
  // 16-token tile mt: rows 16 mt .. of x (a tile past N reads row 0 and zeroes it)
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int nt = a.N - 16 * mt;
    const uint16_t* xt = a.x + (nt > 0 ? (int64_t)16 * mt * a.d_model : 0);
    load_a_rows<B>(xt + (int64_t)(ok0 ? c0 : 0) * B, a.d_model, ok0 && nt > 0 ? nt : 0, i, g, a0[mt]);
    load_a_rows<B>(xt + (int64_t)(ok1 ? c1 : 0) * B, a.d_model, ok1 && nt > 0 ? nt : 0, i, g, a1[mt]);
  }
  asm volatile("" ::: "memory");
  const uint32_t pf = prefetch_down_share<B, 4>(a, r, decode_gu_per_xcd(a.R_ff), tid);
  asm volatile("" ::: "memory");
  f32x4 acc[MT][CW];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int m = 0; m < CW; ++m) acc[mt][m] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    if (use0) mfma_tile<B>(a0[mt], t0, acc[mt]);
    if (use1) mfma_tile<B>(a1[mt], t1, acc[mt]);
  }
  // the eight waves' sums meet in LDS, one 16-token tile at a time
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    if (mt > 0) __syncthreads();   // the previous tile's sums have been read
#pragma unroll
    for (int m = 0; m < CW; ++m) red[w][m][lane] = acc[mt][m];
    __syncthreads();
    if (tid < 64 * CW) {
      const int m = tid >> 6, l = tid & 63;
      f32x4 gs = red[0][m][l], us = red[4][m][l];
#pragma unroll
      for (int ww = 1; ww < 4; ++ww) {
        gs += red[ww][m][l];
        us += red[4 + ww][m][l];
      }
      const int col = r * B + CW * (l & 15) + m;
      const float bgc = a.bg ? a.bg[col] : 0.f, buc = a.bu ? a.bu[col] : 0.f;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int tk = 16 * mt + 4 * (l >> 4) + v;
        if (tk < a.N) a.h[(int64_t)tk * d_ff + col] = f2bf(silu_f(gs[v] + bgc) * (us[v] + buc));
      }
    }
  }
  if (pf == 0x9e3779b9u && a.N < 0) a.h[0] = 0;                 // never true: keeps the loads
}

// ---------------------------------------------------------------------------
// down: output columns 16q .. 16q + 15 of down row rm; the B / 16 units of a row
// are workgroups 8 * (B / 16 * (rm / 8) + q) + rm % 8
// ---------------------------------------------------------------------------
template <int B, int DEC_DS, int MT>
__global__ __launch_bounds__(512, 1) void decode_dn_kernel(DecodeArgs a) {
  constexpr int CW = TileShape<B>::CW;   // = B / 16
  constexpr int NKS = TileShape<B>::NKS;
  __shared__ f32x4 red[8][MT][64];
  __shared__ __attribute__((aligned(16))) uint16_t xs[8][32 * 16];   // per-wave transpose buffer
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = uniform(tid >> 6);
  const int i = lane & 15, g = lane >> 4;
  const int b = (int)blockIdx.x;
  const int xc = b & 7, tq = b >> 3;
  const int q = tq % CW, rm = 8 * (tq / CW) + xc;
  if (rm >= a.R_m) return;
  const int64_t d_ff = (int64_t)a.R_ff * B;
  // Lane l reads row 32 ks + l / 2, columns 16q + 8 (l & 1) .. + 7 of each of its tiles; the
  // same loads in every wave (an unused slot reads the row's first tile).
  const int drow = lane >> 1;
  u32x4 dq[DEC_DS][NKS], av[DEC_DS][MT][NKS];
  int dc[DEC_DS];
  // Request order (a wave's loads return in order): the column indices (one vector load, lane
  // j holding slot w + 8j's), the tiles, whose addresses need no index, then the h fragments
  // the indices select, issued as soon as the indices are back.
  const int kl = w + 8 * (lane < DEC_DS ? lane : 0);
  const int cl = a.cd[(int64_t)rm * a.Kd + (kl < a.Kd ? kl : 0)];
  asm volatile("" ::: "memory");
#pragma unroll
  for (int j = 0; j < DEC_DS; ++j) {
    const int k = w + 8 * j;
    const int64_t e = (int64_t)rm * a.Kd + (k < a.Kd ? k : 0);
    const uint16_t* tile = a.vd + e * B * B + 16 * q + 8 * (lane & 1);
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) {
      const int row = 32 * ks + drow;
      dq[j][ks] = *reinterpret_cast<const u32x4*>(tile + (int64_t)(row < B ? row : 0) * B);
    }
  }
  asm volatile("" ::: "memory");
#pragma unroll
  for (int j = 0; j < DEC_DS; ++j) {
    const int c = (w + 8 * j < a.Kd) ? __builtin_amdgcn_readlane(cl, j) : -1;
    dc[j] = (c >= 0 && c < a.R_ff) ? c : -1;
    // 16-token tile mt: rows 16 mt .. of h (a tile past N reads row 0 and zeroes it)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int nt = a.N - 16 * mt;
      const uint16_t* ht = a.h + (nt > 0 ? (int64_t)16 * mt * d_ff : 0);
      load_a_rows<B>(ht + (int64_t)(dc[j] >= 0 ? dc[j] : 0) * B, d_ff, dc[j] >= 0 && nt > 0 ? nt : 0, i, g,
                     av[j][mt]);
    }
  }
  // each (tile, k-step) of 32 rows x 16 columns goes through this wave's LDS buffer to become
  // the B fragment of lane (n, g): rows 8g .. 8g + 7 of column n
  f32x4 acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
  uint16_t* xw = xs[w];
#pragma unroll
  for (int j = 0; j < DEC_DS; ++j) {
    if (dc[j] < 0) continue;
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) {
      *reinterpret_cast<u32x4*>(xw + drow * 16 + 8 * (lane & 1)) = dq[j][ks];
      // rows 8g .. 8g + 7 of column n = lane & 15, by two transposing 64-bit reads
      const u32x4 f = tr_frag(xw, 16, 0, 0, lane);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) acc[mt] = mfma_bf16(av[j][mt][ks], f, acc[mt]);
    }
  }
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) red[w][mt][lane] = acc[mt];
  __syncthreads();
  if (tid < 64 * MT) {
    const int mt = tid >> 6, l = tid & 63;
    f32x4 ps = red[0][mt][l];
#pragma unroll
    for (int ww = 1; ww < 8; ++ww) ps += red[ww][mt][l];
    const int col = rm * B + 16 * q + (l & 15);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int tk = 16 * mt + 4 * (l >> 4) + v;
      if (tk < a.N) {
        const int64_t idx = (int64_t)tk * a.d_model + col;
        float o = ps[v] + (a.bd ? a.bd[col] : 0.f);
        if (a.state) {
          o += a.state[idx];
          a.state[idx] = o;
          if (a.out) a.out[idx] = f2bf(o);
        } else {
          if (a.resid) o += bf2f(a.resid[idx]);
          a.out[idx] = f2bf(o);
        }
      }
    }
  }
}

// Whether the decode kernels take this shape: at most 8 gate and 8 up slots per h
// row, 1 .. 8 * DEC_DS_MAX down slots (empty slot lists excluded: unused slots read
// each weight's first tile).
bool decode_supported(int Kg, int Ku, int Kd) {
  return Kg >= 1 && Ku >= 1 && Kd >= 1 && Kg <= 8 && Ku <= 8 && Kd <= 8 * DEC_DS_MAX;
}

int launch_decode(int B, const DecodeArgs& a, hipStream_t st) {
  if (a.N == 0) return 0;
  if (!decode_supported(a.Kg, a.Ku, a.Kd) || a.R_ff <= 0 || a.R_m <= 0) return -2;
  const unsigned g1 = 8u * (unsigned)decode_gu_per_xcd(a.R_ff);
  const unsigned g2 = 8u * (unsigned)(B / 16) * (unsigned)((a.R_m + 7) / 8);
  // three down slots per wave up to Kd = 24, four beyond (a fourth slot of dead loads costs
  // the shorter lists time); one, two or four 16-token tiles
  const bool ds4 = a.Kd > 24;
  const int mt = a.N <= 16 ? 1 : (a.N <= 32 ? 2 : 4);
#define LBK_DEC_MT(BB, MM)                                                                           \
  if (mt == MM) {                                                                                    \
    hipLaunchKernelGGL((decode_gu_kernel<BB, MM>), dim3(g1), dim3(512), 0, st, a);                   \
    if (ds4) hipLaunchKernelGGL((decode_dn_kernel<BB, 4, MM>), dim3(g2), dim3(512), 0, st, a);       \
    else hipLaunchKernelGGL((decode_dn_kernel<BB, 3, MM>), dim3(g2), dim3(512), 0, st, a);           \
  }
#define LBK_DEC(BB)                                                                                  \
  case BB:                                                                                           \
    LBK_DEC_MT(BB, 1) LBK_DEC_MT(BB, 2) LBK_DEC_MT(BB, 4)                                            \
    break;
  switch (B) {
    LBK_DEC(16)
    LBK_DEC(32)
    LBK_DEC(64)
    default: return -2;
  }
#undef LBK_DEC
#undef LBK_DEC_MT
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace lbk
