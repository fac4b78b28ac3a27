// lbk_bwd.hip — backward of the Block-ELL SwiGLU FFN (gfx950, bf16 MFMA).
//
// With g = W_gate x, u = W_up x, h = silu(g) * u and out = W_down h (+ x), the
// gradients for an output gradient dy are
//   dh = dy W_down                    (transposed block-sparse product)
//   dg = dh * u * silu'(g), du = dh * silu(g)
//   dx = dg W_gate + du W_up (+ dy)
//   dW[r,k] = X[:, col(r,k)]^T G[:, r]  per tile, (X, G) = (x, dg), (x, du), (h, dy).
//
//   tlist_kernel   transposed topology: for every input column block c the slots
//                  (r, k) with col[r,k] = c, in ascending r*K + k (ballot
//                  compaction, deterministic), for gate, up and down in one launch.
//   tprod_kernel   (the general case; the two kernels after it cover the common shapes)
//                  out[:, c] = sum over the slots of column block c of
//                  A[:, r] W[r,k]^T.  A workgroup owns 64 tokens and four column
//                  blocks, one per wave (each tile is read once per workgroup);
//                  the raw [B_in, B_out] tile is the MFMA's A operand (row
//                  d of the tile holds the 8 consecutive B_out values a lane
//                  needs), the activation rows the B operand, so each lane ends
//                  with 4 consecutive output columns of one token; two list
//                  entries are in flight at a time.  Epilogue:
//                  the SiLU*mul backward (dh -> dg, du) or the optional + dy (-> dx).
//   dh_panel_kernel  dh -> dg, du when d_model <= 2048: the dy rows of 64 (32)
//                  tokens sit in LDS as the forward's XOR-swizzled panel and each
//                  of NW waves (8; 16 at B = 16) streams the list entries of its
//                  column blocks (c = w, w + NW, ...): tile rows from global memory,
//                  dy fragments from the panel.
//   dx_stage_kernel  dx when the output blocks fit the waves' accumulators (16
//                  waves where they fit 128 VGPRs, else 8): the dg and du columns
//                  of 64 tokens pass through LDS 512 at a time, and a cursor per
//                  output block walks its sorted list, whose first 64 entries
//                  stay in a register.
//   dxf_kernel     dx at B = 32: the same stages, one output block per wave and a
//                  4-slot ring of tiles over the wave's whole list (both sources,
//                  all stages), the list entries read one pass ahead.
//   dwg_kernel     tile gradients of a weight with narrow input rows (gate / up,
//                  d_model <= 1024, B = 32, K <= 8): a workgroup owns 8 block rows
//                  and stages the whole x row slice once per 32 tokens for their
//                  64 tiles (taken when it fills the CUs, 256 workgroups).
//   dwt_kernel     the same with the roles exchanged for a weight with narrow output
//                  rows (down, d_model <= 1024, B = 32): a workgroup owns 8 input
//                  column blocks, stages the whole dy row slice, and its waves walk
//                  the pooled transposed lists of the 8 blocks.
//   dw_kernel      tile gradients: a workgroup owns one block row, up to 8 of
//                  its slots (one per wave) and a chunk of tokens; token slices
//                  of X and G are staged row-major in LDS and read back
//                  transposed with ds_read_b64_tr_b16 (the token index is the
//                  MFMA's k); every wave accumulates its tile in fp32 and the
//                  chunk's partial tile goes to the workspace.
//   dw_reduce_kernel  sums the chunks' partials in fixed order -> bf16 (dead slots 0).
// No atomics anywhere: every sum has a fixed order, so the results are deterministic.
#include "lbk_device.h"
#include "lbk_internal.h"

namespace lbk {

// ---------------------------------------------------------------------------
// transposed topology
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void tlist_kernel(TListJobs jobs) {
  int jt = 0;
#pragma unroll
  for (int u = 1; u < TListJobs::kMax; ++u)
    if (u < jobs.n && (int64_t)blockIdx.x >= jobs.first[u]) jt = u;
  const TListJob& J = jobs.job[jt];
  const int c = (int)((int64_t)blockIdx.x - jobs.first[jt]);
  const int RK = J.R * J.K;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  __shared__ int wsum[4];
  int base = 0;
  for (int e0 = 0; e0 < RK; e0 += 256) {
    const int e = e0 + tid;
    const bool hit = e < RK && J.col[e] == c;   // c < C: dead slots never match
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
    if (hit) J.list[(int64_t)c * RK + off + rank] = e;
    base += tot;
    __syncthreads();
  }
  if (tid == 0) J.cnt[c] = base;
}

int launch_tlist(const TListJob* jobs, int n, hipStream_t st) {
  if (n < 1 || n > TListJobs::kMax) return -2;
  TListJobs J{};
  J.n = n;
  int64_t blocks = 0;
  for (int t = 0; t < n; ++t) {
    J.job[t] = jobs[t];
    J.first[t] = blocks;
    blocks += jobs[t].C;
  }
  if (blocks == 0) return 0;
  hipLaunchKernelGGL(tlist_kernel, dim3((unsigned)blocks), dim3(256), 0, st, J);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

// ---------------------------------------------------------------------------
// transposed block-sparse product
// ---------------------------------------------------------------------------
__device__ __forceinline__ u32x4 ld16(const uint16_t* p) { return *reinterpret_cast<const u32x4*>(p); }

// Tile row that operand lane i loads for 16-row group m (CW = B / 16 groups).  With CW >= 2 the
// groups interleave in fours, d = 32 (m / 2) + 8 (i / 4) + 4 (m % 2) + i % 4, so that the
// accumulator lane (n, g) ends with the 8 consecutive output columns 32 p + 8 g .. + 7 of groups
// m = 2p, 2p + 1 (16-byte epilogue loads and stores); with CW = 1 (B = 16) d = i.
template <int CW>
__device__ __forceinline__ int op_row(int i, int m) {
  if constexpr (CW == 1) return i;
  else return 32 * (m >> 1) + 8 * (i >> 2) + 4 * (m & 1) + (i & 3);
}

// epilogue of one token row: the lane's accumulator values v8 (8 consecutive columns starting at
// col, or 4 for B = 16): SiLU*mul backward (MODE 0) or + residual (MODE 1)
template <int MODE, int NV>
__device__ __forceinline__ void tprod_epilogue(const TProdArgs& a, int64_t off, const float (&v)[NV]) {
  if constexpr (MODE == 0) {
    float gv[NV], uv[NV], dgv[NV], duv[NV];
    load_bf16x<NV>(a.g + off, gv);
    load_bf16x<NV>(a.u + off, uv);
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const float sg = __builtin_amdgcn_rcpf(1.0f + __expf(-gv[j]));   // sigmoid(g)
      dgv[j] = v[j] * uv[j] * (sg + gv[j] * sg * (1.0f - sg));
      duv[j] = v[j] * gv[j] * sg;
    }
    store_bf16x<NV>(a.dg + off, dgv);
    store_bf16x<NV>(a.du + off, duv);
  } else {
    float rv[NV], o[NV];
#pragma unroll
    for (int j = 0; j < NV; ++j) rv[j] = 0.f;
    if (a.resid) load_bf16x<NV>(a.resid + off, rv);
#pragma unroll
    for (int j = 0; j < NV; ++j) o[j] = v[j] + rv[j];
    store_bf16x<NV>(a.out + off, o);
  }
}

// lane (i, g) of acc[m] (one 16-token group): columns of output block c of token tn
template <int MODE, int CW>
__device__ __forceinline__ void tprod_store(const TProdArgs& a, int64_t tn, int c, int g, const f32x4 (&acc)[CW]) {
  constexpr int B = 16 * CW;
  if constexpr (CW == 1) {
    float v[4] = {acc[0][0], acc[0][1], acc[0][2], acc[0][3]};
    tprod_epilogue<MODE, 4>(a, tn * a.ldo + (int64_t)c * B + 4 * g, v);
  } else {
#pragma unroll
    for (int p = 0; p < CW / 2; ++p) {
      float v[8];
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int u = 0; u < 4; ++u) v[4 * h + u] = acc[2 * p + h][u];
      tprod_epilogue<MODE, 8>(a, tn * a.ldo + (int64_t)c * B + 32 * p + 8 * g, v);
    }
  }
}

template <int B, int MODE>
__global__ __launch_bounds__(256) void tprod_kernel(TProdArgs a) {
  constexpr int CW = B / 16;                 // 16-column groups of a tile
  constexpr int NKS = B >= 32 ? B / 32 : 1;  // 32-deep k-steps
  constexpr int TQ = 4;                      // 16-token groups of the workgroup's 64 tokens
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = uniform(tid >> 6);
  const int i = lane & 15, g = lane >> 4;
  const int c = (int)blockIdx.y * 4 + w;     // this wave's output column block
  if (c >= a.C) return;                      // no barrier in this kernel
  const int64_t t0 = (int64_t)blockIdx.x * 64;
  // B = 16: a tile row has 16 values, so lanes g >= 2 (k 16..31) read lane g - 2's bytes and
  // carry zeros in the activation operand
  const int gk = (B == 16) ? (g & 1) : g;
  const bool kz = (B == 16) && g >= 2;
  int64_t trow[TQ];                          // clamped token rows of the lane's B fragments
#pragma unroll
  for (int q = 0; q < TQ; ++q) {
    const int64_t t = t0 + 16 * q + i;
    trow[q] = t < a.N ? t : a.N - 1;
  }
  f32x4 acc[TQ][CW];
#pragma unroll
  for (int q = 0; q < TQ; ++q)
#pragma unroll
    for (int m = 0; m < CW; ++m) acc[q][m] = f32x4{0.f, 0.f, 0.f, 0.f};

  // operands of one list entry: activation fragments of the 64 tokens (B operand) and the
  // tile rows (A operand)
  struct Ent {
    u32x4 bv[NKS][TQ], av[NKS][CW];
  };
  for (int s = 0; s < a.nsrc; ++s) {
    const TProdSrc S = a.src[s];
    const int cnt = S.cnt[c];
    const int32_t* L = S.list + (int64_t)c * S.cap;
    auto load = [&](int e, Ent& E) {
      const int r = e / S.K;
      const uint16_t* tile = S.w + (int64_t)e * B * B + 8 * gk;
      const uint16_t* acol = S.a + (int64_t)r * B + 8 * gk;
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) {
#pragma unroll
        for (int m = 0; m < CW; ++m) E.av[ks][m] = ld16(tile + op_row<CW>(i, m) * B + 32 * ks);
#pragma unroll
        for (int q = 0; q < TQ; ++q) E.bv[ks][q] = ld16(acol + trow[q] * S.lda + 32 * ks);
      }
    };
    auto compute = [&](const Ent& E) {
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks)
#pragma unroll
        for (int q = 0; q < TQ; ++q) {
          const u32x4 bv = kz ? u32x4{0, 0, 0, 0} : E.bv[ks][q];
#pragma unroll
          for (int m = 0; m < CW; ++m) acc[q][m] = mfma_bf16(E.av[ks][m], bv, acc[q][m]);
        }
    };
    for (int j0 = 0; j0 < cnt; j0 += 64) {
      const int lv = (j0 + lane < cnt) ? L[j0 + lane] : 0;   // 64 entries, one per lane
      const int jn = (cnt - j0) < 64 ? (cnt - j0) : 64;
      // two entries in flight: every load goes out (entries past the end re-read the last one)
      auto ent = [&](int jj) { return __builtin_amdgcn_readlane(lv, jj < jn ? jj : jn - 1); };
      Ent E0, E1;
      load(ent(0), E0);
      for (int jj = 0; jj < jn; jj += 2) {
        load(ent(jj + 1), E1);
        compute(E0);
        load(ent(jj + 2), E0);
        if (jj + 1 < jn) compute(E1);
      }
    }
  }

  // lane (i, g) of acc[q] holds token t0 + 16q + i (columns as op_row arranges them)
#pragma unroll
  for (int q = 0; q < TQ; ++q) {
    const int64_t tn = t0 + 16 * q + i;
    if (tn < a.N) tprod_store<MODE, CW>(a, tn, c, g, acc[q]);
  }
}

// ---------------------------------------------------------------------------
// dh = dy W_down -> dg, du with the dy rows of the workgroup's tokens in LDS
// ---------------------------------------------------------------------------
// The panel layout of the forward's gate/up kernel: token row 16*q + n of the 16*MT rows sits at
// row slot n*MT + q, and its 16-byte chunk c at chunk c ^ n.
template <int MT>
__device__ __forceinline__ uint32_t bpanel_addr(int row, int chunk, int rowb) {
  const int n = row & 15, q = row >> 4;
  return (uint32_t)((n * MT + q) * rowb + ((chunk ^ n) << 4));
}

// magic numbers of the division by each source's K (round-up method: s = ceil(log2 K); exact for
// dividends below 2^31): e / K = (umulhi(e, kmul) + e) >> ksh
static void set_kdiv(TProdArgs& a) {
  for (int s = 0; s < a.nsrc; ++s) {
    const uint64_t d = (uint64_t)(a.src[s].K > 0 ? a.src[s].K : 1);
    int sh = 0;
    while ((1ull << sh) < d) ++sh;
    a.src[s].kmul = (uint32_t)(((1ull << 32) * ((1ull << sh) - d)) / d + 1);
    a.src[s].ksh = sh;
  }
}
__device__ __forceinline__ int kdiv(const TProdSrc& S, int e) {
  return (int)((__umulhi((uint32_t)e, S.kmul) + (uint32_t)e) >> S.ksh);
}

template <int B, int MT, int NW>
__global__ __launch_bounds__(64 * NW, 1) void dh_panel_kernel(TProdArgs a) {
  constexpr int NT = 64 * NW;
  constexpr int CW = B / 16;
  constexpr int NKS = B >= 32 ? B / 32 : 1;
  constexpr int TM = 16 * MT;
  constexpr int ROWB = 8192 / MT;            // panel row stride: 2048 B (MT = 4) or 4096 B (MT = 2)
  extern __shared__ __attribute__((aligned(16))) unsigned char panel[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = uniform(tid >> 6);
  const int i = lane & 15, g = lane >> 4;
  // workgroup -> (token block, slice sl of nsl: column blocks sl + nsl (w + 8 j))
  const int sl = (int)(blockIdx.x % (unsigned)a.nsl);
  const int64_t t0 = (int64_t)(blockIdx.x / (unsigned)a.nsl) * TM;
  const TProdSrc S = a.src[0];
  const int d_model = (int)S.lda;

  // ---- panel: dy rows t0 .. t0 + TM - 1, every load at a clamped address
  {
    constexpr int CPR = ROWB / 16;
    constexpr int PIT = TM * CPR / NT;
    const int cpr = d_model / 8;
    u32x4 pv[PIT];
#pragma unroll
    for (int it = 0; it < PIT; ++it) {
      const int e = tid + NT * it;
      const int row = e / CPR, cc = e % CPR;
      const int64_t t = t0 + row;
      const bool ok = cc < cpr && t < a.N;
      pv[it] = ld16(S.a + (ok ? t : t0) * d_model + 8 * (ok ? cc : 0));
    }
#pragma unroll
    for (int it = 0; it < PIT; ++it) {
      const int e = tid + NT * it;
      const int row = e / CPR, cc = e % CPR;
      const bool ok = cc < cpr && t0 + row < a.N;
      if (cc < cpr) *reinterpret_cast<u32x4*>(panel + bpanel_addr<MT>(row, cc, ROWB)) = ok ? pv[it] : u32x4{0, 0, 0, 0};
    }
  }
  __syncthreads();

  const int gk = (B == 16) ? (g & 1) : g;
  const bool kz = (B == 16) && g >= 2;
  const uint32_t lbase = (uint32_t)(i * MT * ROWB);
  struct Ent {
    u32x4 av[NKS][CW];
    u32x2 a16;   // B = 16: the 16x16x16 fragment (tile row i, k = 4g .. 4g + 3)
    int r;
  };
  auto load = [&](int e, Ent& E) {
    if constexpr (B == 16) {
      E.a16 = *reinterpret_cast<const u32x2*>(S.w + (int64_t)e * B * B + i * B + 4 * g);
    } else {
      const uint16_t* tile = S.w + (int64_t)e * B * B + 8 * gk;
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks)
#pragma unroll
        for (int m = 0; m < CW; ++m) E.av[ks][m] = ld16(tile + op_row<CW>(i, m) * B + 32 * ks);
    }
    E.r = kdiv(S, e);
  };
  f32x4 acc[MT][CW];
  auto compute = [&](const Ent& E) {
    const int r = uniform(E.r);
    if constexpr (B == 16) {
      // dy[16q + i][16r + 4g ..]: 16-byte chunk 2r + g / 2 of the swizzled row, its half g & 1
      const uint32_t pa = lbase + ((uint32_t)(((r * 2 + (g >> 1)) ^ i) << 4) | (uint32_t)((g & 1) << 3));
#pragma unroll
      for (int q = 0; q < MT; ++q)
        acc[q][0] = mfma_bf16_k16(E.a16, *reinterpret_cast<const u32x2*>(panel + pa + q * ROWB), acc[q][0]);
      return;
    }
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) {
      const uint32_t pa = lbase + ((((r * (B / 8) + 4 * ks + gk)) ^ i) << 4);
#pragma unroll
      for (int q = 0; q < MT; ++q) {
        const u32x4 bv0 = *reinterpret_cast<const u32x4*>(panel + pa + q * ROWB);   // dy[16q + i][r*B + 32ks + 8g ..]
        const u32x4 bv = kz ? u32x4{0, 0, 0, 0} : bv0;
#pragma unroll
        for (int m = 0; m < CW; ++m) acc[q][m] = mfma_bf16(E.av[ks][m], bv, acc[q][m]);
      }
    }
  };

  // the gate pre-activation and up output at this lane's outputs, fetched before the entries
  // of a column block so that their latency overlaps its MFMAs (clamped rows, always loaded)
  constexpr int NV = CW == 1 ? 4 : 8, NP = CW == 1 ? 1 : CW / 2;
  typedef uint32_t raw_t __attribute__((ext_vector_type(NV / 2)));
  raw_t graw[MT][NP], uraw[MT][NP];
  auto col_of = [&](int c, int p) { return (int64_t)c * B + (CW == 1 ? 4 * g : 32 * p + 8 * g); };
  // a block's count and first 64 list entries are read one block ahead (the list read at a
  // clamped index, so it needs no count), so that a block issues its tile loads at once instead
  // of waiting for its list behind its g / u loads
  const int cstep = NW * a.nsl;
  const int clast = (int)(S.cap < 64 ? S.cap : 64) - 1;
  int cnt_n = 0, lv_n = 0;
  {
    const int cf = sl + a.nsl * w;
    if (cf < a.C) {
      cnt_n = S.cnt[cf];
      lv_n = S.list[(int64_t)cf * S.cap + (lane < clast ? lane : clast)];
    }
  }
  for (int c = sl + a.nsl * w; c < a.C; c += cstep) {
    const int cnt = cnt_n, lv0 = lv_n;
    if (c + cstep < a.C) {
      cnt_n = S.cnt[c + cstep];
      lv_n = S.list[(int64_t)(c + cstep) * S.cap + (lane < clast ? lane : clast)];
    }
#pragma unroll
    for (int q = 0; q < MT; ++q) {
      const int64_t tn = t0 + 16 * q + i;
      const int64_t row = (tn < a.N ? tn : a.N - 1) * a.ldo;
#pragma unroll
      for (int p = 0; p < NP; ++p) {
        graw[q][p] = *reinterpret_cast<const raw_t*>(a.g + row + col_of(c, p));
        uraw[q][p] = *reinterpret_cast<const raw_t*>(a.u + row + col_of(c, p));
      }
    }
#pragma unroll
    for (int q = 0; q < MT; ++q)
#pragma unroll
      for (int m = 0; m < CW; ++m) acc[q][m] = f32x4{0.f, 0.f, 0.f, 0.f};
    const int32_t* L = S.list + (int64_t)c * S.cap;
    for (int j0 = 0; j0 < cnt; j0 += 64) {
      // 64 entries, one per lane (the first 64 from the read ahead)
      const int lv = j0 == 0 ? lv0 : ((j0 + lane < cnt) ? L[j0 + lane] : 0);
      const int jn = (cnt - j0) < 64 ? (cnt - j0) : 64;
      auto ent = [&](int jj) { return __builtin_amdgcn_readlane(lv, jj < jn ? jj : jn - 1); };
      if constexpr (B == 16) {
        // slot pairs: ring position p holds entries 2p and 2p + 1, one 16x16x32 MFMA per token
        // tile.  Lanes g < 2 hold row i, columns 8 (g & 1) .. + 7 of entry 2p's tile, lanes
        // g >= 2 those of entry 2p + 1's (zeroed when the list ends at 2p + 1); the dy panel
        // fragment is the 16-byte chunk 2 r + (g & 1) of the lane's entry's row block r.  A
        // DHP-position ring as below (positions past the end reload the last entry)
        constexpr int DHP = 4;
        const int np = (jn + 1) >> 1;
        Ent E[DHP];
        auto loadp = [&](int p, Ent& E) {
          const int e1 = ent(2 * p), e2 = ent(2 * p + 1);
          const int e = g < 2 ? e1 : e2;
          E.av[0][0] = *reinterpret_cast<const u32x4*>(S.w + (int64_t)e * (B * B) + i * B + 8 * (g & 1));
          E.r = kdiv(S, e1) | (kdiv(S, e2) << 10) | (2 * p + 1 < jn ? 1 << 20 : 0);
        };
        auto computep = [&](const Ent& E) {
          const int rr = uniform(E.r);
          const int rl = g < 2 ? (rr & 1023) : ((rr >> 10) & 1023);
          const u32x4 av = (g < 2 || ((rr >> 20) & 1)) ? E.av[0][0] : u32x4{0, 0, 0, 0};
          const uint32_t pa = lbase + ((uint32_t)((rl * 2 + (g & 1)) ^ i) << 4);
#pragma unroll
          for (int q = 0; q < MT; ++q)
            acc[q][0] = mfma_bf16(av, *reinterpret_cast<const u32x4*>(panel + pa + q * ROWB), acc[q][0]);
        };
#pragma unroll
        for (int k = 0; k < DHP - 1; ++k) loadp(k, E[k]);
        for (int pp = 0; pp < np; pp += DHP) {
#pragma unroll
          for (int k = 0; k < DHP; ++k) {
            loadp(pp + k + DHP - 1, E[(k + DHP - 1) % DHP]);
            if (k == 0 || pp + k < np) computep(E[k]);
          }
        }
      } else {
        // a DHR-entry ring: DHR - 1 tile loads in flight ahead of the MFMAs (positions past the
        // end reload the last entry and are not computed)
        constexpr int DHR = B == 64 ? 2 : 6;
        Ent E[DHR];
#pragma unroll
        for (int k = 0; k < DHR - 1; ++k) load(ent(k), E[k]);
        for (int jj = 0; jj < jn; jj += DHR) {
#pragma unroll
          for (int k = 0; k < DHR; ++k) {
            load(ent(jj + k + DHR - 1), E[(k + DHR - 1) % DHR]);
            if (k == 0 || jj + k < jn) compute(E[k]);
          }
        }
      }
    }
    // epilogue: lane (i, g) of acc[q] holds dh of token t0 + 16q + i (columns as op_row
    // arranges them): dg = dh * u * silu'(g), du = dh * silu(g)
#pragma unroll
    for (int q = 0; q < MT; ++q) {
      const int64_t tn = t0 + 16 * q + i;
      if (tn >= a.N) continue;
#pragma unroll
      for (int p = 0; p < NP; ++p) {
        float dh[NV], dgv[NV], duv[NV];
#pragma unroll
        for (int j = 0; j < NV; ++j) dh[j] = acc[q][CW == 1 ? 0 : 2 * p + j / 4][j % 4];
#pragma unroll
        for (int j = 0; j < NV; ++j) {
          const uint32_t gw = graw[q][p][j / 2], uw = uraw[q][p][j / 2];
          const float gv = (j & 1) ? bf_hi(gw) : bf_lo(gw), uv = (j & 1) ? bf_hi(uw) : bf_lo(uw);
          const float sg = __builtin_amdgcn_rcpf(1.0f + __expf(-gv));   // sigmoid(g)
          dgv[j] = dh[j] * uv * (sg + gv * sg * (1.0f - sg));
          duv[j] = dh[j] * gv * sg;
        }
        store_bf16x<NV>(a.dg + tn * a.ldo + col_of(c, p), dgv);
        store_bf16x<NV>(a.du + tn * a.ldo + col_of(c, p), duv);
      }
    }
  }
}

// dh through the LDS panel when the dy rows of 16*MT tokens fit (d_model <= 2048, one source)
// With fewer token blocks than CUs, the column blocks are split over nsl workgroups per token
// block (about 256 workgroups, at least one column block per wave), each loading the dy panel.
template <int B, int MT, int NW>
static int launch_dh_panel_t(const TProdArgs& a0, hipStream_t st) {
  constexpr size_t lds = (size_t)16 * MT * (8192 / MT);
  auto kern = dh_panel_kernel<B, MT, NW>;
  if (hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                          (int)lds) != hipSuccess)
    return -1;
  TProdArgs a = a0;
  set_kdiv(a);
  const int64_t ntb = (a.N + 16 * MT - 1) / (16 * MT);
  const int smax = a.C / NW > 1 ? a.C / NW : 1;
  a.nsl = ntb >= 256 ? 1 : (int)std::min<int64_t>((256 + ntb - 1) / ntb, smax);
  hipLaunchKernelGGL(kern, dim3((unsigned)(ntb * a.nsl)), dim3(64 * NW), lds, st, a);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

static int launch_dh_panel(int B, const TProdArgs& a, hipStream_t st) {
  const int64_t d_model = a.src[0].lda;
  const int mt = d_model <= 1024 ? 4 : (d_model <= 2048 ? 2 : 0);
  if (mt == 0 || d_model % 8) return -2;
  // 16 waves at B = 16 (their registers fit 128 VGPRs): B = 16 backward at d_model 1024, d_ff 4096
  // 1.93 -> 1.87 ms; at B = 32 16 waves spill (0.739 against 0.715 ms)
  if (B == 16 && mt == 4) return launch_dh_panel_t<16, 4, 16>(a, st);
#define LBK_DH(BB, MM) if (B == BB && mt == MM) return launch_dh_panel_t<BB, MM, 8>(a, st);
  LBK_DH(16, 4) LBK_DH(16, 2) LBK_DH(32, 4) LBK_DH(32, 2) LBK_DH(64, 4) LBK_DH(64, 2)
#undef LBK_DH
  return -2;
}

// ---------------------------------------------------------------------------
// dx = dg W_gate + du W_up (+ dy) with the activations staged through LDS
// ---------------------------------------------------------------------------
// A workgroup owns 64 tokens and every output column block: wave w owns blocks c = w + 8 o
// (o < OPW).  The columns of dg, then du, pass through LDS 512 at a time (double buffered, the
// next stage's loads in flight during the current one, as in the forward's down kernel).  A
// block's list is sorted by slot, hence by the source column block r = e / K, so the entries of
// a stage are the next run of the list: a cursor per block walks it, 64 entries at a time held
// one per lane.
// activation columns per stage: 512 (longer runs of a block's list per stage), 256 for B = 64
// (its larger accumulators leave no registers for the bigger stage)
template <int B>
struct DxStage { static constexpr int COLS = B == 64 ? 256 : 512; };

template <int B, int OPW, int NW>
__global__ __launch_bounds__(64 * NW, 1) void dx_stage_kernel(TProdArgs a) {
  constexpr int NT = 64 * NW;
  constexpr int CW = B / 16;
  constexpr int NKS = B >= 32 ? B / 32 : 1;
  constexpr int MT = 4;
  constexpr int COLS = DxStage<B>::COLS;
  constexpr int G = COLS / B;                        // source column blocks per stage
  constexpr int SROWB = COLS * 2;                    // bytes per token row of a stage
  constexpr int SBYTES = 64 * SROWB;                 // 64 KB (32 KB for B = 64)
  constexpr int PER_T = SBYTES / 16 / NT;            // 16-byte chunks per thread per stage
  extern __shared__ __attribute__((aligned(16))) unsigned char stg[];   // two stages
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = uniform(tid >> 6);
  const int i = lane & 15, g = lane >> 4;
  // workgroup -> (64-token block, slice sl of nsl: output blocks sl + nsl (w + NW o))
  const int sl = (int)(blockIdx.x % (unsigned)a.nsl);
  const int64_t t0 = (int64_t)(blockIdx.x / (unsigned)a.nsl) * 64;
  const int gk = (B == 16) ? (g & 1) : g;
  const bool kz = (B == 16) && g >= 2;

  // stages: source s covers ceil(R_s / G) stages; global stage -> (source, first block)
  const int R0 = (int)(a.src[0].lda / B);
  const int ns0 = (R0 + G - 1) / G;
  const int ns1 = a.nsrc > 1 ? ((int)(a.src[1].lda / B) + G - 1) / G : 0;
  const int nstages = ns0 + ns1;

  u32x4 sreg[PER_T];
  auto stage_fetch = [&](int s) {
    const TProdSrc& S = a.src[s < ns0 ? 0 : 1];
    const int64_t col0 = (int64_t)(s < ns0 ? s : s - ns0) * COLS;
#pragma unroll
    for (int u = 0; u < PER_T; ++u) {
      const int e = tid + NT * u;
      const int row = e / (SROWB / 16), cc = e - row * (SROWB / 16);
      const int64_t t = t0 + row, col = col0 + 8 * cc;
      const bool ok = t < a.N && col < S.lda;
      const u32x4 v = ld16(S.a + (ok ? t : t0) * S.lda + (ok ? col : 0));
      sreg[u] = ok ? v : u32x4{0, 0, 0, 0};
    }
  };
  auto stage_store = [&](int buf) {
#pragma unroll
    for (int u = 0; u < PER_T; ++u) {
      const int e = tid + NT * u;
      const int row = e / (SROWB / 16), cc = e - row * (SROWB / 16);
      *reinterpret_cast<u32x4*>(stg + buf * SBYTES + bpanel_addr<MT>(row, cc, SROWB)) = sreg[u];
    }
  };

  f32x4 acc[OPW][MT][CW];
#pragma unroll
  for (int o = 0; o < OPW; ++o)
#pragma unroll
    for (int q = 0; q < MT; ++q)
#pragma unroll
      for (int m = 0; m < CW; ++m) acc[o][q][m] = f32x4{0.f, 0.f, 0.f, 0.f};

  struct Ent {
    u32x4 av[NKS][CW];
    u32x2 a16;                                       // B = 16: the 16x16x16 fragment
    int r;                                           // source column block
  };
  const uint32_t lbase = (uint32_t)(i * MT * SROWB);
  int cur[OPW];                                      // list cursors of the current source
  int lvr[OPW];                                      // first 64 list entries of each output block

  stage_fetch(0);
  stage_store(0);
  __syncthreads();
  for (int s = 0; s < nstages; ++s) {
    const int src = s < ns0 ? 0 : 1;
    const int st = s < ns0 ? s : s - ns0;
    const TProdSrc& S = a.src[src];
    if (st == 0) {
      // a new source: each output block's first 64 list entries into a register (lane j holds
      // entry j), so that a stage finds its run with a ballot instead of a global load
#pragma unroll
      for (int o = 0; o < OPW; ++o) {
        cur[o] = 0;
        const int c = sl + a.nsl * (w + NW * o);
        const int cnt = c < a.C ? S.cnt[c] : 0;
        lvr[o] = lane < cnt ? S.list[(int64_t)c * S.cap + lane] : 0x7fffffff;
      }
    }
    if (s + 1 < nstages) stage_fetch(s + 1);
    const unsigned char* sb = stg + (s & 1) * SBYTES;
    const int rlo = st * G, rhi = rlo + G;           // source column blocks of this stage
    auto load = [&](int e, Ent& E) {
      if constexpr (B == 16) {
        E.a16 = *reinterpret_cast<const u32x2*>(S.w + (int64_t)e * B * B + i * B + 4 * g);
      } else {
        const uint16_t* tile = S.w + (int64_t)e * B * B + 8 * gk;
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks)
#pragma unroll
          for (int m = 0; m < CW; ++m) E.av[ks][m] = ld16(tile + op_row<CW>(i, m) * B + 32 * ks);
      }
      E.r = e / S.K;
    };
#pragma unroll
    for (int o = 0; o < OPW; ++o) {
      const int c = sl + a.nsl * (w + NW * o);
      if (c >= a.C) continue;
      auto compute = [&](const Ent& E) {
        const int rb = uniform(E.r) - rlo;           // column block within the stage
        if constexpr (B == 16) {
          const uint32_t pa = lbase + ((uint32_t)(((rb * 2 + (g >> 1)) ^ i) << 4) | (uint32_t)((g & 1) << 3));
#pragma unroll
          for (int q = 0; q < MT; ++q)
            acc[o][q][0] = mfma_bf16_k16(E.a16, *reinterpret_cast<const u32x2*>(sb + pa + q * SROWB), acc[o][q][0]);
          return;
        }
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) {
          const uint32_t pa = lbase + (((rb * (B / 8) + 4 * ks + gk) ^ i) << 4);
#pragma unroll
          for (int q = 0; q < MT; ++q) {
            const u32x4 bv0 = *reinterpret_cast<const u32x4*>(sb + pa + q * SROWB);
            const u32x4 bv = kz ? u32x4{0, 0, 0, 0} : bv0;
#pragma unroll
            for (int m = 0; m < CW; ++m) acc[o][q][m] = mfma_bf16(E.av[ks][m], bv, acc[o][q][m]);
          }
        }
      };
      const int cnt = S.cnt[c];
      const int32_t* L = S.list + (int64_t)c * S.cap;
      int jc = cur[o];
      while (jc < cnt) {
        // entries of this stage: the run from jc whose source block is below rhi.  Within the
        // first 64 entries they come from the register (lanes jc .. jc + n - 1), beyond them
        // from the next 64 entries loaded here (lanes 0 .. n - 1)
        const bool inreg = jc < 64;
        const int lv = inreg ? lvr[o] : ((jc + lane < cnt) ? L[jc + lane] : 0x7fffffff);
        const int base = inreg ? jc : 0;
        const int lim = inreg ? (cnt < 64 ? cnt : 64) : cnt - jc;
        const uint64_t m = __ballot(lane >= base && lane < lim && lv / S.K < rhi);
        const int n = __builtin_popcountll(m);       // a contiguous run of lanes (sorted list)
        if (n == 0) break;
        auto ent = [&](int jj) { return __builtin_amdgcn_readlane(lv, base + (jj < n ? jj : n - 1)); };
        if constexpr (B == 16) {
          // 8-byte tile fragments: a 3-entry ring keeps two loads in flight ahead of the MFMAs
          // (positions past the run reload its last entry and are not computed)
          constexpr int DXR = 3;
          Ent E[DXR];
#pragma unroll
          for (int k = 0; k < DXR - 1; ++k) load(ent(k), E[k]);
          for (int jj = 0; jj < n; jj += DXR) {
#pragma unroll
            for (int k = 0; k < DXR; ++k) {
              load(ent(jj + k + DXR - 1), E[(k + DXR - 1) % DXR]);
              if (jj + k < n) compute(E[k]);
            }
          }
        } else {
          Ent E0, E1;
          load(ent(0), E0);
          for (int jj = 0; jj < n; jj += 2) {
            load(ent(jj + 1), E1);
            compute(E0);
            load(ent(jj + 2), E0);
            if (jj + 1 < n) compute(E1);
          }
        }
        jc += n;
        if (base + n < 64) break;                    // the run ended inside this chunk
      }
      cur[o] = jc;
    }
    if (s + 1 < nstages) stage_store((s + 1) & 1);
    __syncthreads();
  }

  // epilogue: dx = acc (+ dy)
#pragma unroll
  for (int o = 0; o < OPW; ++o) {
    const int c = sl + a.nsl * (w + NW * o);
    if (c >= a.C) continue;
#pragma unroll
    for (int q = 0; q < MT; ++q) {
      const int64_t tn = t0 + 16 * q + i;
      if (tn < a.N) tprod_store<1, CW>(a, tn, c, g, acc[o][q]);
    }
  }
}

template <int B, int OPW, int NW>
static int launch_dx_stage_t(const TProdArgs& a, hipStream_t st) {
  constexpr size_t lds = 2 * (size_t)64 * DxStage<B>::COLS * 2;
  auto kern = dx_stage_kernel<B, OPW, NW>;
  if (lds > 65536 && hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                         hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess)
    return -1;
  hipLaunchKernelGGL(kern, dim3((unsigned)((a.N + 63) / 64 * a.nsl)), dim3(64 * NW), lds, st, a);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

// dxf_kernel<B, D>: dx at B = 32 (and at B = 16 past the staged kernel's widths) with one output
// block per wave (16 waves; the output blocks are dealt to nsl workgroups per 64-token block,
// which share an XCD) and a D-slot ring of tiles that
// runs over the wave's whole list -- the sorted entries of source 0, then of source 1 -- across
// the 512-column stages of both sources, so D tile loads stay in flight where dx_stage_kernel
// had one.  A stage change is a workgroup barrier taken inline when the next entry lies in a
// later stage; every wave passes all of them.  The list entries a pass fetches are read one pass
// ahead (lane j of a window holds entry j of the pass), so no load waits on a list read.
constexpr int DXF_WAVES = 16;
constexpr int DXF_RING = 4;
template <int B, int D>
__global__ __launch_bounds__(64 * DXF_WAVES, 1) void dxf_kernel(TProdArgs a) {
  constexpr int NW = DXF_WAVES, NT = 64 * NW;
  constexpr int CW = B / 16, MT = 4;
  constexpr int COLS = DxStage<B>::COLS;
  constexpr int G = COLS / B;                        // source column blocks per stage
  constexpr int SROWB = COLS * 2;
  constexpr int SBYTES = 64 * SROWB;
  constexpr int PER_T = SBYTES / 16 / NT;
  // B = 32: one 32-deep k-step per tile; B = 16: the 16x16x16 form (8-byte fragments)
  static_assert(B == 32 || B == 16, "tile size");
  extern __shared__ __attribute__((aligned(16))) unsigned char stg[];   // two stages
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = uniform(tid >> 6);
  const int i = lane & 15, g = lane >> 4;
  // workgroup -> (64-token block tb, slice sl); the slices of a token block share an XCD
  int64_t tb = blockIdx.x;
  int sl = 0;
  if (a.nsl > 1) {
    const int64_t b = blockIdx.x, rest = b >> 3;
    sl = (int)(rest % a.nsl);
    tb = 8 * (rest / a.nsl) + (b & 7);
  }
  const int64_t t0 = tb * 64;
  if (t0 >= a.N) return;   // the whole workgroup, before any barrier
  const int c = sl + a.nsl * w;                      // this wave's output column block
  const bool has = c < a.C;
  const int cs_ = has ? c : 0;

  const int R0 = (int)(a.src[0].lda / B);
  const int ns0 = (R0 + G - 1) / G;
  const int ns1 = a.nsrc > 1 ? ((int)(a.src[1].lda / B) + G - 1) / G : 0;
  const int nstages = ns0 + ns1;
  const TProdSrc& S0 = a.src[0];
  const TProdSrc& S1 = a.src[a.nsrc > 1 ? 1 : 0];

  // stage loads: unconditional (clamped address), zeros selected at the LDS store
  u32x4 sreg[PER_T];
  int sok = 0;
  auto stage_fetch = [&](int s) {
    const TProdSrc& S = s < ns0 ? S0 : S1;
    const int64_t col0 = (int64_t)(s < ns0 ? s : s - ns0) * COLS;
    sok = 0;
#pragma unroll
    for (int u = 0; u < PER_T; ++u) {
      const int e = tid + NT * u;
      const int row = e / (SROWB / 16), cc = e - row * (SROWB / 16);
      const int64_t t = t0 + row, col = col0 + 8 * cc;
      const bool ok = t < a.N && col < S.lda;
      sok |= ok ? 1 << u : 0;
      sreg[u] = ld16(S.a + (ok ? t : t0) * S.lda + (ok ? col : 0));
    }
  };
  auto stage_store = [&](int buf) {
#pragma unroll
    for (int u = 0; u < PER_T; ++u) {
      const int e = tid + NT * u;
      const int row = e / (SROWB / 16), cc = e - row * (SROWB / 16);
      *reinterpret_cast<u32x4*>(stg + buf * SBYTES + bpanel_addr<MT>(row, cc, SROWB)) =
          (sok >> u) & 1 ? sreg[u] : u32x4{0, 0, 0, 0};
    }
  };

  // the wave's list: entries 0 .. n0 - 1 from source 0, then n1 from source 1
  const int n0 = has ? S0.cnt[cs_] : 0;
  const int n1 = has && a.nsrc > 1 ? S1.cnt[cs_] : 0;
  const int32_t* L0 = S0.list + (int64_t)cs_ * S0.cap;
  const int32_t* L1 = S1.list + (int64_t)cs_ * S1.cap;
  // entries base .. base + 2D - 1 in lanes 0 .. 2D - 1 (an unconditional load at a clamped
  // index; entries past the list are recognised by their index, not by the loaded value)
  auto window = [&](int base) {
    const int j = base + (lane < 2 * D ? lane : 0);
    const int32_t* p = j < n0 ? L0 + j : (j - n0 < n1 ? L1 + (j - n0) : L0);
    return *p;
  };

  struct Slot {
    u32x4 av[CW];
    u32x2 a16;   // B = 16: the 16x16x16 fragment (tile row i, k = 4g .. 4g + 3)
    int st;      // stage (-1: past the list)
    int cb;      // column block within the stage
  };
  // slot S <- entry j of the list (its value e read from the window)
  auto fetch = [&](Slot& S, int j, int e) {
    const bool live = j < n0 + n1;
    const bool s1 = j >= n0;
    // r = e / K by multiply and shift (a division by a run-time value is a long sequence)
    const int r = live ? kdiv(s1 ? S1 : S0, e) : 0;
    const int64_t tile = live ? e : 0;              // past the list: tile 0 of source 0, unused
    if constexpr (B == 16) {
      S.a16 = *reinterpret_cast<const u32x2*>((live && s1 ? S1.w : S0.w) + tile * B * B + i * B + 4 * g);
    } else {
      const uint16_t* tp = (live && s1 ? S1.w : S0.w) + tile * B * B + 8 * g;
#pragma unroll
      for (int m = 0; m < CW; ++m) S.av[m] = ld16(tp + op_row<CW>(i, m) * B);
    }
    S.st = live ? (s1 ? ns0 : 0) + r / G : -1;
    S.cb = r - (r / G) * G;
  };
  const uint32_t lbase = (uint32_t)(i * MT * SROWB);
  f32x4 acc[MT][CW];
#pragma unroll
  for (int q = 0; q < MT; ++q)
#pragma unroll
    for (int m = 0; m < CW; ++m) acc[q][m] = f32x4{0.f, 0.f, 0.f, 0.f};
  auto compute = [&](const Slot& S, const unsigned char* sb) {
    if constexpr (B == 16) {
      // rows 16q + i, k = 4g .. 4g + 3 of the block: 16-byte chunk 2 cb + g / 2, its half g & 1
      const uint32_t pa = lbase + ((uint32_t)(((S.cb * 2 + (g >> 1)) ^ i) << 4) | (uint32_t)((g & 1) << 3));
#pragma unroll
      for (int q = 0; q < MT; ++q)
        acc[q][0] = mfma_bf16_k16(S.a16, *reinterpret_cast<const u32x2*>(sb + pa + q * SROWB), acc[q][0]);
      return;
    }
    const uint32_t pa = lbase + (((S.cb * (B / 8) + g) ^ i) << 4);
#pragma unroll
    for (int q = 0; q < MT; ++q) {
      const u32x4 bv = *reinterpret_cast<const u32x4*>(sb + pa + q * SROWB);
#pragma unroll
      for (int m = 0; m < CW; ++m) acc[q][m] = mfma_bf16(S.av[m], bv, acc[q][m]);
    }
  };

  Slot R[D];
  // the ring's first entries, and those of the first pass in lanes D .. 2D - 1 of the same window
  // (read here, so the window register enters the loop with its load complete)
  int wcur = window(0);
#pragma unroll
  for (int s = 0; s < D; ++s) fetch(R[s], s, __builtin_amdgcn_readlane(wcur, s));
  int nxt = D;                                      // list index of the next entry to fetch
  int woff = D;                                     // lane of the pass's first entry in its window
  stage_fetch(0);
  stage_store(0);
  __syncthreads();
  if (nstages > 1) stage_fetch(1);
  int cs = 0;
  auto transition = [&]() {
    stage_store((cs + 1) & 1);
    __syncthreads();
    ++cs;
    if (cs + 1 < nstages) stage_fetch(cs + 1);
  };
  // every slot is refetched on every pass (past the list: tile 0, not computed), so the tile
  // loads are never skipped and the compiler's memory-counter waits stay exact.  Two passes per
  // iteration with the two window registers in turn (no copy of a window whose load is in flight)
  int walt = 0;
  auto pass = [&](const int& wuse, int& wload) {
    wload = window(nxt + D);                         // the next pass's entries
#pragma unroll
    for (int s = 0; s < D; ++s) {
      Slot& S = R[s];
      if (S.st >= 0) {
        while (cs < S.st) transition();
        compute(S, stg + (cs & 1) * SBYTES);
      }
      fetch(S, nxt + s, __builtin_amdgcn_readlane(wuse, woff + s));
    }
    nxt += D;
    woff = 0;
    return R[0].st >= 0;
  };
  while (pass(wcur, walt) && pass(walt, wcur)) {
  }
  while (cs + 1 < nstages) transition();

  // epilogue: dx = acc (+ dy)
  if (!has) return;
#pragma unroll
  for (int q = 0; q < MT; ++q) {
    const int64_t tn = t0 + 16 * q + i;
    if (tn < a.N) tprod_store<1, CW>(a, tn, c, g, acc[q]);
  }
}

template <int B>
static int launch_dxf(const TProdArgs& a0, hipStream_t st) {
  constexpr size_t lds = 2 * (size_t)64 * DxStage<B>::COLS * 2;
  TProdArgs a = a0;
  set_kdiv(a);
  const int64_t ntb = (a.N + 63) / 64;
  a.nsl = (a.C + DXF_WAVES - 1) / DXF_WAVES;
  const int64_t grid = a.nsl == 1 ? ntb : 8 * a.nsl * ((ntb + 7) / 8);
  auto kern = dxf_kernel<B, DXF_RING>;
  if (hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                          (int)lds) != hipSuccess)
    return -1;
  hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(64 * DXF_WAVES), lds, st, a);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

// staged dx when every output block fits the waves' accumulators (OPW * B / 16 <= 8) and the
// sources' widths are whole stages of 16-byte chunks
static int launch_dx_stage(int B, const TProdArgs& a0, hipStream_t st) {
  if (a0.nsrc < 1 || a0.nsrc > 2) return -2;
  for (int s = 0; s < a0.nsrc; ++s)
    if (a0.src[s].lda % B) return -2;
  // With fewer 64-token blocks than CUs, the output blocks are split over nsl workgroups per
  // token block so that each wave owns one (each workgroup stages all the activation columns).
  TProdArgs a = a0;
  const int64_t ntb = (a.N + 63) / 64;
  const int per_wg = B == 64 ? 8 : 16;
  a.nsl = ntb >= 256 ? 1 : (a.C + per_wg - 1) / per_wg;
  const int cs = (a.C + a.nsl - 1) / a.nsl;        // output blocks per slice
  // B = 32: the deep-ring kernel (headline backward 0.710 -> 0.688 ms; 64 / 1024 / 4096 tokens
  // 0.109 / 0.131 / 0.213 -> 0.105 / 0.127 / 0.199 ms)
  if (B == 32) return launch_dxf<32>(a0, st);
  // 16 waves (four per SIMD to hide the tile loads) when their accumulators fit 128 VGPRs:
  // headline backward 0.785 -> 0.740 ms, B = 16 at d_model 512 / 1024 0.497 -> 0.447 and
  // 2.10 -> 1.95 ms against 8 waves; B = 64 keeps 8 waves (16 would spill)
  const int o16 = (cs + 15) / 16;
  if (B == 16 && o16 <= 1) return launch_dx_stage_t<16, 1, 16>(a, st);
  if (B == 16 && o16 <= 2) return launch_dx_stage_t<16, 2, 16>(a, st);
  if (B == 16 && o16 <= 4) return launch_dx_stage_t<16, 4, 16>(a, st);
  if (B == 32 && o16 <= 1) return launch_dx_stage_t<32, 1, 16>(a, st);
  if (B == 32 && o16 <= 2) return launch_dx_stage_t<32, 2, 16>(a, st);
  const int opw = (cs + 7) / 8;
#define LBK_DX(BB, OO) if (B == BB && opw <= OO) return launch_dx_stage_t<BB, OO, 8>(a, st);
  if (B == 16) { LBK_DX(16, 1) LBK_DX(16, 2) LBK_DX(16, 4) LBK_DX(16, 8) }
  if (B == 32) { LBK_DX(32, 1) LBK_DX(32, 2) LBK_DX(32, 4) }
  if (B == 64) { LBK_DX(64, 1) LBK_DX(64, 2) }
#undef LBK_DX
  // B = 16 with more output blocks than the staged kernel's accumulators hold (N >= 16321 tokens
  // and more than 64 output blocks): the deep-ring kernel, one output block per wave, in place of
  // the per-entry kernel (1024 x 8192 product backward at 16384 tokens 1.275 -> 0.658 ms).  Where
  // the staged kernel fits it stays: the deep ring stages the activations once per 16 output
  // blocks and was slower there (SwiGLU backward at d_model 1024 0.823 -> 0.886 ms)
  if (B == 16) return launch_dxf<16>(a0, st);
  return -2;
}

int launch_tprod(int B, int mode, const TProdArgs& a, hipStream_t st) {
  if (a.N == 0 || a.C == 0) return 0;
  if (mode == 0 && a.nsrc == 1) {
    const int rc = launch_dh_panel(B, a, st);
    if (rc != -2) return rc;
  }
  if (mode == 1) {
    const int rc = launch_dx_stage(B, a, st);
    if (rc != -2) return rc;
  }
  const dim3 grid((unsigned)((a.N + 63) / 64), (unsigned)((a.C + 3) / 4));
#define LBK_TP(BB)                                                                      \
  if (B == BB) {                                                                        \
    if (mode == 0) hipLaunchKernelGGL((tprod_kernel<BB, 0>), grid, dim3(256), 0, st, a); \
    else hipLaunchKernelGGL((tprod_kernel<BB, 1>), grid, dim3(256), 0, st, a);           \
    return hipGetLastError() == hipSuccess ? 0 : -1;                                    \
  }
  LBK_TP(16) LBK_TP(32) LBK_TP(64)
#undef LBK_TP
  return -2;
}

// ---------------------------------------------------------------------------
// tile gradients
// ---------------------------------------------------------------------------
template <int B>
struct DWShape {
  static constexpr int TS = B == 64 ? 32 : 64;   // tokens per staged slice
  static constexpr int ROW = B + 8;              // LDS row length in elements (16 bytes of padding)
};

template <int B>
__global__ __launch_bounds__(512) void dw_kernel(DWJobs jobs) {
  constexpr int CW = B / 16;
  constexpr int CPT = B / 8;                 // 16-byte chunks per token row of a tile
  constexpr int TS = DWShape<B>::TS, ROW = DWShape<B>::ROW;
  int jt = 0;
#pragma unroll
  for (int u = 1; u < DWJobs::kMax; ++u)
    if (u < jobs.n && (int64_t)blockIdx.x >= jobs.first[u]) jt = u;
  const DWJob& J = jobs.job[jt];
  const int64_t b = (int64_t)blockIdx.x - jobs.first[jt];
  const int KG = (J.K + 7) / 8;              // slot groups of a row
  const int ch = (int)(b % J.nchunk);
  const int rg = (int)(b / J.nchunk);
  const int r = rg / KG, kg = rg - r * KG;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = uniform(tid >> 6);
  const int i = lane & 15, g = lane >> 4;
  const int k = 8 * kg + w;
  const bool slot = k < J.K;
  const int col = slot ? J.col[(int64_t)r * J.K + k] : -1;
  const bool live = col >= 0 && col < J.C;
  // LDS: row-major token slices, xs[wave][token][column] of X, gs[token][column] of G
  __shared__ __attribute__((aligned(16))) uint16_t xs[8][TS * ROW];
  __shared__ __attribute__((aligned(16))) uint16_t gs[TS * ROW];

  f32x4 acc[CW][CW];
#pragma unroll
  for (int md = 0; md < CW; ++md)
#pragma unroll
    for (int mD = 0; mD < CW; ++mD) acc[md][mD] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int64_t tbeg = (int64_t)ch * J.chunk;
  const int64_t tend = (tbeg + J.chunk) < jobs.N ? (tbeg + J.chunk) : jobs.N;
  const int64_t xcol = (int64_t)(live ? col : 0) * B;
  const int64_t gcol = (int64_t)r * B;
  for (int64_t t0 = tbeg; t0 < tend; t0 += TS) {
    // stage: each 16-byte chunk (token, 8 columns) is loaded at a clamped row, zeroed beyond
    // the chunk, and stored as it is
#pragma unroll
    for (int q0 = 0; q0 < TS * CPT; q0 += 64) {               // this wave's X slice
      const int q = q0 + lane;
      const int tt = q / CPT, cc = q - tt * CPT;
      const int64_t t = t0 + tt;
      const u32x4 v0 = ld16(J.x + (t < jobs.N ? t : jobs.N - 1) * J.ldx + xcol + 8 * cc);
      *reinterpret_cast<u32x4*>(&xs[w][tt * ROW + 8 * cc]) = (t < tend) ? v0 : u32x4{0, 0, 0, 0};
    }
    for (int q = tid; q < TS * CPT; q += 512) {               // the G slice, shared
      const int tt = q / CPT, cc = q - tt * CPT;
      const int64_t t = t0 + tt;
      const u32x4 v0 = ld16(J.gy + (t < jobs.N ? t : jobs.N - 1) * J.ldg + gcol + 8 * cc);
      *reinterpret_cast<u32x4*>(&gs[tt * ROW + 8 * cc]) = (t < tend) ? v0 : u32x4{0, 0, 0, 0};
    }
    __syncthreads();
    // dW[d][D] += sum_t X[t][d] G[t][D]: A operand = X^T (lane: column 16md + i, 8 tokens),
    // B operand = G (lane: column 16mD + n, the same 8 tokens)
#pragma unroll
    for (int ks = 0; ks < TS / 32; ++ks) {
      u32x4 bv[CW];
#pragma unroll
      for (int mD = 0; mD < CW; ++mD) bv[mD] = tr_frag(gs, ROW, 32 * ks, 16 * mD, lane);
#pragma unroll
      for (int md = 0; md < CW; ++md) {
        const u32x4 av = tr_frag(xs[w], ROW, 32 * ks, 16 * md, lane);
#pragma unroll
        for (int mD = 0; mD < CW; ++mD) acc[md][mD] = mfma_bf16(av, bv[mD], acc[md][mD]);
      }
    }
    __syncthreads();
  }
  if (!live) return;
  // lane (n, g) of acc[md][mD] holds dW[16md + 4g + v][16mD + n]
  float* part = J.part + ((int64_t)ch * J.R * J.K + (int64_t)r * J.K + k) * B * B;
#pragma unroll
  for (int md = 0; md < CW; ++md)
#pragma unroll
    for (int mD = 0; mD < CW; ++mD)
#pragma unroll
      for (int v = 0; v < 4; ++v) part[(16 * md + 4 * g + v) * B + 16 * mD + i] = acc[md][mD][v];
}

// The tile gradient (B = 16, 32) with the token slices double-buffered in LDS and filled by
// direct global->LDS loads (global_load_lds_dwordx4), so slice s + 1 streams in while slice s is
// multiplied.  The slices are unpadded rows (64 bytes at B = 32, 32 at B = 16), laid out so that
// the transposed reads of a half-wave (rows t..t+3 and t+8..t+11) cover all 64 banks once:
// at B = 32 the 16-byte chunk c of row t sits at chunk c ^ ((t & 8) >> 2); at B = 16 (a row is two
// chunks) row t sits at row slot t ^ ((t & 8) >> 1).  A load instruction fills 1 KB in place: lane
// l of instruction j brings the chunk whose position is 64 j + l.  The waits are explicit
// (s_waitcnt vmcnt with the next slice's loads still in flight) and the barriers carry no fence,
// which would wait for those loads too.
namespace {
template <int B>
struct DWD {
  static_assert(B == 16 || B == 32, "tile gradients through LDS loads: B = 16 or 32");
  static constexpr int TS = B == 32 ? 64 : 128;   // tokens per slice (4 KB of one operand)
  static constexpr int CPR = B / 8;                // 16-byte chunks per token row
  // row slot of token row t (B = 16), identity at B = 32
  __device__ static int slot(int t) { return B == 16 ? (t ^ ((t & 8) >> 1)) : t; }
  // element offset of (row t, column col) in a slice
  __device__ static int at(int t, int col) {
    if constexpr (B == 32) return t * 32 + 8 * ((col >> 3) ^ ((t & 8) >> 2)) + (col & 7);
    else return slot(t) * 16 + col;
  }
  // (token row, chunk) of 16-byte position P of a slice (the inverse of the layout)
  __device__ static void pos(int P, int& t, int& c) {
    if constexpr (B == 32) {
      t = P >> 2;
      c = (P & 3) ^ ((t & 8) >> 2);
    } else {
      t = slot(P >> 1);   // the row permutation is its own inverse
      c = P & 1;
    }
  }
};

// transposed operand of a slice: lane (s, g) gets column c0 + 4 (s & 3) .. + 3 of rows
// t0 + 8 g + s / 4 and + 4 (as tr_frag on a plain row-major slice)
template <int B>
__device__ __forceinline__ u32x4 dwd_frag(const uint16_t* slice, int t0, int c0, int lane) {
  const int s = lane & 15, g = lane >> 4;
  const int row = t0 + 8 * g + (s >> 2);
  const int col = c0 + 4 * (s & 3);
  typedef __attribute__((address_space(3))) i16x4 lds_i16x4;
  const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(slice + DWD<B>::at(row, col)));
  const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(slice + DWD<B>::at(row + 4, col)));
  const u32x2 a = __builtin_bit_cast(u32x2, lo), b = __builtin_bit_cast(u32x2, hi);
  return u32x4{a[0], a[1], b[0], b[1]};
}

// 1 KB of a slice (instruction j) from rows t0.. of a [N, ld] matrix, columns col0 .. col0 + B - 1,
// rows at or past N read from row N - 1
template <int B>
__device__ __forceinline__ void dwd_load(const uint16_t* src, int64_t ld, int64_t col0, int64_t t0, int64_t N,
                                         uint16_t* slice, int j, int lane) {
  int row, c;
  DWD<B>::pos(64 * j + lane, row, c);
  const int64_t t = t0 + row < N ? t0 + row : N - 1;
  // issued from inline assembly, so the compiler counts no load of its own here and inserts no
  // wait for these LDS writes before the reads of the other buffer; the kernel waits explicitly
  const uint32_t lds = static_cast<uint32_t>(
      reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) void*)(slice + 512 * j)));
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src + t * ld + col0 + 8 * c),
               "s"(lds) : "memory", "m0");
}

// barrier without a fence: this wave's LDS reads have returned, its loads in flight stay so
__device__ __forceinline__ void dwd_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }
}  // namespace

template <int B>
__global__ __launch_bounds__(512) void dw_dma_kernel(DWJobs jobs) {
  constexpr int CW = B / 16, TS = DWD<B>::TS, CPR = DWD<B>::CPR;
  int jt = 0;
#pragma unroll
  for (int u = 1; u < DWJobs::kMax; ++u)
    if (u < jobs.n && (int64_t)blockIdx.x >= jobs.first[u]) jt = u;
  const DWJob& J = jobs.job[jt];
  const int64_t b = (int64_t)blockIdx.x - jobs.first[jt];
  const int KG = (J.K + 7) / 8;
  const int ch = (int)(b % J.nchunk);
  const int rg = (int)(b / J.nchunk);
  const int r = rg / KG, kg = rg - r * KG;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = uniform(tid >> 6);
  const int i = lane & 15, g = lane >> 4;
  const int k = 8 * kg + w;
  const bool slot = k < J.K;
  const int col = slot ? J.col[(int64_t)r * J.K + k] : -1;
  const bool live = col >= 0 && col < J.C;
  __shared__ __attribute__((aligned(16))) uint16_t xs0[8][TS * B], xs1[8][TS * B];
  __shared__ __attribute__((aligned(16))) uint16_t gs0[TS * B], gs1[TS * B];

  f32x4 acc[CW][CW];
#pragma unroll
  for (int md = 0; md < CW; ++md)
#pragma unroll
    for (int mD = 0; mD < CW; ++mD) acc[md][mD] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int64_t N = jobs.N;
  const int64_t tbeg = (int64_t)ch * J.chunk;
  const int64_t tend = (tbeg + J.chunk) < N ? (tbeg + J.chunk) : N;
  const int ns = tbeg < tend ? (int)((tend - tbeg + TS - 1) / TS) : 0;
  const int64_t xcol = (int64_t)(live ? col : 0) * B;
  const int64_t gcol = (int64_t)r * B;
  // a slice into one buffer pair: four instructions of this wave's X slice, one of the shared
  // G slice for waves 0-3
  auto issue = [&](int s, uint16_t* xd, uint16_t* gd) {
    const int64_t t0 = tbeg + (int64_t)s * TS;
#pragma unroll
    for (int j = 0; j < 4; ++j) dwd_load<B>(J.x, J.ldx, xcol, t0, N, xd, j, lane);
    if (w < 4) dwd_load<B>(J.gy, J.ldg, gcol, t0, N, gd, w, lane);
  };
  // slice s from (xb, gb) while slice s + 1 streams into (xn, gn); the loop below passes the
  // buffers as the fixed arrays, so the compiler sees that the reads and the loads in flight
  // touch different memory and puts no wait of its own before the reads
  auto step = [&](int s, uint16_t* xb, uint16_t* gb, uint16_t* xn, uint16_t* gn) {
    const int64_t t0 = tbeg + (int64_t)s * TS;
    if (s + 1 < ns) {
      issue(s + 1, xn, gn);
      // this wave's loads of slice s are done once only slice s + 1's (5 or 4) are in flight
      if (w < 4) __builtin_amdgcn_s_waitcnt(0x0F70 | 5);
      else __builtin_amdgcn_s_waitcnt(0x0F70 | 4);
    } else {
      __builtin_amdgcn_s_waitcnt(0x0F70);
    }
    dwd_barrier();
    if (t0 + TS > tend) {
      // the last slice of the data: rows at or past tend hold clamped copies; zero them
      const int valid = (int)(tend - t0);
      for (int q = lane; q < TS * CPR; q += 64) {
        int row, c;
        DWD<B>::pos(q, row, c);
        if (row >= valid) *reinterpret_cast<u32x4*>(xb + 8 * q) = u32x4{0, 0, 0, 0};
      }
      for (int q = tid; q < TS * CPR; q += 512) {
        int row, c;
        DWD<B>::pos(q, row, c);
        if (row >= valid) *reinterpret_cast<u32x4*>(gb + 8 * q) = u32x4{0, 0, 0, 0};
      }
      __syncthreads();
    }
    // dW[d][D] += sum_t X[t][d] G[t][D] (operands as in dw_kernel)
#pragma unroll
    for (int ks = 0; ks < TS / 32; ++ks) {
      u32x4 bv[CW];
#pragma unroll
      for (int mD = 0; mD < CW; ++mD) bv[mD] = dwd_frag<B>(gb, 32 * ks, 16 * mD, lane);
#pragma unroll
      for (int md = 0; md < CW; ++md) {
        const u32x4 av = dwd_frag<B>(xb, 32 * ks, 16 * md, lane);
#pragma unroll
        for (int mD = 0; mD < CW; ++mD) acc[md][mD] = mfma_bf16(av, bv[mD], acc[md][mD]);
      }
    }
    // every wave's reads of this buffer pair have returned before slice s + 2 is loaded into it
    dwd_barrier();
  };
  if (ns > 0) issue(0, xs0[w], gs0);
  for (int s = 0; s < ns; s += 2) {
    step(s, xs0[w], gs0, xs1[w], gs1);
    if (s + 1 < ns) step(s + 1, xs1[w], gs1, xs0[w], gs0);
  }
  if (!live) return;
  float* part = J.part + ((int64_t)ch * J.R * J.K + (int64_t)r * J.K + k) * B * B;
#pragma unroll
  for (int md = 0; md < CW; ++md)
#pragma unroll
    for (int mD = 0; mD < CW; ++mD)
#pragma unroll
      for (int v = 0; v < 4; ++v) part[(16 * md + 4 * g + v) * B + 16 * mD + i] = acc[md][mD][v];
}

// ---------------------------------------------------------------------------
// tile gradients of a weight whose input rows are narrow (gate / up: x at most 1024 wide)
// ---------------------------------------------------------------------------
// dwg_kernel<XI>: a workgroup owns 8 block rows r0 .. r0 + 7 (one per wave, at most 8 slots each)
// and a chunk of tokens.  Per 32-token slice it stages the whole input row x[t, 0 : C B] and
// G[t, r0 B : (r0 + 8) B] in LDS (double-buffered, direct global->LDS loads as in dw_dma_kernel;
// XI load instructions of x per wave), and each wave computes the K tiles of its row from them,
// so x is read once per slice for the 64 tiles of the workgroup instead of once per tile:
// 2.5 KB per tile and 64 tokens against 4.5.  Row t of a slice keeps its 16-byte chunk c at
// c ^ h(t), h(t) = 2 (t & 3) | (t & 8): the transposed reads of a half-wave (rows t .. t + 3 and
// t + 8 .. t + 11, two chunks each) then cover the 64 banks once (the row strides are multiples
// of 256 bytes).  Tokens are accumulated in the order of dw_dma_kernel (32-token k-steps).
namespace {
struct DWG {
  static constexpr int TS = 32;          // tokens per slice
  static constexpr int RB = 8;           // block rows per workgroup, one per wave
  static constexpr int GW = RB * 32;     // G slice row (elements)
  static constexpr int XWMAX = 1024;     // x slice row (elements)
  __device__ static int h(int t) { return ((t & 3) << 1) | (t & 8); }
  __device__ static int at(int t, int col, int rowe) { return t * rowe + 8 * ((col >> 3) ^ h(t)) + (col & 7); }
};

// transposed operand of a slice with rows of rowe elements (the lane mapping of dwd_frag)
__device__ __forceinline__ u32x4 dwg_frag(const uint16_t* slice, int rowe, int c0, int lane) {
  const int s = lane & 15, g = lane >> 4;
  const int row = 8 * g + (s >> 2);
  const int col = c0 + 4 * (s & 3);
  typedef __attribute__((address_space(3))) i16x4 lds_i16x4;
  const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(slice + DWG::at(row, col, rowe)));
  const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(slice + DWG::at(row + 4, col, rowe)));
  const u32x2 a = __builtin_bit_cast(u32x2, lo), b = __builtin_bit_cast(u32x2, hi);
  return u32x4{a[0], a[1], b[0], b[1]};
}

// 1 KB (instruction j) of a slice with rows of rowe elements from rows t0.. of a [N, ld] matrix,
// columns col0 .. col0 + rowe - 1: lane l brings the chunk stored at position 64 j + l; rows at or
// past N read row N - 1 (zeroed before use)
__device__ __forceinline__ void dwg_load(const uint16_t* src, int64_t ld, int64_t col0, int rowe, int64_t t0,
                                         int64_t N, uint16_t* slice, int j, int lane) {
  const int cpr = rowe / 8;
  const int P = 64 * j + lane;
  const int t = P / cpr, cp = P - t * cpr;
  const int c = cp ^ DWG::h(t);
  const int64_t tt = t0 + t < N ? t0 + t : N - 1;
  const uint32_t lds = static_cast<uint32_t>(
      reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) void*)(slice + 512 * j)));
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src + tt * ld + col0 + 8 * c),
               "s"(lds) : "memory", "m0");
}
// 1 KB of a slice into LDS at slice_j from this lane's source address (dwg_load's transfer with
// the address formed by the caller)
__device__ __forceinline__ void dwt_load(const uint16_t* src, uint16_t* slice_j) {
  const uint32_t lds = static_cast<uint32_t>(
      reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) void*)slice_j));
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(lds) : "memory", "m0");
}
}  // namespace

template <int XI>
__global__ __launch_bounds__(512, 1) void dwg_kernel(DWJobs jobs) {
  constexpr int B = 32, CW = 2, TS = DWG::TS, GW = DWG::GW, KMAX = 8;
  constexpr int XW = XI * 8 * 16;                  // x slice row: 8 waves x XI KB over 32 tokens
  static_assert(XW <= DWG::XWMAX, "x slice row");
  extern __shared__ __attribute__((aligned(16))) uint16_t dwg_smem[];
  int jt = 0;
#pragma unroll
  for (int u = 1; u < DWJobs::kMax; ++u)
    if (u < jobs.n && (int64_t)blockIdx.x >= jobs.first[u]) jt = u;
  const DWJob& J = jobs.job[jt];
  const int64_t b = (int64_t)blockIdx.x - jobs.first[jt];
  const int ch = (int)(b % J.nchunk);
  const int r0 = DWG::RB * (int)(b / J.nchunk);
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = uniform(tid >> 6);
  const int i = lane & 15, g = lane >> 4;
  const int r = r0 + w;                            // this wave's block row (R is a multiple of 8)
  uint16_t* const xs0 = dwg_smem;
  uint16_t* const xs1 = dwg_smem + TS * XW;
  uint16_t* const gs0 = dwg_smem + 2 * TS * XW;
  uint16_t* const gs1 = gs0 + TS * GW;
  // the row's live slots (scalar loads, consumed here so that no wait for them falls in the loop)
  int cl[KMAX];
  unsigned live = 0;
#pragma unroll
  for (int k = 0; k < KMAX; ++k) {
    cl[k] = k < J.K ? J.col[(int64_t)r * J.K + k] : -1;
    live |= (cl[k] >= 0 && cl[k] < J.C) ? 1u << k : 0u;
  }
  live = (unsigned)uniform((int)live);

  f32x4 acc[KMAX][CW][CW];
#pragma unroll
  for (int k = 0; k < KMAX; ++k)
#pragma unroll
    for (int md = 0; md < CW; ++md)
#pragma unroll
      for (int mD = 0; mD < CW; ++mD) acc[k][md][mD] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int64_t N = jobs.N;
  const int64_t tbeg = (int64_t)ch * J.chunk;
  const int64_t tend = (tbeg + J.chunk) < N ? (tbeg + J.chunk) : N;
  const int ns = tbeg < tend ? (int)((tend - tbeg + TS - 1) / TS) : 0;
  const int64_t gcol = (int64_t)r0 * B;
  // the job's operands in registers (the loads' memory clobber would reload them from the
  // argument block before every issue)
  const uint16_t* const jx = J.x;
  const uint16_t* const jg = J.gy;
  const int64_t ldx = J.ldx, ldg = J.ldg;
  auto issue = [&](int s, uint16_t* xd, uint16_t* gd) {
    const int64_t t0 = tbeg + (int64_t)s * TS;
#pragma unroll
    for (int j = 0; j < XI; ++j) dwg_load(jx, ldx, 0, XW, t0, N, xd, w * XI + j, lane);
#pragma unroll
    for (int j = 0; j < 2; ++j) dwg_load(jg, ldg, gcol, GW, t0, N, gd, w * 2 + j, lane);
  };
  auto step = [&](int s, uint16_t* xb, uint16_t* gb, uint16_t* xn, uint16_t* gn) {
    const int64_t t0 = tbeg + (int64_t)s * TS;
    if (s + 1 < ns) {
      issue(s + 1, xn, gn);
      // this wave's loads of slice s are done once only slice s + 1's (XI + 2) are in flight
      __builtin_amdgcn_s_waitcnt(0x0F70 | (XI + 2));
    } else {
      __builtin_amdgcn_s_waitcnt(0x0F70);
    }
    dwd_barrier();
    if (t0 + TS > tend) {
      // the last slice of the data: rows at or past tend hold clamped copies; zero them
      const int valid = (int)(tend - t0);
      for (int q = tid; q < (TS - valid) * (XW / 8); q += 512)
        *reinterpret_cast<u32x4*>(xb + (int64_t)valid * XW + 8 * q) = u32x4{0, 0, 0, 0};
      for (int q = tid; q < (TS - valid) * (GW / 8); q += 512)
        *reinterpret_cast<u32x4*>(gb + (int64_t)valid * GW + 8 * q) = u32x4{0, 0, 0, 0};
      __syncthreads();
    }
    // dW[d][D] += sum_t X[t][d] G[t][D] over the slice's 32 tokens (one k-step)
    u32x4 bv[CW];
#pragma unroll
    for (int mD = 0; mD < CW; ++mD) bv[mD] = dwg_frag(gb, GW, 32 * w + 16 * mD, lane);
#pragma unroll
    for (int k = 0; k < KMAX; ++k) {
      if ((live >> k) & 1) {
        const int c = uniform(cl[k]);
#pragma unroll
        for (int md = 0; md < CW; ++md) {
          const u32x4 av = dwg_frag(xb, XW, 32 * c + 16 * md, lane);
#pragma unroll
          for (int mD = 0; mD < CW; ++mD) acc[k][md][mD] = mfma_bf16(av, bv[mD], acc[k][md][mD]);
        }
      }
    }
    // every wave's reads of this buffer pair have returned before slice s + 2 is loaded into it
    dwd_barrier();
  };
  if (ns > 0) issue(0, xs0, gs0);
  for (int s = 0; s < ns; s += 2) {
    step(s, xs0, gs0, xs1, gs1);
    if (s + 1 < ns) step(s + 1, xs1, gs1, xs0, gs0);
  }
#pragma unroll
  for (int k = 0; k < KMAX; ++k) {
    if (!((live >> k) & 1)) continue;
    float* part = J.part + ((int64_t)ch * J.R * J.K + (int64_t)r * J.K + k) * B * B;
#pragma unroll
    for (int md = 0; md < CW; ++md)
#pragma unroll
      for (int mD = 0; mD < CW; ++mD)
#pragma unroll
        for (int v = 0; v < 4; ++v) part[(16 * md + 4 * g + v) * B + 16 * mD + i] = acc[k][md][mD][v];
  }
}

// ---------------------------------------------------------------------------
// tile gradients of a weight whose output rows are narrow (down: G = dy at most 1024 wide)
// ---------------------------------------------------------------------------
// dwt_kernel<XI>: dwg_kernel with the operands' roles exchanged.  A workgroup owns 8 input column
// blocks c0 .. c0 + 7 and a chunk of tokens; per 32-token slice it stages the whole G row
// G[t, 0 : R B] (XI load instructions per wave) and X[t, c0 B : (c0 + 8) B].  The slots that read
// the 8 column blocks (the transposed lists, in list order, block after block) are pooled and
// wave w takes pooled entries w, w + 8, ..., at most KT of them per pass over the tokens (a second
// pass only when the 8 blocks have more than 8 KT slots together).  Entry e = r K + k multiplies
// X[:, c B ..] (A operand, from the narrow slice) by G[:, r B ..] (B operand, from the wide one)
// into its partial tile, stored where dw_dma_kernel stores it, in the same token order.
template <int XI>
__global__ __launch_bounds__(512, 1) void dwt_kernel(DWJobs jobs) {
  constexpr int B = 32, CW = 2, TS = DWG::TS, GW = DWG::GW, KT = 11;
  constexpr int XW = XI * 8 * 16;                  // G slice row: 8 waves x XI KB over 32 tokens
  static_assert(XW <= DWG::XWMAX, "G slice row");
  extern __shared__ __attribute__((aligned(16))) uint16_t dwg_smem[];
  int jt = 0;
#pragma unroll
  for (int u = 1; u < DWJobs::kMax; ++u)
    if (u < jobs.n && (int64_t)blockIdx.x >= jobs.first[u]) jt = u;
  const DWJob& J = jobs.job[jt];
  const int64_t b = (int64_t)blockIdx.x - jobs.first[jt];
  const int ch = (int)(b % J.nchunk);
  const int c0 = 8 * (int)(b / J.nchunk);         // C is a multiple of 8
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = uniform(tid >> 6);
  const int i = lane & 15, g = lane >> 4;
  uint16_t* const ws0 = dwg_smem;                  // G slices (wide)
  uint16_t* const ws1 = dwg_smem + TS * XW;
  uint16_t* const ns0 = dwg_smem + 2 * TS * XW;    // X slices (narrow)
  uint16_t* const ns1 = ns0 + TS * GW;
  const int K = J.K, RK = J.R * J.K;
  // pooled slot count of the 8 column blocks
  int total = 0;
#pragma unroll
  for (int q = 0; q < 8; ++q) total += J.tcnt[c0 + q];
  total = uniform(total);
  const int npass = (total + 8 * KT - 1) / (8 * KT);

  const int64_t N = jobs.N;
  const int64_t tbeg = (int64_t)ch * J.chunk;
  const int64_t tend = (tbeg + J.chunk) < N ? (tbeg + J.chunk) : N;
  const int ns = tbeg < tend ? (int)((tend - tbeg + TS - 1) / TS) : 0;
  const uint16_t* const jx = J.x;
  const uint16_t* const jg = J.gy;
  const int64_t ldx = J.ldx, ldg = J.ldg;
  const int64_t xcol = (int64_t)c0 * B;
  // element offsets of this lane's slice loads from the slice's first row (row t, stored chunk
  // position P = 64 j + lane of instruction j, source chunk c = (P mod cpr) ^ h(t)), formed once:
  // a full slice then needs only its row base, a scalar (32-bit offsets: 32 rows of ldg and ldx
  // elements stay below 2^31)
  uint32_t offw[XI], offn[2];
#pragma unroll
  for (int j = 0; j < XI; ++j) {
    const int P = 64 * (w * XI + j) + lane, t = P / (XW / 8), c = (P - t * (XW / 8)) ^ DWG::h(t);
    offw[j] = (uint32_t)(t * ldg + 8 * c);
  }
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int P = 64 * (w * 2 + j) + lane, t = P / (GW / 8), c = (P - t * (GW / 8)) ^ DWG::h(t);
    offn[j] = (uint32_t)(t * ldx + xcol + 8 * c);
  }
  auto issue = [&](int s, uint16_t* wd, uint16_t* nd) {
    int64_t t0 = tbeg + (int64_t)s * TS;
    asm volatile("" : "+s"(t0));   // no addresses of the first slice formed ahead of the pass loop
    if (t0 + TS <= N) {
      const uint16_t* bw = jg + t0 * ldg;
      const uint16_t* bn = jx + t0 * ldx;
#pragma unroll
      for (int j = 0; j < XI; ++j) dwt_load(bw + offw[j], wd + 512 * (w * XI + j));
#pragma unroll
      for (int j = 0; j < 2; ++j) dwt_load(bn + offn[j], nd + 512 * (w * 2 + j));
    } else {
      // the last slice of the data: rows at or past N read row N - 1 (the lane index through an
      // empty asm, so that these addresses are not formed ahead and kept across the loop)
      int ln = lane;
      asm volatile("" : "+v"(ln));
#pragma unroll
      for (int j = 0; j < XI; ++j) dwg_load(jg, ldg, 0, XW, t0, N, wd, w * XI + j, ln);
#pragma unroll
      for (int j = 0; j < 2; ++j) dwg_load(jx, ldx, xcol, GW, t0, N, nd, w * 2 + j, ln);
    }
  };
  for (int p = 0; p < npass; ++p) {
    // this wave's entries of pass p: lane u < KT holds entry u as one word, row r (R <= 32) |
    // column block within the group << 6 | slot index e = r K + k << 9 (e < 2^23)
    int pre[8];                                    // start of each block's run in the pool
    pre[0] = 0;
#pragma unroll
    for (int q = 1; q < 8; ++q) pre[q] = pre[q - 1] + J.tcnt[c0 + q - 1];
    const int j = 8 * KT * p + w + 8 * lane;
    const bool valid = lane < KT && j < total;
    int cb = 0, base = 0;
#pragma unroll
    for (int q = 1; q < 8; ++q)
      if (j >= pre[q]) {
        cb = q;
        base = pre[q];
      }
    const int e = valid ? J.tlist[(int64_t)(c0 + cb) * RK + (j - base)] : 0;
    const int entv = (e / K) | (cb << 6) | (e << 9);
    // a wave's entries of the pass are a prefix u < nu
    const int nu = uniform(__popcll(__ballot(valid)));
    f32x4 acc[KT][CW][CW];
#pragma unroll
    for (int u = 0; u < KT; ++u)
#pragma unroll
      for (int md = 0; md < CW; ++md)
#pragma unroll
        for (int mD = 0; mD < CW; ++mD) acc[u][md][mD] = f32x4{0.f, 0.f, 0.f, 0.f};
    auto step = [&](int s, uint16_t* wb, uint16_t* nb, uint16_t* wn, uint16_t* nn) {
      const int64_t t0 = tbeg + (int64_t)s * TS;
      if (s + 1 < ns) {
        issue(s + 1, wn, nn);
        // this wave's loads of slice s are done once only slice s + 1's (XI + 2) are in flight
        __builtin_amdgcn_s_waitcnt(0x0F70 | (XI + 2));
      } else {
        __builtin_amdgcn_s_waitcnt(0x0F70);
      }
      dwd_barrier();
      if (t0 + TS > tend) {
        // the last slice of the data: rows at or past tend hold clamped copies; zero them
        const int valid = (int)(tend - t0);
        for (int q = tid; q < (TS - valid) * (XW / 8); q += 512)
          *reinterpret_cast<u32x4*>(wb + (int64_t)valid * XW + 8 * q) = u32x4{0, 0, 0, 0};
        for (int q = tid; q < (TS - valid) * (GW / 8); q += 512)
          *reinterpret_cast<u32x4*>(nb + (int64_t)valid * GW + 8 * q) = u32x4{0, 0, 0, 0};
        __syncthreads();
      }
      // dW[e][d][D] += sum_t X[t][c B + d] G[t][r B + D] over the slice's 32 tokens
#pragma unroll
      for (int u = 0; u < KT; ++u) {
        if (u < nu) {
          const int word = __builtin_amdgcn_readlane(entv, u);
          const int cb = (word >> 6) & 7, rm = word & 63;
          u32x4 av[CW], bv[CW];
#pragma unroll
          for (int md = 0; md < CW; ++md) av[md] = dwg_frag(nb, GW, 32 * cb + 16 * md, lane);
#pragma unroll
          for (int mD = 0; mD < CW; ++mD) bv[mD] = dwg_frag(wb, XW, 32 * rm + 16 * mD, lane);
#pragma unroll
          for (int md = 0; md < CW; ++md)
#pragma unroll
            for (int mD = 0; mD < CW; ++mD) acc[u][md][mD] = mfma_bf16(av[md], bv[mD], acc[u][md][mD]);
        }
        // one entry's fragments live at a time (the accumulators take 176 VGPRs)
        __builtin_amdgcn_sched_barrier(0);
      }
      // every wave's reads of this buffer pair have returned before slice s + 2 is loaded into it
      dwd_barrier();
    };
    if (ns > 0) issue(0, ws0, ns0);
    for (int s = 0; s < ns; s += 2) {
      step(s, ws0, ns0, ws1, ns1);
      if (s + 1 < ns) step(s + 1, ws1, ns1, ws0, ns0);
    }
#pragma unroll
    for (int u = 0; u < KT; ++u) {
      if (u >= nu) continue;
      float* part = J.part + ((int64_t)ch * RK + ((unsigned)__builtin_amdgcn_readlane(entv, u) >> 9)) * B * B;
#pragma unroll
      for (int md = 0; md < CW; ++md)
#pragma unroll
        for (int mD = 0; mD < CW; ++mD)
#pragma unroll
          for (int v = 0; v < 4; ++v) part[(16 * md + 4 * g + v) * B + 16 * mD + i] = acc[u][md][mD][v];
    }
  }
}

// ---------------------------------------------------------------------------
// tile gradients at B = 16: the blocked forms above with 16 waves
// ---------------------------------------------------------------------------
// A 16 x 16 tile over a 32-token slice is one 16x16x32 MFMA whose operands are one transposed
// fragment each (dwg_frag covers 16 columns), so a wave's accumulators are one f32x4 per tile and
// 16 waves fit 128 VGPRs.  The slices keep the layout of dwg_kernel: 32 rows of the wide operand
// (XW elements) and of a 256-column narrow one, double-buffered (160 KB at XW = 1024).
//
// dwg16_kernel<XI>: a workgroup owns 16 block rows r0 .. r0 + 15 (one per wave, at most 16 slots
// each) and a token chunk; per slice it stages x[t, 0 : C 16] and G[t, r0 16 : (r0 + 16) 16].
template <int XI>
__global__ __launch_bounds__(1024, 1) void dwg16_kernel(DWJobs jobs) {
  constexpr int B = 16, TS = DWG::TS, NW = 16, RB = 16, GW = RB * 16, KMAX = 16;
  constexpr int XW = XI * NW * 16;                 // x slice row: 16 waves x XI KB over 32 tokens
  static_assert(XW <= DWG::XWMAX && GW == DWG::GW, "slice rows");
  extern __shared__ __attribute__((aligned(16))) uint16_t dwg_smem[];
  int jt = 0;
#pragma unroll
  for (int u = 1; u < DWJobs::kMax; ++u)
    if (u < jobs.n && (int64_t)blockIdx.x >= jobs.first[u]) jt = u;
  const DWJob& J = jobs.job[jt];
  const int64_t b = (int64_t)blockIdx.x - jobs.first[jt];
  const int ch = (int)(b % J.nchunk);
  const int r0 = RB * (int)(b / J.nchunk);
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = uniform(tid >> 6);
  const int i = lane & 15, g = lane >> 4;
  const int r = r0 + w;                            // this wave's block row (R is a multiple of 16)
  uint16_t* const xs0 = dwg_smem;
  uint16_t* const xs1 = dwg_smem + TS * XW;
  uint16_t* const gs0 = dwg_smem + 2 * TS * XW;
  uint16_t* const gs1 = gs0 + TS * GW;
  int cl[KMAX];
  unsigned live = 0;
#pragma unroll
  for (int k = 0; k < KMAX; ++k) {
    cl[k] = k < J.K ? J.col[(int64_t)r * J.K + k] : -1;
    live |= (cl[k] >= 0 && cl[k] < J.C) ? 1u << k : 0u;
  }
  live = (unsigned)uniform((int)live);
  f32x4 acc[KMAX];
#pragma unroll
  for (int k = 0; k < KMAX; ++k) acc[k] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int64_t N = jobs.N;
  const int64_t tbeg = (int64_t)ch * J.chunk;
  const int64_t tend = (tbeg + J.chunk) < N ? (tbeg + J.chunk) : N;
  const int ns = tbeg < tend ? (int)((tend - tbeg + TS - 1) / TS) : 0;
  const int64_t gcol = (int64_t)r0 * B;
  const uint16_t* const jx = J.x;
  const uint16_t* const jg = J.gy;
  const int64_t ldx = J.ldx, ldg = J.ldg;
  auto issue = [&](int s, uint16_t* xd, uint16_t* gd) {
    const int64_t t0 = tbeg + (int64_t)s * TS;
#pragma unroll
    for (int j = 0; j < XI; ++j) dwg_load(jx, ldx, 0, XW, t0, N, xd, w * XI + j, lane);
    dwg_load(jg, ldg, gcol, GW, t0, N, gd, w, lane);
  };
  auto step = [&](int s, uint16_t* xb, uint16_t* gb, uint16_t* xn, uint16_t* gn) {
    const int64_t t0 = tbeg + (int64_t)s * TS;
    if (s + 1 < ns) {
      issue(s + 1, xn, gn);
      // this wave's loads of slice s are done once only slice s + 1's (XI + 1) are in flight
      __builtin_amdgcn_s_waitcnt(0x0F70 | (XI + 1));
    } else {
      __builtin_amdgcn_s_waitcnt(0x0F70);
    }
    dwd_barrier();
    if (t0 + TS > tend) {
      const int valid = (int)(tend - t0);
      for (int q = tid; q < (TS - valid) * (XW / 8); q += 1024)
        *reinterpret_cast<u32x4*>(xb + (int64_t)valid * XW + 8 * q) = u32x4{0, 0, 0, 0};
      for (int q = tid; q < (TS - valid) * (GW / 8); q += 1024)
        *reinterpret_cast<u32x4*>(gb + (int64_t)valid * GW + 8 * q) = u32x4{0, 0, 0, 0};
      __syncthreads();
    }
    // dW[d][D] += sum_t X[t][c 16 + d] G[t][r 16 + D] over the slice's 32 tokens
    const u32x4 bv = dwg_frag(gb, GW, 16 * w, lane);
#pragma unroll
    for (int k = 0; k < KMAX; ++k) {
      if ((live >> k) & 1) {
        const u32x4 av = dwg_frag(xb, XW, 16 * uniform(cl[k]), lane);
        acc[k] = mfma_bf16(av, bv, acc[k]);
      }
    }
    dwd_barrier();
  };
  if (ns > 0) issue(0, xs0, gs0);
  for (int s = 0; s < ns; s += 2) {
    step(s, xs0, gs0, xs1, gs1);
    if (s + 1 < ns) step(s + 1, xs1, gs1, xs0, gs0);
  }
#pragma unroll
  for (int k = 0; k < KMAX; ++k) {
    if (!((live >> k) & 1)) continue;
    float* part = J.part + ((int64_t)ch * J.R * J.K + (int64_t)r * J.K + k) * B * B;
#pragma unroll
    for (int v = 0; v < 4; ++v) part[(4 * g + v) * B + i] = acc[k][v];
  }
}

// dwt16_kernel<XI>: dwt_kernel at B = 16 with 16 waves: a workgroup owns 16 input column blocks
// (256 columns) and stages the whole G row (R 16 <= 1024); the slots of the 16 blocks are pooled
// and wave w takes pooled entries w, w + 16, ..., at most KT per pass.
template <int XI>
__global__ __launch_bounds__(1024, 1) void dwt16_kernel(DWJobs jobs) {
  constexpr int B = 16, TS = DWG::TS, NW = 16, GW = 256, KT = 20, NCB = 16;
  constexpr int XW = XI * NW * 16;                 // G slice row: 16 waves x XI KB over 32 tokens
  static_assert(XW <= DWG::XWMAX && GW == DWG::GW, "slice rows");
  extern __shared__ __attribute__((aligned(16))) uint16_t dwg_smem[];
  int jt = 0;
#pragma unroll
  for (int u = 1; u < DWJobs::kMax; ++u)
    if (u < jobs.n && (int64_t)blockIdx.x >= jobs.first[u]) jt = u;
  const DWJob& J = jobs.job[jt];
  const int64_t b = (int64_t)blockIdx.x - jobs.first[jt];
  const int ch = (int)(b % J.nchunk);
  const int c0 = NCB * (int)(b / J.nchunk);       // C is a multiple of 16
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = uniform(tid >> 6);
  const int i = lane & 15, g = lane >> 4;
  uint16_t* const ws0 = dwg_smem;                  // G slices (wide)
  uint16_t* const ws1 = dwg_smem + TS * XW;
  uint16_t* const ns0 = dwg_smem + 2 * TS * XW;    // X slices (narrow)
  uint16_t* const ns1 = ns0 + TS * GW;
  const int K = J.K, RK = J.R * J.K;
  int total = 0;
#pragma unroll
  for (int q = 0; q < NCB; ++q) total += J.tcnt[c0 + q];
  total = uniform(total);
  const int npass = (total + NW * KT - 1) / (NW * KT);

  const int64_t N = jobs.N;
  const int64_t tbeg = (int64_t)ch * J.chunk;
  const int64_t tend = (tbeg + J.chunk) < N ? (tbeg + J.chunk) : N;
  const int ns = tbeg < tend ? (int)((tend - tbeg + TS - 1) / TS) : 0;
  const uint16_t* const jx = J.x;
  const uint16_t* const jg = J.gy;
  const int64_t ldx = J.ldx, ldg = J.ldg;
  const int64_t xcol = (int64_t)c0 * B;
  // per-lane element offsets of the slice loads from the slice's first row (as in dwt_kernel)
  uint32_t offw[XI], offn;
#pragma unroll
  for (int j = 0; j < XI; ++j) {
    const int P = 64 * (w * XI + j) + lane, t = P / (XW / 8), c = (P - t * (XW / 8)) ^ DWG::h(t);
    offw[j] = (uint32_t)(t * ldg + 8 * c);
  }
  {
    const int P = 64 * w + lane, t = P / (GW / 8), c = (P - t * (GW / 8)) ^ DWG::h(t);
    offn = (uint32_t)(t * ldx + xcol + 8 * c);
  }
  auto issue = [&](int s, uint16_t* wd, uint16_t* nd) {
    int64_t t0 = tbeg + (int64_t)s * TS;
    asm volatile("" : "+s"(t0));   // no addresses of the first slice formed ahead of the pass loop
    if (t0 + TS <= N) {
      const uint16_t* bw = jg + t0 * ldg;
#pragma unroll
      for (int j = 0; j < XI; ++j) dwt_load(bw + offw[j], wd + 512 * (w * XI + j));
      dwt_load(jx + t0 * ldx + offn, nd + 512 * w);
    } else {
      int ln = lane;
      asm volatile("" : "+v"(ln));
#pragma unroll
      for (int j = 0; j < XI; ++j) dwg_load(jg, ldg, 0, XW, t0, N, wd, w * XI + j, ln);
      dwg_load(jx, ldx, xcol, GW, t0, N, nd, w, ln);
    }
  };
  for (int p = 0; p < npass; ++p) {
    // lane u < KT holds entry u of this wave's pass: row r (R <= 64) | column block within the
    // group << 6 | slot index e = r K + k << 10 (e < 2^22)
    int pre[NCB];
    pre[0] = 0;
#pragma unroll
    for (int q = 1; q < NCB; ++q) pre[q] = pre[q - 1] + J.tcnt[c0 + q - 1];
    const int j = NW * KT * p + w + NW * lane;
    const bool valid = lane < KT && j < total;
    int cb = 0, base = 0;
#pragma unroll
    for (int q = 1; q < NCB; ++q)
      if (j >= pre[q]) {
        cb = q;
        base = pre[q];
      }
    const int e = valid ? J.tlist[(int64_t)(c0 + cb) * RK + (j - base)] : 0;
    const int entv = (e / K) | (cb << 6) | (e << 10);
    const int nu = uniform(__popcll(__ballot(valid)));
    f32x4 acc[KT];
#pragma unroll
    for (int u = 0; u < KT; ++u) acc[u] = f32x4{0.f, 0.f, 0.f, 0.f};
    auto step = [&](int s, uint16_t* wb, uint16_t* nb, uint16_t* wn, uint16_t* nn) {
      const int64_t t0 = tbeg + (int64_t)s * TS;
      if (s + 1 < ns) {
        issue(s + 1, wn, nn);
        __builtin_amdgcn_s_waitcnt(0x0F70 | (XI + 1));
      } else {
        __builtin_amdgcn_s_waitcnt(0x0F70);
      }
      dwd_barrier();
      if (t0 + TS > tend) {
        const int valid_t = (int)(tend - t0);
        for (int q = tid; q < (TS - valid_t) * (XW / 8); q += 1024)
          *reinterpret_cast<u32x4*>(wb + (int64_t)valid_t * XW + 8 * q) = u32x4{0, 0, 0, 0};
        for (int q = tid; q < (TS - valid_t) * (GW / 8); q += 1024)
          *reinterpret_cast<u32x4*>(nb + (int64_t)valid_t * GW + 8 * q) = u32x4{0, 0, 0, 0};
        __syncthreads();
      }
      // dW[e][d][D] += sum_t X[t][c 16 + d] G[t][r 16 + D] over the slice's 32 tokens
#pragma unroll
      for (int u = 0; u < KT; ++u) {
        if (u < nu) {
          const int word = __builtin_amdgcn_readlane(entv, u);
          const int cbu = (word >> 6) & 15, rm = word & 63;
          const u32x4 av = dwg_frag(nb, GW, 16 * cbu, lane);
          const u32x4 bv = dwg_frag(wb, XW, 16 * rm, lane);
          acc[u] = mfma_bf16(av, bv, acc[u]);
        }
      }
      dwd_barrier();
    };
    if (ns > 0) issue(0, ws0, ns0);
    for (int s = 0; s < ns; s += 2) {
      step(s, ws0, ns0, ws1, ns1);
      if (s + 1 < ns) step(s + 1, ws1, ns1, ws0, ns0);
    }
#pragma unroll
    for (int u = 0; u < KT; ++u) {
      if (u >= nu) continue;
      float* part = J.part + ((int64_t)ch * RK + ((unsigned)__builtin_amdgcn_readlane(entv, u) >> 10)) * B * B;
#pragma unroll
      for (int v = 0; v < 4; ++v) part[(4 * g + v) * B + i] = acc[u][v];
    }
  }
}

// dW[e] = sum over chunks of the partial tiles (fixed order), bf16; dead slots -> 0.  Four
// consecutive elements of one tile per thread (16-byte partial loads, four chunks in flight)
__global__ __launch_bounds__(256) void dw_reduce_kernel(DWJobs jobs, int B) {
  int jt = 0;
#pragma unroll
  for (int u = 1; u < DWJobs::kMax; ++u)
    if (u < jobs.n && (int64_t)blockIdx.x >= jobs.rfirst[u]) jt = u;
  const DWJob& J = jobs.job[jt];
  const int64_t idx = (((int64_t)blockIdx.x - jobs.rfirst[jt]) * 256 + threadIdx.x) * 4;
  const int64_t per = (int64_t)J.R * J.K * B * B;
  if (idx >= per) return;
  const int64_t e = idx / ((int64_t)B * B);
  const int col = J.col[e];
  f32x4 s = {0.f, 0.f, 0.f, 0.f};
  if (col >= 0 && col < J.C) {
    const float* p = J.part + idx;
    const int nc = J.nchunk;
    int ch = 0;
    for (; ch + 4 <= nc; ch += 4) {
      f32x4 v[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) v[q] = *reinterpret_cast<const f32x4*>(p + (int64_t)(ch + q) * per);
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int m = 0; m < 4; ++m) s[m] += v[q][m];
    }
    for (; ch < nc; ++ch) {
      const f32x4 v = *reinterpret_cast<const f32x4*>(p + (int64_t)ch * per);
#pragma unroll
      for (int m = 0; m < 4; ++m) s[m] += v[m];
    }
  }
  const float o[4] = {s[0], s[1], s[2], s[3]};
  store_bf16<4>(J.dw + idx, o);
}

// the transposed-list kernels: column blocks per workgroup, and whether a weight's shape fits
static int dwt_blocks(int B) { return B == 32 ? 8 : 16; }
static bool dwt_shape(int B, int R, int C, int64_t ldg) {
  if (B == 32) return C % 8 == 0 && (R == 8 || R == 16 || R == 32) && ldg >= (int64_t)R * 32;
  if (B == 16) return C % 16 == 0 && (R == 16 || R == 32 || R == 64) && ldg >= (int64_t)R * 16;
  return false;
}

int dw_job_chunk(int B, int R, int C, int64_t ldg, int64_t N) {
  const bool wide_in = (int64_t)C * B > 1024;
  // one workgroup per CU (160 KB of LDS): with fewer than 256 the slot-per-wave kernel is faster
  // (at 128 workgroups: 151 against 117 us for the config-2 down weight)
  const int64_t half = DW_CHUNK / 2;
  const bool fills = (int64_t)(C / dwt_blocks(B)) * ((N + half - 1) / half) >= 256;
  return wide_in && dwt_shape(B, R, C, ldg) && fills ? (int)half : DW_CHUNK;
}

int launch_dw(int B, const DWJob* jobs_in, int n, int64_t N, hipStream_t st) {
  if (n < 1 || n > DWJobs::kMax) return -2;
  DWJob jobs[DWJobs::kMax];
  for (int t = 0; t < n; ++t) {
    jobs[t] = jobs_in[t];
    jobs[t].chunk = dw_job_chunk(B, jobs[t].R, jobs[t].C, jobs[t].ldg, N);   // whole slices of 32 and 64 tokens
    jobs[t].nchunk = N > 0 ? (int)((N + jobs[t].chunk - 1) / jobs[t].chunk) : 0;
  }
  DWJobs J{};
  J.n = n;
  J.N = N;
  int64_t rblocks = 0;
  for (int t = 0; t < n; ++t) {
    J.job[t] = jobs[t];
    J.rfirst[t] = rblocks;
    rblocks += ((int64_t)jobs[t].R * jobs[t].K * B * B / 4 + 255) / 256;
  }
  // B = 32 weights with at most 8 slots per row, rows in whole groups of 8 and narrow input rows
  // (the gate and up weights of d_model <= 1024) take dwg_kernel, one launch per input width;
  // the rest dw_dma_kernel (dw_kernel at B = 64)
  // (the x slice row C * 32 is XI KB per wave over the 8 waves, XI in {1, 2, 4, 8}: C in {4, 8, 16, 32})
  auto narrow = [&](const DWJob& j) {
    return B == 32 && j.K <= 8 && j.R % DWG::RB == 0 && (j.C == 4 || j.C == 8 || j.C == 16 || j.C == 32) &&
           j.ldx >= (int64_t)j.C * 32;
  };
  bool taken[DWJobs::kMax] = {};
  for (int t = 0; t < n; ++t) {
    if (taken[t] || !narrow(jobs[t])) continue;
    DWJobs G = J;
    G.n = 0;
    int64_t gb = 0;
    for (int u = t; u < n; ++u)
      if (!taken[u] && narrow(jobs[u]) && jobs[u].C == jobs[t].C) {
        taken[u] = true;
        G.job[G.n] = jobs[u];
        G.first[G.n++] = gb;
        gb += (int64_t)(jobs[u].R / DWG::RB) * jobs[u].nchunk;
      }
    // one workgroup per CU (160 KB of LDS each): with fewer than 256 the wide-grid kernel is faster
    // (at 4096 tokens, 64 workgroups: whole backward 0.198 -> 0.258 ms)
    if (gb < 256) {
      for (int u = t; u < n; ++u)
        if (narrow(jobs[u]) && jobs[u].C == jobs[t].C) taken[u] = false;
      continue;
    }
    const int xi = jobs[t].C / 4;                    // 1 KB load instructions of x per wave and slice
    const size_t lds = (size_t)2 * 32 * 2 * (jobs[t].C * 32 + DWG::RB * 32);
    auto kern = xi == 8 ? dwg_kernel<8> : xi == 4 ? dwg_kernel<4> : xi == 2 ? dwg_kernel<2> : dwg_kernel<1>;
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)lds) != hipSuccess)
      return -1;
    hipLaunchKernelGGL(kern, dim3((unsigned)gb), dim3(512), lds, st, G);
    if (hipGetLastError() != hipSuccess) return -1;
  }
  // B = 16 weights with at most 16 slots per row, rows in whole groups of 16 and input rows of
  // 256 to 1024 elements (the gate and up weights of such models) take dwg16_kernel
  // (XI = C / 16 in {1, 2, 4}: C in {16, 32, 64})
  auto narrow16 = [&](const DWJob& j) {
    return B == 16 && j.K <= 16 && j.R % 16 == 0 && (j.C == 16 || j.C == 32 || j.C == 64) &&
           j.ldx >= (int64_t)j.C * 16;
  };
  for (int t = 0; t < n; ++t) {
    if (taken[t] || !narrow16(jobs[t])) continue;
    DWJobs G = J;
    G.n = 0;
    int64_t gb = 0;
    for (int u = t; u < n; ++u)
      if (!taken[u] && narrow16(jobs[u]) && jobs[u].C == jobs[t].C) {
        taken[u] = true;
        G.job[G.n] = jobs[u];
        G.first[G.n++] = gb;
        gb += (int64_t)(jobs[u].R / 16) * jobs[u].nchunk;
      }
    if (gb < 256) {
      for (int u = t; u < n; ++u)
        if (narrow16(jobs[u]) && jobs[u].C == jobs[t].C) taken[u] = false;
      continue;
    }
    const int xi = jobs[t].C / 16;                   // 1 KB load instructions of x per wave and slice
    const size_t lds = (size_t)2 * 32 * 2 * (jobs[t].C * 16 + DWG::GW);
    auto kern = xi == 4 ? dwg16_kernel<4> : xi == 2 ? dwg16_kernel<2> : dwg16_kernel<1>;
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)lds) != hipSuccess)
      return -1;
    hipLaunchKernelGGL(kern, dim3((unsigned)gb), dim3(1024), lds, st, G);
    if (hipGetLastError() != hipSuccess) return -1;
  }
  // weights given the half chunk (narrow output rows, R B <= 1024: the down weight of d_model <=
  // 1024, with enough workgroups) and their transposed lists take dwt_kernel (dwt16_kernel at
  // B = 16), one launch per output width
  auto narrow_out = [&](const DWJob& j) { return j.chunk == DW_CHUNK / 2 && j.tcnt && j.tlist; };
  for (int t = 0; t < n; ++t) {
    if (taken[t] || !narrow_out(jobs[t])) continue;
    DWJobs G = J;
    G.n = 0;
    int64_t gb = 0;
    for (int u = t; u < n; ++u)
      if (!taken[u] && narrow_out(jobs[u]) && jobs[u].R == jobs[t].R) {
        taken[u] = true;
        G.job[G.n] = jobs[u];
        G.first[G.n++] = gb;
        gb += (int64_t)(jobs[u].C / dwt_blocks(B)) * jobs[u].nchunk;
      }
    // 1 KB load instructions of G per wave and slice: R B / 128 over 8 waves (B = 32) or 16 (B = 16)
    const int xi = B == 32 ? jobs[t].R / 4 : jobs[t].R / 16;
    const size_t lds = (size_t)2 * 32 * 2 * (jobs[t].R * B + DWG::GW);
    auto kern = B == 32 ? (xi == 8 ? dwt_kernel<8> : xi == 4 ? dwt_kernel<4> : dwt_kernel<2>)
                        : (xi == 4 ? dwt16_kernel<4> : xi == 2 ? dwt16_kernel<2> : dwt16_kernel<1>);
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)lds) != hipSuccess)
      return -1;
    hipLaunchKernelGGL(kern, dim3((unsigned)gb), dim3(B == 32 ? 512 : 1024), lds, st, G);
    if (hipGetLastError() != hipSuccess) return -1;
  }
  DWJobs D = J;
  D.n = 0;
  int64_t blocks = 0;
  for (int t = 0; t < n; ++t) {
    if (taken[t]) continue;
    D.job[D.n] = jobs[t];
    D.first[D.n++] = blocks;
    blocks += (int64_t)jobs[t].R * ((jobs[t].K + 7) / 8) * jobs[t].nchunk;
  }
  if (blocks > 0) {
    const DWJobs& J = D;
    if (B == 16) hipLaunchKernelGGL(dw_dma_kernel<16>, dim3((unsigned)blocks), dim3(512), 0, st, J);
    else if (B == 32) hipLaunchKernelGGL(dw_dma_kernel<32>, dim3((unsigned)blocks), dim3(512), 0, st, J);
    else if (B == 64) hipLaunchKernelGGL(dw_kernel<64>, dim3((unsigned)blocks), dim3(512), 0, st, J);
    else return -2;
    if (hipGetLastError() != hipSuccess) return -1;
  }
  if (rblocks > 0) hipLaunchKernelGGL(dw_reduce_kernel, dim3((unsigned)rblocks), dim3(256), 0, st, J, B);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace lbk
