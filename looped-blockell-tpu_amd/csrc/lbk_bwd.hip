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
//   tprod_kernel   out[:, c] = sum over the slots of column block c of
//                  A[:, r] W[r,k]^T.  A workgroup owns 64 tokens x one column
//                  block; the raw [B_in, B_out] tile is the MFMA's A operand (row
//                  d of the tile holds the 8 consecutive B_out values a lane
//                  needs), the activation rows the B operand, so each lane ends
//                  with 4 consecutive output columns of one token.  Epilogue:
//                  the SiLU*mul backward (dh -> dg, du) or the optional + dy (-> dx).
//   dw_kernel      tile gradients: a workgroup owns one block row, up to 8 of
//                  its slots (one per wave) and a chunk of tokens; 32-token
//                  slices of X and G are staged transposed in LDS (the token
//                  index is the MFMA's k) and every wave accumulates its tile in
//                  fp32; the chunk's partial tile goes to the workspace.
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

template <int B, int MODE>
__global__ __launch_bounds__(256) void tprod_kernel(TProdArgs a) {
  constexpr int CW = B / 16;                 // 16-column groups of a tile
  constexpr int NKS = B >= 32 ? B / 32 : 1;  // 32-deep k-steps
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = uniform(tid >> 6);
  const int i = lane & 15, g = lane >> 4;
  const int c = (int)blockIdx.y;
  const int64_t tn = (int64_t)blockIdx.x * 64 + 16 * w + i;   // this lane's token
  const int64_t tl = tn < a.N ? tn : a.N - 1;                 // clamped row for the loads
  // B = 16: a tile row has 16 values, so lanes g >= 2 (k 16..31) read lane g - 2's bytes and
  // carry zeros in the activation operand
  const int gk = (B == 16) ? (g & 1) : g;
  const bool kz = (B == 16) && g >= 2;
  f32x4 acc[CW];
#pragma unroll
  for (int m = 0; m < CW; ++m) acc[m] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (int s = 0; s < a.nsrc; ++s) {
    const TProdSrc S = a.src[s];
    const int cnt = S.cnt[c];
    const int32_t* L = S.list + (int64_t)c * S.cap;
    const uint16_t* arow = S.a + tl * S.lda + 8 * gk;
    for (int j0 = 0; j0 < cnt; j0 += 64) {
      const int lv = (j0 + lane < cnt) ? L[j0 + lane] : 0;   // 64 entries, one per lane
      const int jn = (cnt - j0) < 64 ? (cnt - j0) : 64;
      for (int jj = 0; jj < jn; ++jj) {
        const int e = __builtin_amdgcn_readlane(lv, jj);
        const int r = e / S.K;
        const uint16_t* tile = S.w + (int64_t)e * B * B + (int64_t)i * B + 8 * gk;
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) {
          const u32x4 bv0 = ld16(arow + (int64_t)r * B + 32 * ks);
          const u32x4 bv = kz ? u32x4{0, 0, 0, 0} : bv0;
#pragma unroll
          for (int m = 0; m < CW; ++m) {
            const u32x4 av = ld16(tile + 16 * m * B + 32 * ks);   // W[16m + i][32ks + 8g ..]
            acc[m] = mfma_bf16(av, bv, acc[m]);
          }
        }
      }
    }
  }

  // lane (i, g) holds out[token tn][c*B + 16m + 4g + v], v < 4
  if (tn >= a.N) return;
#pragma unroll
  for (int m = 0; m < CW; ++m) {
    const int64_t off = tn * a.ldo + (int64_t)c * B + 16 * m + 4 * g;
    float o[4];
    if constexpr (MODE == 0) {
      float gv[4], uv[4], dgv[4], duv[4];
      load_bf16<4>(a.g + off, gv);
      load_bf16<4>(a.u + off, uv);
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const float dh = acc[m][v];
        const float sg = __builtin_amdgcn_rcpf(1.0f + __expf(-gv[v]));   // sigmoid(g)
        dgv[v] = dh * uv[v] * (sg + gv[v] * sg * (1.0f - sg));
        duv[v] = dh * gv[v] * sg;
      }
      store_bf16<4>(a.dg + off, dgv);
      store_bf16<4>(a.du + off, duv);
    } else {
      float rv[4] = {0.f, 0.f, 0.f, 0.f};
      if (a.resid) load_bf16<4>(a.resid + off, rv);
#pragma unroll
      for (int v = 0; v < 4; ++v) o[v] = acc[m][v] + rv[v];
      store_bf16<4>(a.out + off, o);
    }
  }
}

int launch_tprod(int B, int mode, const TProdArgs& a, hipStream_t st) {
  if (a.N == 0 || a.C == 0) return 0;
  const dim3 grid((unsigned)((a.N + 63) / 64), (unsigned)a.C);
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
constexpr int DW_TS = 32;   // tokens per staged slice (one MFMA k-step)

template <int B>
__global__ __launch_bounds__(512) void dw_kernel(DWJobs jobs) {
  constexpr int CW = B / 16;
  constexpr int CPT = B / 8;                 // 16-byte chunks per token row of a tile
  int jt = 0;
#pragma unroll
  for (int u = 1; u < DWJobs::kMax; ++u)
    if (u < jobs.n && (int64_t)blockIdx.x >= jobs.first[u]) jt = u;
  const DWJob& J = jobs.job[jt];
  const int64_t b = (int64_t)blockIdx.x - jobs.first[jt];
  const int KG = (J.K + 7) / 8;              // slot groups of a row
  const int ch = (int)(b % jobs.nchunk);
  const int rg = (int)(b / jobs.nchunk);
  const int r = rg / KG, kg = rg - r * KG;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = uniform(tid >> 6);
  const int i = lane & 15, g = lane >> 4;
  const int k = 8 * kg + w;
  const bool slot = k < J.K;
  const int col = slot ? J.col[(int64_t)r * J.K + k] : -1;
  const bool live = col >= 0 && col < J.C;
  // LDS, transposed slices: xt[wave][column][token], gt[column][token]
  __shared__ __attribute__((aligned(16))) uint16_t xt[8][B][DW_TS];
  __shared__ __attribute__((aligned(16))) uint16_t gt[B][DW_TS];

  f32x4 acc[CW][CW];
#pragma unroll
  for (int md = 0; md < CW; ++md)
#pragma unroll
    for (int mD = 0; mD < CW; ++mD) acc[md][mD] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int64_t tbeg = (int64_t)ch * jobs.chunk;
  const int64_t tend = (tbeg + jobs.chunk) < jobs.N ? (tbeg + jobs.chunk) : jobs.N;
  const int64_t xcol = (int64_t)(live ? col : 0) * B;
  const int64_t gcol = (int64_t)r * B;
  for (int64_t t0 = tbeg; t0 < tend; t0 += DW_TS) {
    // stage: every chunk (token, 8 columns) is loaded at a clamped row, zeroed beyond N,
    // and written transposed (8 two-byte stores)
    for (int q = lane; q < DW_TS * CPT; q += 64) {            // this wave's X slice
      const int tt = q / CPT, cc = q - tt * CPT;
      const int64_t t = t0 + tt;
      const u32x4 v0 = ld16(J.x + (t < jobs.N ? t : jobs.N - 1) * J.ldx + xcol + 8 * cc);
      const u32x4 v = (t < tend) ? v0 : u32x4{0, 0, 0, 0};
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        xt[w][8 * cc + 2 * p][tt] = (uint16_t)(v[p] & 0xffffu);
        xt[w][8 * cc + 2 * p + 1][tt] = (uint16_t)(v[p] >> 16);
      }
    }
    for (int q = tid; q < DW_TS * CPT; q += 512) {            // the G slice, shared
      const int tt = q / CPT, cc = q - tt * CPT;
      const int64_t t = t0 + tt;
      const u32x4 v0 = ld16(J.gy + (t < jobs.N ? t : jobs.N - 1) * J.ldg + gcol + 8 * cc);
      const u32x4 v = (t < tend) ? v0 : u32x4{0, 0, 0, 0};
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        gt[8 * cc + 2 * p][tt] = (uint16_t)(v[p] & 0xffffu);
        gt[8 * cc + 2 * p + 1][tt] = (uint16_t)(v[p] >> 16);
      }
    }
    __syncthreads();
    // dW[d][D] += sum_t X[t][d] G[t][D]: A operand lane (i, g) = X^T[16md + i][8g ..],
    // B operand lane (n, g) = G^T[16mD + n][8g ..]
#pragma unroll
    for (int md = 0; md < CW; ++md) {
      const u32x4 av = *reinterpret_cast<const u32x4*>(&xt[w][16 * md + i][8 * g]);
#pragma unroll
      for (int mD = 0; mD < CW; ++mD) {
        const u32x4 bv = *reinterpret_cast<const u32x4*>(&gt[16 * mD + i][8 * g]);
        acc[md][mD] = mfma_bf16(av, bv, acc[md][mD]);
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

// dW[e] = sum over chunks of the partial tiles (fixed order), bf16; dead slots -> 0
__global__ __launch_bounds__(256) void dw_reduce_kernel(DWJobs jobs, int B) {
  int jt = 0;
#pragma unroll
  for (int u = 1; u < DWJobs::kMax; ++u)
    if (u < jobs.n && (int64_t)blockIdx.x >= jobs.rfirst[u]) jt = u;
  const DWJob& J = jobs.job[jt];
  const int64_t idx = ((int64_t)blockIdx.x - jobs.rfirst[jt]) * 256 + threadIdx.x;
  const int64_t per = (int64_t)J.R * J.K * B * B;
  if (idx >= per) return;
  const int64_t e = idx / ((int64_t)B * B);
  const int col = J.col[e];
  float s = 0.f;
  if (col >= 0 && col < J.C)
    for (int ch = 0; ch < jobs.nchunk; ++ch) s += J.part[(int64_t)ch * per + idx];
  J.dw[idx] = f2bf(s);
}

int launch_dw(int B, const DWJob* jobs, int n, int64_t N, int chunk, hipStream_t st) {
  if (n < 1 || n > DWJobs::kMax || chunk < DW_TS || chunk % DW_TS) return -2;
  DWJobs J{};
  J.n = n;
  J.N = N;
  J.chunk = chunk;
  J.nchunk = N > 0 ? (int)((N + chunk - 1) / chunk) : 0;
  int64_t blocks = 0, rblocks = 0;
  for (int t = 0; t < n; ++t) {
    J.job[t] = jobs[t];
    J.first[t] = blocks;
    blocks += (int64_t)jobs[t].R * ((jobs[t].K + 7) / 8) * J.nchunk;
    J.rfirst[t] = rblocks;
    rblocks += ((int64_t)jobs[t].R * jobs[t].K * B * B + 255) / 256;
  }
  if (blocks > 0) {
    if (B == 16) hipLaunchKernelGGL(dw_kernel<16>, dim3((unsigned)blocks), dim3(512), 0, st, J);
    else if (B == 32) hipLaunchKernelGGL(dw_kernel<32>, dim3((unsigned)blocks), dim3(512), 0, st, J);
    else if (B == 64) hipLaunchKernelGGL(dw_kernel<64>, dim3((unsigned)blocks), dim3(512), 0, st, J);
    else return -2;
    if (hipGetLastError() != hipSuccess) return -1;
  }
  if (rblocks > 0) hipLaunchKernelGGL(dw_reduce_kernel, dim3((unsigned)rblocks), dim3(256), 0, st, J, B);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace lbk
