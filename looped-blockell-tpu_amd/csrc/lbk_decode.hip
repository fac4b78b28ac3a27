// lbk_decode.hip — decode-shaped SwiGLU FFN (N <= 16 tokens) in one launch (gfx950).
//
// With 16 tokens every weight byte feeds 16 MACs, so the forward is a stream of
// the weights through HBM: what matters is having most of them in flight at
// once and not paying a second launch (~2.5 us each on this part).  One grid of
// G >= max(R_ff, R_m) workgroups, at most one per CU so all are resident, does
// both projections:
//
//   phase 1  workgroup b < R_ff computes h row block b (and b + G, ...): waves
//            0-3 take the gate slots, waves 4-7 the up slots, each wave issuing
//            the loads of two tiles before their MFMAs (raw [B_in, B_out] tiles,
//            transposed into MFMA fragments in registers); the partial sums meet
//            in LDS and h = silu(g) * u is published with a flag that carries
//            this call's tag.
//   phase 2  down row rm is split into S slot ranges of at most 8 slots; unit
//            (rm, s) runs on workgroup rm * S + s, one slot per wave, and its
//            tiles are requested at kernel start, so the down weights stream in
//            together with the gate/up weights and every CU pulls about the same
//            number of bytes.  Each wave waits (bounded spin) for the flag of the
//            h block it reads; the unit's sum goes to the workspace, and the last
//            of the S units of a row to arrive (tagged counter) adds the S sums in
//            fixed order plus the residual and stores the bf16 output, so the
//            result is deterministic.
//
// Cross-XCD visibility of h: the L2 is per XCD and not coherent for ordinary
// accesses, and agent-scope release/acquire fences write back or invalidate
// whole L2s (measured 3x slower here).  Instead h is written and read only with
// agent-scope atomic accesses (device-coherent); each writer wave waits for its
// stores to complete (s_waitcnt 0) before the workgroup barrier that precedes
// the flag store, and readers issue their h loads only after the flag load has
// returned the expected tag.
//
// Call tags: the host gives every call a 64-bit epoch (a process-wide counter
// from a random start).  Flags are published as the epoch and the per-row
// counters carry its low bits, so nothing in the workspace needs clearing and
// garbage in a fresh workspace matches only with probability about 2^-52.
// Because the epoch is fixed at call time, the entry point does not use this
// kernel while the stream is being captured into a graph.
#include "lbk_device.h"
#include "lbk_internal.h"

namespace lbk {

namespace {

constexpr int DEC_SPIN_LIMIT = 1 << 22;   // polling bound (~seconds); every wait ends

// Counter word: tag << 12 | count, tag = low 52 bits of the epoch, count up to
// 4095.  Returns this arrival's 1-based count for the tag
// (-1 if the bounded retry ran out).
__device__ __forceinline__ int arrive(uint64_t* cnt, uint64_t epoch) {
  const uint64_t tag = epoch & ((1ull << 52) - 1);
  uint64_t old = __hip_atomic_load(cnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  for (int tries = 0; tries < 4096; ++tries) {
    const uint64_t nw = ((old >> 12) == tag) ? old + 1 : ((tag << 12) | 1ull);
    if (__hip_atomic_compare_exchange_strong(cnt, &old, nw, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT))
      return (int)(nw & 4095);
  }
  return -1;
}

// all of this wave's memory operations complete, and no compiler motion across
__device__ __forceinline__ void drain_memory() {
  __builtin_amdgcn_s_waitcnt(0);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

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

// A fragments of x rows (ordinary loads; rows >= N are zero)
template <int B>
__device__ __forceinline__ void load_a_x(const uint16_t* base, int64_t ld, int N, int i, int g,
                                         u32x4 (&a)[TileShape<B>::NKS]) {
#pragma unroll
  for (int ks = 0; ks < TileShape<B>::NKS; ++ks)
    a[ks] = (i < N) ? load_afrag<B>(base + (int64_t)i * ld, ks, g) : u32x4{0, 0, 0, 0};
}

// A fragments of h rows through device-coherent 8-byte atomic loads
template <int B>
__device__ __forceinline__ void load_a_h(const uint16_t* base, int64_t ld, int N, int i, int g,
                                         u32x4 (&a)[TileShape<B>::NKS]) {
#pragma unroll
  for (int ks = 0; ks < TileShape<B>::NKS; ++ks) {
    a[ks] = u32x4{0, 0, 0, 0};
    if (i < N && !(B == 16 && g >= 2)) {
      const uint64_t* p = reinterpret_cast<const uint64_t*>(base + (int64_t)i * ld + 32 * ks + 8 * g);
      const uint64_t lo = __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const uint64_t hi = __hip_atomic_load(p + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      a[ks] = u32x4{(uint32_t)lo, (uint32_t)(lo >> 32), (uint32_t)hi, (uint32_t)(hi >> 32)};
    }
  }
}

}  // namespace

template <int B>
__global__ __launch_bounds__(512, 1) void decode_kernel(DecodeArgs a) {
  constexpr int CW = TileShape<B>::CW;
  constexpr int NKS = TileShape<B>::NKS;
  __shared__ f32x4 red[8][CW][64];
  __shared__ int s_last;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = uniform(tid >> 6);
  const int i = lane & 15, g = lane >> 4;
  const int G = (int)gridDim.x, b = (int)blockIdx.x;
  const int C_in = a.d_model / B;
  const int64_t d_ff = (int64_t)a.R_ff * B;
  const uint64_t flag_val = a.epoch;
  const int units = a.R_m * a.S;
  const int P = (a.Kd + a.S - 1) / a.S;   // slots per unit (<= 8)

  // ---- down unit of this workgroup: its tile is requested now
  WRaw<B> dt;
  int d_rm = -1, d_c = -1;
  auto down_fetch = [&](int u) {
    d_rm = u / a.S;
    const int k = (u - d_rm * a.S) * P + w;
    d_c = -1;
    if (w < P && k < a.Kd) {
      const int c = a.cd[(int64_t)d_rm * a.Kd + k];
      if (c >= 0 && c < a.R_ff) {
        d_c = c;
        load_wraw<B>(a.vd + ((int64_t)d_rm * a.Kd + k) * B * B, lane, dt);
      }
    }
  };
  if (b < units) down_fetch(b);

  // ---- phase 1: h row blocks
  const bool gate_wave = w < 4;
  const int Km = gate_wave ? a.Kg : a.Ku;
  const uint16_t* vm = gate_wave ? a.vg : a.vu;
  const int32_t* cm = gate_wave ? a.cg : a.cu;
  for (int r = b; r < a.R_ff; r += G) {
    f32x4 acc[CW];
#pragma unroll
    for (int m = 0; m < CW; ++m) acc[m] = f32x4{0.f, 0.f, 0.f, 0.f};
    // this wave's slots k = (w & 3) + 4j, two at a time, both tiles requested first
    for (int k0 = w & 3; k0 < Km; k0 += 8) {
      const int k1 = k0 + 4;
      const int c0 = cm[(int64_t)r * Km + k0];
      const int c1 = k1 < Km ? cm[(int64_t)r * Km + k1] : -1;
      WRaw<B> t0, t1;
      load_wraw<B>(vm + ((int64_t)r * Km + k0) * B * B, lane, t0);
      if (k1 < Km) load_wraw<B>(vm + ((int64_t)r * Km + k1) * B * B, lane, t1);
      u32x4 a0[NKS], a1[NKS];
      const bool ok0 = c0 >= 0 && c0 < C_in, ok1 = c1 >= 0 && c1 < C_in;
      load_a_x<B>(a.x + (int64_t)(ok0 ? c0 : 0) * B, a.d_model, ok0 ? a.N : 0, i, g, a0);
      load_a_x<B>(a.x + (int64_t)(ok1 ? c1 : 0) * B, a.d_model, ok1 ? a.N : 0, i, g, a1);
      mfma_tile<B>(a0, t0, acc);
      if (k1 < Km) mfma_tile<B>(a1, t1, acc);
    }
#pragma unroll
    for (int m = 0; m < CW; ++m) red[w][m][lane] = acc[m];
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
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int t = 4 * (l >> 4) + v;
        if (t < a.N)
          __hip_atomic_store(&a.h[(int64_t)t * d_ff + col], f2bf(silu_f(gs[v]) * us[v]), __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    drain_memory();
    __syncthreads();
    if (tid == 0) __hip_atomic_store(&a.flags[r], flag_val, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }

  // ---- phase 2: down units
  for (int u = b; u < units; u += G) {
    if (u != b) down_fetch(u);
    f32x4 acc[CW];
#pragma unroll
    for (int m = 0; m < CW; ++m) acc[m] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (d_c >= 0) {
      int spins = 0;
      while (__hip_atomic_load(&a.flags[d_c], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != flag_val &&
             spins < DEC_SPIN_LIMIT) {
        __builtin_amdgcn_s_sleep(2);
        ++spins;
      }
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
      u32x4 av[NKS];
      load_a_h<B>(a.h + (int64_t)d_c * B, d_ff, a.N, i, g, av);
      mfma_tile<B>(av, dt, acc);
    }
#pragma unroll
    for (int m = 0; m < CW; ++m) red[w][m][lane] = acc[m];
    __syncthreads();
    const int s = u - d_rm * a.S;
    if (tid < 64 * CW) {
      const int m = tid >> 6, l = tid & 63;
      f32x4 ps = red[0][m][l];
#pragma unroll
      for (int ww = 1; ww < 8; ++ww) ps += red[ww][m][l];
      const int col = d_rm * B + CW * (l & 15) + m;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int t = 4 * (l >> 4) + v;
        if (t < a.N)
          __hip_atomic_store(&a.parts[((int64_t)s * a.N + t) * a.d_model + col], ps[v], __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    drain_memory();
    __syncthreads();
    if (tid == 0) s_last = arrive(&a.rowcnt[d_rm], a.epoch) == a.S;
    __syncthreads();
    if (s_last) {
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
      // the row block's N x B outputs: fixed-order sum of the S unit sums + residual
      for (int e = tid; e < a.N * B; e += 512) {
        const int t = e / B, col = d_rm * B + (e - t * B);
        float v = 0.f;
        for (int ss = 0; ss < a.S; ++ss)
          v += __hip_atomic_load(&a.parts[((int64_t)ss * a.N + t) * a.d_model + col], __ATOMIC_RELAXED,
                                 __HIP_MEMORY_SCOPE_AGENT);
        if (a.resid) v += bf2f(a.resid[(int64_t)t * a.d_model + col]);
        a.out[(int64_t)t * a.d_model + col] = f2bf(v);
      }
    }
    __syncthreads();
  }

}

static int num_cus() {
  static int n = 0;
  if (n == 0) {
    int dev = 0, v = 0;
    if (hipGetDevice(&dev) == hipSuccess &&
        hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess)
      n = v;
  }
  return n > 0 ? n : 256;
}

// Grid of the decode kernel: one workgroup per CU (all resident), which must
// cover the R_ff h row blocks and the R_m * S down units; 0 if it cannot.
int decode_grid(int R_ff, int R_m, int S) {
  const int cus = num_cus();
  if (R_ff > cus || R_m * S > cus || cus > 4095) return 0;
  return cus;
}

// Slot ranges per down row: at most 8 slots each (one per wave), and as many
// ranges as the CUs allow so that the down weights spread over the grid.
int decode_splits(int Kd, int R_m) {
  if (Kd <= 0 || R_m <= 0) return 1;
  int S = (Kd + 7) / 8;
  const int fit = num_cus() / R_m;
  if (fit > S) S = fit < Kd ? fit : Kd;
  return S;
}

int launch_decode(int B, const DecodeArgs& a, int grid, hipStream_t st) {
  if (a.N == 0) return 0;
  if (grid <= 0 || grid < a.R_m * a.S || grid < a.R_ff) return -2;
  switch (B) {
    case 16: hipLaunchKernelGGL(decode_kernel<16>, dim3(grid), dim3(512), 0, st, a); break;
    case 32: hipLaunchKernelGGL(decode_kernel<32>, dim3(grid), dim3(512), 0, st, a); break;
    case 64: hipLaunchKernelGGL(decode_kernel<64>, dim3(grid), dim3(512), 0, st, a); break;
    default: return -2;
  }
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace lbk
