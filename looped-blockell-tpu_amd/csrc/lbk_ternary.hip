// lbk_ternary.hip — int8 / ternary kernels for gfx950.
//
// Ternary Block-ELL product (weights {-1,0,+1}, one fp32 scale per block,
// int8 activations with a per-token scale):
//   P[n,r,k,j] = sum_i xq[n, col[r,k]*B + i] * t[r,k,i,j]          (int32, exact)
//   y[n, r*B+j] = sx[n] * sum_k s[r,k] * P[n,r,k,j]
// The per-block scale forces one scaling step per output element per block.
// On gfx950 a wave64 VALU op costs as much issue time as ~1/2 of the int8 MFMA
// work of one 64-deep block for one output, so the scale is applied as an
// integer multiply-add: each block row r uses m[r,k] = rint(s[r,k] * 2^e[r])
// with e[r] chosen so that sum_k m*P cannot overflow int32 for any int8 input;
// acc = sum_k m[r,k] * P  (v_mad_i32_i24), and finally
// y = f32(f32(acc) * 2^-e[r]) * sx[n].  The int32 partials P are exact and can
// be exported; the scale is carried with >= 13 bits of relative precision.
//
// The 2-bit weights are unpacked in registers right before the MFMA: a packed
// word holds 16 consecutive input indices of one output column, laid out so
// that (word >> 2q) & 0x03030303 gives 4 codes in 4 bytes, and one v_perm
// against a constant table turns the codes into int8 {0, +1, -1}.
#include "lbk_device.h"
#include "lbk_internal.h"
#include "lbk_tern_device.h"

namespace lbk {

// ---------------------------------------------------------------------------
// per-token absmax int8 quantisation: one wave per row
// ---------------------------------------------------------------------------
// one wave per row: rows of at most 512 * QA_REG values are read once into registers (all loads
// issued before the reduction), longer rows in two passes
constexpr int QA_REG = 8;

__device__ __forceinline__ u32x2 quantize8(const u32x4& v, float scale) {
  uint32_t packed[2] = {0u, 0u};
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const float a = fminf(fmaxf(rintf(__fmul_rn(bf_lo(v[u]), scale)), -128.f), 127.f);
    const float b = fminf(fmaxf(rintf(__fmul_rn(bf_hi(v[u]), scale)), -128.f), 127.f);
    const uint32_t qa = (uint32_t)((int)a) & 0xffu, qb = (uint32_t)((int)b) & 0xffu;
    packed[u >> 1] |= (qa | (qb << 8)) << (16 * (u & 1));
  }
  return u32x2{packed[0], packed[1]};
}

__device__ __forceinline__ float absmax8(const u32x4& v, float amax) {
#pragma unroll
  for (int u = 0; u < 4; ++u) amax = fmaxf(amax, fmaxf(fabsf(bf_lo(v[u])), fabsf(bf_hi(v[u]))));
  return amax;
}

__global__ __launch_bounds__(256) void quantize_act_kernel(const uint16_t* __restrict__ x, int64_t N, int F,
                                                           int64_t ldx, int8_t* __restrict__ xq,
                                                           float* __restrict__ sx) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= N) return;
  const uint16_t* xr = x + row * ldx;
  int8_t* qr = xq + row * (int64_t)F;
  float amax = 0.f;
  if (F <= 512 * QA_REG) {
    u32x4 v[QA_REG];
#pragma unroll
    for (int u = 0; u < QA_REG; ++u) {
      const int c = 8 * lane + 512 * u;
      v[u] = c < F ? *reinterpret_cast<const u32x4*>(xr + c) : u32x4{0, 0, 0, 0};
    }
#pragma unroll
    for (int u = 0; u < QA_REG; ++u) amax = absmax8(v[u], amax);
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o, 64));
    amax = fmaxf(amax, 1e-8f);
    const float scale = __fdiv_rn(128.0f, amax);
#pragma unroll
    for (int u = 0; u < QA_REG; ++u) {
      const int c = 8 * lane + 512 * u;
      if (c < F) *reinterpret_cast<u32x2*>(qr + c) = quantize8(v[u], scale);
    }
  } else {
    for (int c = 8 * lane; c < F; c += 512) amax = absmax8(*reinterpret_cast<const u32x4*>(xr + c), amax);
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o, 64));
    amax = fmaxf(amax, 1e-8f);
    const float scale = __fdiv_rn(128.0f, amax);
    for (int c = 8 * lane; c < F; c += 512)
      *reinterpret_cast<u32x2*>(qr + c) = quantize8(*reinterpret_cast<const u32x4*>(xr + c), scale);
  }
  if (lane == 0) sx[row] = amax * 0.0078125f;
}

// ---------------------------------------------------------------------------
// pack int8 {-1,0,1} tiles [R,K,B_in,B_out] -> words [R,K,B_out,B_in/16]
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void pack_ternary_kernel(const int8_t* __restrict__ t, int64_t nwords, int B,
                                                           uint32_t* __restrict__ packed) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= nwords) return;
  const int E = B / 16;
  const int e = (int)(idx % E);
  const int D = (int)((idx / E) % B);
  const int64_t blk = idx / ((int64_t)E * B);
  const int8_t* tile = t + blk * B * B;
  uint32_t w = 0;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const uint32_t code = (uint32_t)tile[(16 * e + i) * B + D] & 3u;
    w |= code << (8 * (i & 3) + 2 * (i >> 2));
  }
  packed[idx] = w;
}

// ---------------------------------------------------------------------------
// per-block absmean ternary quantisation of bf16 latent weights -> packed + scales
// one workgroup per block
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void ternary_quantize_weights_kernel(const uint16_t* __restrict__ values, int B,
                                                                       uint32_t* __restrict__ packed,
                                                                       float* __restrict__ scales) {
  __shared__ float part[256];
  const int64_t blk = blockIdx.x;
  const uint16_t* tile = values + blk * B * B;
  const int n = B * B;
  float s = 0.f;
  for (int e = threadIdx.x; e < n; e += 256) s += fabsf(bf2f(tile[e]));
  part[threadIdx.x] = s;
  __syncthreads();
  for (int o = 128; o >= 1; o >>= 1) {
    if ((int)threadIdx.x < o) part[threadIdx.x] += part[threadIdx.x + o];
    __syncthreads();
  }
  const float mean = fmaxf(__fdiv_rn(part[0], (float)n), 1e-8f);
  if (threadIdx.x == 0) scales[blk] = mean;
  const int E = B / 16;
  for (int widx = threadIdx.x; widx < B * E; widx += 256) {
    const int D = widx / E, e = widx - D * E;
    uint32_t w = 0;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const float q = fminf(fmaxf(rintf(__fdiv_rn(bf2f(tile[(16 * e + i) * B + D]), mean)), -1.f), 1.f);
      const uint32_t code = (uint32_t)((int)q) & 3u;
      w |= code << (8 * (i & 3) + 2 * (i >> 2));
    }
    packed[blk * B * E + widx] = w;
  }
}

// ---------------------------------------------------------------------------
// ternary product, rowblock style: workgroup = 64 tokens x one block row
// ---------------------------------------------------------------------------
template <int B> struct TernShape;
template <> struct TernShape<16> { static constexpr int NM = 1; };
template <> struct TernShape<32> { static constexpr int NM = 2; };
template <> struct TernShape<64> { static constexpr int NM = 4; };

// B fragment of one 16-column sub-tile m for lane (j, g)
template <int B>
__device__ __forceinline__ void load_tfrag(const uint32_t* __restrict__ tile, int m, int j, int g, i32x4& b64,
                                           long& b32) {
  if constexpr (B == 64) {
    const uint32_t w = tile[(16 * m + j) * 4 + g];
    b64 = i32x4{(int)unpack4(w, 0), (int)unpack4(w, 1), (int)unpack4(w, 2), (int)unpack4(w, 3)};
  } else if constexpr (B == 32) {
    const uint32_t w = tile[(16 * m + j) * 2 + (g >> 1)];
    const int q0 = 2 * (g & 1);
    b32 = (long)((uint64_t)unpack4(w, q0) | ((uint64_t)unpack4(w, q0 + 1) << 32));
  } else {
    if (g < 2) {
      const uint32_t w = tile[j];
      b32 = (long)((uint64_t)unpack4(w, 2 * g) | ((uint64_t)unpack4(w, 2 * g + 1) << 32));
    } else {
      b32 = 0;
    }
  }
}

template <int B, int MODE>
__global__ __launch_bounds__(256) void ternary_rowblock_kernel(TernaryLaunch a) {
  constexpr int NM = TernShape<B>::NM;
  constexpr int NL = (MODE == 1) ? 2 : 1;
  const int lane = threadIdx.x & 63;
  const int w = uniform(threadIdx.x >> 6);
  const int r = blockIdx.y;
  const int64_t t0 = (int64_t)blockIdx.x * 64 + 16 * w;
  const int i = lane & 15, g = lane >> 4;
  const int64_t my_tok = t0 + i;
  const bool tok_ok = my_tok < a.N;
  const int8_t* xrow = a.xq + (tok_ok ? my_tok : 0) * (int64_t)a.C * B;

  int32_t acc[NL][NM][4];
#pragma unroll
  for (int l = 0; l < NL; ++l)
#pragma unroll
    for (int m = 0; m < NM; ++m)
#pragma unroll
      for (int v = 0; v < 4; ++v) acc[l][m][v] = 0;
  float mult[NL];

#pragma unroll
  for (int l = 0; l < NL; ++l) {
    const uint32_t* pk = (l == 0) ? a.p0 : a.p1;
    const float* sc = (l == 0) ? a.s0 : a.s1;
    const int32_t* cols = (l == 0) ? a.c0 : a.c1;
    const int K = (l == 0) ? a.K0 : a.K1;
    const RowFix fx = row_fixed_point<B>(sc + (int64_t)r * K, cols + (int64_t)r * K, K, a.C);
    mult[l] = fx.mult;
    for (int k = 0; k < K; ++k) {
      const int col = uniform(cols[(int64_t)r * K + k]);
      const bool live = col >= 0 && col < a.C;
      if (!live) {
        if (MODE == 0 && a.partials) {
          // dead slot: partials are zero
#pragma unroll
          for (int m = 0; m < NM; ++m)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
              const int64_t t = t0 + 4 * g + v;
              if (t < a.N) a.partials[((t * a.R + r) * K + k) * B + 16 * m + i] = 0;
            }
        }
        continue;
      }
      const int mk = (int)rintf(ldexpf(sc[(int64_t)r * K + k], fx.e));
      const uint32_t* tile = pk + ((int64_t)r * K + k) * (B * B / 16);
      i32x4 a64 = {0, 0, 0, 0};
      long a32 = 0;
      if (tok_ok) {
        if constexpr (B == 64) {
          a64 = *reinterpret_cast<const i32x4*>(xrow + (int64_t)col * B + 16 * g);
        } else if constexpr (B == 32) {
          a32 = *reinterpret_cast<const long*>(xrow + (int64_t)col * B + 8 * g);
        } else {
          if (g < 2) a32 = *reinterpret_cast<const long*>(xrow + (int64_t)col * B + 8 * g);
        }
      }
#pragma unroll
      for (int m = 0; m < NM; ++m) {
        i32x4 b64 = {0, 0, 0, 0};
        long b32 = 0;
        load_tfrag<B>(tile, m, i, g, b64, b32);
        i32x4 P;
        if constexpr (B == 64) P = mfma_i8_k64(a64, b64, i32x4{0, 0, 0, 0});
        else P = mfma_i8_k32(a32, b32, i32x4{0, 0, 0, 0});
        if (MODE == 0 && a.partials) {
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const int64_t t = t0 + 4 * g + v;
            if (t < a.N) a.partials[((t * a.R + r) * K + k) * B + 16 * m + i] = P[v];
          }
        }
#pragma unroll
        for (int v = 0; v < 4; ++v) acc[l][m][v] = __mul24(P[v], mk) + acc[l][m][v];
      }
    }
  }

  // epilogue: lane (j = i, g) owns rows 4g+v, columns 16m + j
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int64_t t = t0 + 4 * g + v;
    if (t >= a.N) continue;
    const float s_tok = a.sx[t];
#pragma unroll
    for (int m = 0; m < NM; ++m) {
      const int64_t oc = (int64_t)r * B + 16 * m + i;
      const int64_t yo = t * (int64_t)a.R * B + oc;
      float o;
      if constexpr (MODE == 1) {
        const float gv = __fmul_rn(__fmul_rn((float)acc[0][m][v], mult[0]), s_tok);
        const float uv = __fmul_rn(__fmul_rn((float)acc[1][m][v], mult[1]), s_tok);
        if (a.acc0) {
          a.acc0[yo] = acc[0][m][v];
          a.acc1[yo] = acc[1][m][v];
        }
        if (a.pre0) {
          a.pre0[yo] = gv;
          a.pre1[yo] = uv;
        }
        o = silu_f(gv) * uv;
      } else {
        o = __fmul_rn(__fmul_rn((float)acc[0][m][v], mult[0]), s_tok);
        if (a.acc0) a.acc0[yo] = acc[0][m][v];
        if (a.pre0) a.pre0[yo] = o;
        if (a.resid) o += bf2f(a.resid[yo]);
      }
      a.y[yo] = f2bf(o);
    }
  }
}

__global__ __launch_bounds__(256) void check_columns_kernel(const int32_t* __restrict__ col, int64_t count, int C,
                                                            int32_t* __restrict__ bad) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= count) return;
  const int c = col[idx];
  if (c < -1 || c >= C) atomicAdd(bad, 1);
}

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------
int launch_quantize_act(const uint16_t* x, int64_t N, int F, int64_t ldx, int8_t* xq, float* sx, hipStream_t st) {
  if (N == 0) return 0;
  hipLaunchKernelGGL(quantize_act_kernel, dim3((unsigned)((N + 3) / 4)), dim3(256), 0, st, x, N, F, ldx, xq, sx);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_pack_ternary(const int8_t* t, int R, int K, int B, uint32_t* packed, hipStream_t st) {
  const int64_t nwords = (int64_t)R * K * B * (B / 16);
  if (nwords == 0) return 0;
  hipLaunchKernelGGL(pack_ternary_kernel, dim3((unsigned)((nwords + 255) / 256)), dim3(256), 0, st, t, nwords, B,
                     packed);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_ternary_quantize_weights(const uint16_t* values, int R, int K, int B, uint32_t* packed, float* scales,
                                    hipStream_t st) {
  const int64_t nblk = (int64_t)R * K;
  if (nblk == 0) return 0;
  hipLaunchKernelGGL(ternary_quantize_weights_kernel, dim3((unsigned)nblk), dim3(256), 0, st, values, B, packed,
                     scales);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

template <int B, int MODE>
static int launch_tern_t(const TernaryLaunch& a, hipStream_t st) {
  dim3 grid((unsigned)((a.N + 63) / 64), (unsigned)a.R);
  hipLaunchKernelGGL((ternary_rowblock_kernel<B, MODE>), grid, dim3(256), 0, st, a);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_ternary(int B, int mode, const TernaryLaunch& a, hipStream_t st) {
  if (a.N == 0 || a.R == 0) return 0;
  if (a.R > 65535 || (a.N + 63) / 64 > 0x7fffffff) return -3;  // grid limits
#define LBK_TR(BB)                                          \
  if (B == BB) return mode == 1 ? launch_tern_t<BB, 1>(a, st) : launch_tern_t<BB, 0>(a, st);
  LBK_TR(16)
  LBK_TR(32)
  LBK_TR(64)
#undef LBK_TR
  return -2;
}

// clears the counter with a kernel (a memset node recorded into a captured graph is avoided)
__global__ __launch_bounds__(64) void zero_counter_kernel(int32_t* __restrict__ p) {
  if (threadIdx.x == 0) p[0] = 0;
}

int launch_check_columns(const int32_t* col, int64_t count, int C, int32_t* bad, hipStream_t st) {
  hipLaunchKernelGGL(zero_counter_kernel, dim3(1), dim3(64), 0, st, bad);
  if (hipGetLastError() != hipSuccess) return -1;
  if (count == 0) return 0;
  hipLaunchKernelGGL(check_columns_kernel, dim3((unsigned)((count + 255) / 256)), dim3(256), 0, st, col, count, C,
                     bad);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace lbk
