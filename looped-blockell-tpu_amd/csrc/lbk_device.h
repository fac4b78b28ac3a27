// lbk_device.h — device-side building blocks shared by the gfx950 kernels.
//
// MFMA fragment conventions (v_mfma_f32_16x16x32_bf16; every kernel's GPU parity test
// exercises them end to end):
//   A (16 x 32, M x K): lane l holds row l%16, k = 8*(l/16) .. +7  (8 bf16)
//   B (32 x 16, K x N): lane l holds col l%16, k = 8*(l/16) .. +7
//   C (16 x 16):        lane l holds col l%16, rows 4*(l/16) + v, v = 0..3
// A and B only need the same k assignment, so any k permutation shared by both
// operands gives the same product.
//
// Weight tiles arrive as [B_in, B_out] (output index contiguous), but the B
// operand wants 8 consecutive *input* indices per lane.  load_wraw/wraw_to_frag
// transpose in registers: with CW = B/16 output columns per lane, lane (j, g)
// loads the CW contiguous outputs CW*j .. CW*j+CW-1 of 8 consecutive input
// rows, then v_perm splits them into CW fragments.  Fragment m of a lane then
// carries output column CW*j + m, so a tile of B outputs is covered by CW
// MFMAs whose column n maps to output CW*n + m, and after the MFMAs every lane
// owns CW *contiguous* outputs per row — which makes the stores contiguous.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace lbk {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

__device__ __forceinline__ float bf2f(uint32_t b16) { return __uint_as_float(b16 << 16); }
__device__ __forceinline__ float bf_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// Round-to-nearest-even float -> bf16 (hardware v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ uint32_t pack2_bf16(float lo, float hi) {
  bf16x2_t v = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, v);
}
__device__ __forceinline__ uint16_t f2bf(float f) {
  __bf16 h = (__bf16)f;
  return __builtin_bit_cast(uint16_t, h);
}

__device__ __forceinline__ f32x4 mfma_bf16(const u32x4& a, const u32x4& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

// 16x16x16 bf16: lane (n, q), n = lane % 16, q = lane / 16, holds k = 4q .. 4q + 3 (8 bytes) of
// row n of A and column n of B; D has the layout of the 16x16x32 form.  A B = 16 tile's K fits
// exactly, with no zero half to mask.
typedef short s16x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ f32x4 mfma_bf16_k16(const u32x2& a, const u32x2& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4_t, a),
                                                   __builtin_bit_cast(s16x4_t, b), c, 0, 0, 0);
}

// int8 MFMAs: 16x16x64 (16 bytes of K per lane) and 16x16x32 (8 bytes).
__device__ __forceinline__ i32x4 mfma_i8_k64(const i32x4& a, const i32x4& b, const i32x4& c) {
  return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ i32x4 mfma_i8_k32(long a, long b, const i32x4& c) {
  return __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float silu_f(float z) {
  // z * sigmoid(z) = z / (1 + exp(-z)); exp via the hardware exp2.
  return z * __builtin_amdgcn_rcpf(1.0f + __expf(-z));
}

// Wave-uniform value (forces scalar registers / scalar branches).
__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

// ---------------------------------------------------------------------------
// Weight tiles: raw transposing loads and conversion to B fragments.
// NKS = number of 32-deep k-steps per tile, CW = output columns per lane.
// For B = 16 the single k-step is half filled: lanes with g >= 2 carry a zero A
// operand (their B operand repeats lanes g - 2 and is multiplied by zero).
// ---------------------------------------------------------------------------
__device__ __forceinline__ void unpack8_bf16(const u32x4& v, float (&f)[8]) {
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    f[2 * q] = bf_lo(v[q]);
    f[2 * q + 1] = bf_hi(v[q]);
  }
}

// The looped core's injection s = decay * s + dt * e over features c .. c + 7 of the element at
// e0 (coef: decay [d], then dt [d])
__device__ __forceinline__ void inject8(float (&s)[8], const uint16_t* __restrict__ e, const float* __restrict__ coef,
                                        int64_t e0, int c, int d) {
  float ef[8];
  unpack8_bf16(*reinterpret_cast<const u32x4*>(e + e0), ef);
  const f32x4 k0 = *reinterpret_cast<const f32x4*>(coef + c), k1 = *reinterpret_cast<const f32x4*>(coef + c + 4);
  const f32x4 t0 = *reinterpret_cast<const f32x4*>(coef + d + c), t1 = *reinterpret_cast<const f32x4*>(coef + d + c + 4);
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    s[q] = k0[q] * s[q] + t0[q] * ef[q];
    s[4 + q] = k1[q] * s[4 + q] + t1[q] * ef[4 + q];
  }
}

template <int B> struct TileShape;
template <> struct TileShape<16> { static constexpr int NKS = 1, CW = 1; };
template <> struct TileShape<32> { static constexpr int NKS = 1, CW = 2; };
template <> struct TileShape<64> { static constexpr int NKS = 2, CW = 4; };

template <int B> struct WRaw;
template <> struct WRaw<16> { uint32_t v[8]; };       // one bf16 per row (zero-extended)
template <> struct WRaw<32> { uint32_t v[8]; };       // two bf16 per row
template <> struct WRaw<64> { u32x2 v[2][8]; };       // four bf16 per row, per k-step

template <int B>
__device__ __forceinline__ void load_wraw(const uint16_t* __restrict__ tile, int lane, WRaw<B>& r);

// Lanes g >= 2 repeat the rows of lanes g - 2 (every lane issues the same loads,
// so the loop around them needs no branch); their A operand is zero, so these
// duplicates contribute nothing.
template <>
__device__ __forceinline__ void load_wraw<16>(const uint16_t* __restrict__ tile, int lane, WRaw<16>& r) {
  const int j = lane & 15, g = (lane >> 4) & 1;
#pragma unroll
  for (int t = 0; t < 8; ++t) r.v[t] = tile[(8 * g + t) * 16 + j];
}
template <>
__device__ __forceinline__ void load_wraw<32>(const uint16_t* __restrict__ tile, int lane, WRaw<32>& r) {
  const int j = lane & 15, g = lane >> 4;
  const uint32_t* p = reinterpret_cast<const uint32_t*>(tile) + (8 * g) * 16 + j;
#pragma unroll
  for (int t = 0; t < 8; ++t) r.v[t] = p[t * 16];
}
template <>
__device__ __forceinline__ void load_wraw<64>(const uint16_t* __restrict__ tile, int lane, WRaw<64>& r) {
  const int j = lane & 15, g = lane >> 4;
  const u32x2* p = reinterpret_cast<const u32x2*>(tile) + (8 * g) * 16 + j;
#pragma unroll
  for (int s = 0; s < 2; ++s)
#pragma unroll
    for (int t = 0; t < 8; ++t) r.v[s][t] = p[(32 * s + t) * 16];
}

// f[ks][m]: fragment for k-step ks and output sub-column m.
template <int B>
__device__ __forceinline__ void wraw_to_frag(const WRaw<B>& r, u32x4 (&f)[TileShape<B>::NKS][TileShape<B>::CW]);

template <>
__device__ __forceinline__ void wraw_to_frag<16>(const WRaw<16>& r, u32x4 (&f)[1][1]) {
#pragma unroll
  for (int u = 0; u < 4; ++u) f[0][0][u] = r.v[2 * u] | (r.v[2 * u + 1] << 16);
}
template <>
__device__ __forceinline__ void wraw_to_frag<32>(const WRaw<32>& r, u32x4 (&f)[1][2]) {
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    f[0][0][u] = __builtin_amdgcn_perm(r.v[2 * u + 1], r.v[2 * u], 0x05040100u);
    f[0][1][u] = __builtin_amdgcn_perm(r.v[2 * u + 1], r.v[2 * u], 0x07060302u);
  }
}
template <>
__device__ __forceinline__ void wraw_to_frag<64>(const WRaw<64>& r, u32x4 (&f)[2][4]) {
#pragma unroll
  for (int s = 0; s < 2; ++s)
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const u32x2 a = r.v[s][2 * u], b = r.v[s][2 * u + 1];
      f[s][0][u] = __builtin_amdgcn_perm(b[0], a[0], 0x05040100u);
      f[s][1][u] = __builtin_amdgcn_perm(b[0], a[0], 0x07060302u);
      f[s][2][u] = __builtin_amdgcn_perm(b[1], a[1], 0x05040100u);
      f[s][3][u] = __builtin_amdgcn_perm(b[1], a[1], 0x07060302u);
    }
}

// ---------------------------------------------------------------------------
// Fragment-major ("packed") bf16 tiles.  Tile t holds the B fragments f[ks][m]
// (as wraw_to_frag would build them) of every lane l of a wave as 16-byte
// chunks, chunk-major: packed[(t*NKS*CW + ks*CW + m)*LANES + l].  A lane then
// fetches all its operands of a tile with NKS*CW dwordx4 loads, each of which
// reads one contiguous LANES*16-byte run across the wave, and no register
// transposition is needed.  For B = 16 only lanes 0..31 are stored (512 bytes
// per tile); lanes 32..63 read lanes 0..31 (their A operand is zero).
// Dword u of chunk (ks, m) of lane (j = l%16, g = l/16) is
//   W[k][c] | W[k+1][c] << 16,  k = 32*ks + 8*g + 2*u,  c = CW*j + m
// (gate/up tiles for B = 32: c = 8*(j/4) + 4*m + j%4, see the gate/up kernel).
// ---------------------------------------------------------------------------
template <int B>
struct PackedTile {
  static constexpr int CHUNKS = TileShape<B>::NKS * TileShape<B>::CW;   // 16-byte chunks per lane
  static constexpr int LANES = B == 16 ? 32 : 64;                       // lanes stored per tile
  static constexpr int U32X4 = LANES * CHUNKS;                          // chunks per tile
};

// Byte offset, within a packed B = 16 tile, of the 8-byte 16x16x16 fragment of `lane`: stored
// lane l' (row l' % 16, k = 8 (l' / 16) .. + 7) holds k = 4q .. 4q + 3 of row n at byte
// 16 l' + 8 (q & 1), l' = n + 16 (q >> 1).
__device__ __forceinline__ uint32_t pfrag16_off(int lane) {
  return (uint32_t)((lane & 15) * 16 + (lane >> 5) * 256 + ((lane >> 4) & 1) * 8);
}
__device__ __forceinline__ u32x2 load_pfrag16(const u32x4* __restrict__ tile, uint32_t off) {
  return *reinterpret_cast<const u32x2*>(reinterpret_cast<const unsigned char*>(tile) + off);
}

template <int B>
__device__ __forceinline__ void load_pfrag(const u32x4* __restrict__ tile, int lane,
                                           u32x4 (&f)[TileShape<B>::NKS][TileShape<B>::CW]) {
  constexpr int NKS = TileShape<B>::NKS, CW = TileShape<B>::CW, LANES = PackedTile<B>::LANES;
  const u32x4* p = tile + (B == 16 ? (lane & 31) : lane);
#pragma unroll
  for (int ks = 0; ks < NKS; ++ks)
#pragma unroll
    for (int m = 0; m < CW; ++m) f[ks][m] = p[(ks * CW + m) * LANES];
}

// ---------------------------------------------------------------------------
// A fragments.  Row pointer `row` points at element (token, column-block
// start); ks selects the 32-deep k-step.  For B = 16, lanes g >= 2 carry zeros.
// ---------------------------------------------------------------------------
template <int B>
__device__ __forceinline__ u32x4 load_afrag(const uint16_t* row, int ks, int g) {
  if (B == 16 && g >= 2) return u32x4{0, 0, 0, 0};
  return *reinterpret_cast<const u32x4*>(row + 32 * ks + 8 * g);
}

// Store CW contiguous bf16 values.
template <int CW>
__device__ __forceinline__ void store_bf16(uint16_t* p, const float (&v)[CW]);
template <>
__device__ __forceinline__ void store_bf16<1>(uint16_t* p, const float (&v)[1]) { *p = f2bf(v[0]); }
template <>
__device__ __forceinline__ void store_bf16<2>(uint16_t* p, const float (&v)[2]) {
  *reinterpret_cast<uint32_t*>(p) = pack2_bf16(v[0], v[1]);
}
template <>
__device__ __forceinline__ void store_bf16<4>(uint16_t* p, const float (&v)[4]) {
  u32x2 w = {pack2_bf16(v[0], v[1]), pack2_bf16(v[2], v[3])};
  *reinterpret_cast<u32x2*>(p) = w;
}

// Store NV (4 or 8) consecutive bf16 values with one 8- or 16-byte store.
template <int NV>
__device__ __forceinline__ void store_bf16x(uint16_t* p, const float (&v)[NV]) {
  if constexpr (NV == 8) {
    *reinterpret_cast<u32x4*>(p) = u32x4{pack2_bf16(v[0], v[1]), pack2_bf16(v[2], v[3]), pack2_bf16(v[4], v[5]),
                                         pack2_bf16(v[6], v[7])};
  } else {
    static_assert(NV == 4, "4 or 8 values");
    *reinterpret_cast<u32x2*>(p) = u32x2{pack2_bf16(v[0], v[1]), pack2_bf16(v[2], v[3])};
  }
}

// Load NV (4 or 8) consecutive bf16 values as floats with one 8- or 16-byte load.
template <int NV>
__device__ __forceinline__ void load_bf16x(const uint16_t* p, float (&v)[NV]) {
  if constexpr (NV == 8) {
    const u32x4 w = *reinterpret_cast<const u32x4*>(p);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      v[2 * u] = bf_lo(w[u]);
      v[2 * u + 1] = bf_hi(w[u]);
    }
  } else {
    static_assert(NV == 4, "4 or 8 values");
    const u32x2 w = *reinterpret_cast<const u32x2*>(p);
    v[0] = bf_lo(w[0]);
    v[1] = bf_hi(w[0]);
    v[2] = bf_lo(w[1]);
    v[3] = bf_hi(w[1]);
  }
}

// Load CW contiguous bf16 values as floats.
template <int CW>
__device__ __forceinline__ void load_bf16(const uint16_t* p, float (&v)[CW]);
template <>
__device__ __forceinline__ void load_bf16<1>(const uint16_t* p, float (&v)[1]) { v[0] = bf2f(*p); }
template <>
__device__ __forceinline__ void load_bf16<2>(const uint16_t* p, float (&v)[2]) {
  const uint32_t w = *reinterpret_cast<const uint32_t*>(p);
  v[0] = bf_lo(w);
  v[1] = bf_hi(w);
}
template <>
__device__ __forceinline__ void load_bf16<4>(const uint16_t* p, float (&v)[4]) {
  const u32x2 w = *reinterpret_cast<const u32x2*>(p);
  v[0] = bf_lo(w[0]);
  v[1] = bf_hi(w[0]);
  v[2] = bf_lo(w[1]);
  v[3] = bf_hi(w[1]);
}

typedef short i16x4 __attribute__((ext_vector_type(4)));

// ds_read_b64_tr_b16: within each 16-lane group, lane l receives element l % 4 of the 64-bit
// blocks read by lanes l / 4, 4 + l / 4, 8 + l / 4 and 12 + l / 4 of the group (measured on
// gfx950).  So if lane s of a group points at row t0 + s / 4, columns c0 + 4 (s % 4) .. + 3 of a
// row-major [row][column] bf16 slice in LDS, lane l gets column c0 + l of rows t0 .. t0 + 3: two
// such reads give the 8 consecutive rows (the MFMA's k) of one column that an operand lane
// holds (lane group g takes rows t0 + 8 g .. t0 + 8 g + 7).
__device__ __forceinline__ u32x4 tr_frag(const uint16_t* slice, int rowlen, int t0, int c0, int lane) {
  const int s = lane & 15, g = lane >> 4;
  const uint16_t* p = slice + (t0 + 8 * g + (s >> 2)) * rowlen + c0 + 4 * (s & 3);
  typedef __attribute__((address_space(3))) i16x4 lds_i16x4;
  const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p));
  const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p + 4 * rowlen));
  const u32x2 a = __builtin_bit_cast(u32x2, lo), b = __builtin_bit_cast(u32x2, hi);
  return u32x4{a[0], a[1], b[0], b[1]};
}

}  // namespace lbk
