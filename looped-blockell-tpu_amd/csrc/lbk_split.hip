// lbk_split.hip — the SwiGLU FFN as two register-lean kernels (gfx950, bf16 MFMA).
//
// gu_kernel<B, MT, NORM, INTER>: a workgroup owns 16*MT tokens.  Their input
// rows sit in LDS as an XOR-swizzled panel (optionally RMSNorm-ed on the way in
// from an fp32 state), next to a table of the gate/up column indices.  Eight
// waves (two per SIMD; gu_kernel_w12, for distinct gate/up topologies with no exports and no
// biases, runs twelve with a shallower ring at B = 32 and sixteen at B = 16) each stream their
// own d_ff block rows (r = w, w+8, ...):
// gate and up tiles are consumed in (gate k, up k) pairs from a GU_RING-deep
// register ring that runs across row boundaries.  The weight tile is the A
// operand of the MFMA, so the accumulators hold h transposed and every lane
// stores 8 (B = 32) or 4 (B = 16) consecutive columns of one token at once.  B = 16 uses the
// 16x16x16 MFMA (a 16-deep tile fills its K), B = 32 the 16x16x32 one.  Weights come pre-packed in
// fragment-major order (two dwordx4 loads per lane per B = 32 tile); every
// position issues the same loads (padding and dead slots read the packed zero
// tile), so the compiler's memory-counter waits stay exact.  h = silu(g) * u is
// stored as bf16 (and the pre-activations when INTER).
//
// dn_kernel<B, MT, RPW>: a workgroup of DN_WAVES = 16 waves owns 16*MT tokens
// and a group of 16*RPW down block rows (RPW = 1 as launched: wave w keeps the
// fp32 accumulators of one row in registers for the whole kernel).  The row
// groups of one token block are dealt to one XCD, so the h tiles they all read
// come from that XCD's L2 after the first group's miss.  h is staged through
// LDS 512 columns at a time (double buffered, next stage's global loads in
// flight while the current one is consumed).  Per stage each wave builds a flat list of its tiles (ballot over
// its column-index rows, ds_permute into place), rows in order, each row's run
// padded to an even length with a zero-tile entry, and streams it through a
// two-slot ring that also prefetches the next stage's first tiles.  The
// epilogue adds the residual, or carries an fp32 state for the looped block.
//
// dnf_kernel<B, D>: the plain forward's down kernel at B = 32 on 64-token blocks: the same
// workgroup and stages, but each wave streams its row through a D-slot ring across the stages
// (no pair padding, stage changes taken inline); see its comment.
#include "lbk_device.h"
#include "lbk_internal.h"

namespace lbk {

__device__ __forceinline__ u32x4 lds16(const unsigned char* base, uint32_t off) {
  return *reinterpret_cast<const u32x4*>(base + off);
}

// ===========================================================================
// gate/up
// ===========================================================================
// Panel layout shared by the kernels here: token row 16*mt + i of a tile of
// 16*MT rows is stored at row slot i*MT + mt (so the MT rows a lane reads are
// ROWB apart and fit the ds_read immediate offset), and 16-byte chunk c of it
// at chunk c ^ i (i = row & 15), which keeps the eight lanes of one LDS read
// phase on distinct banks.
template <int MT>
__device__ __forceinline__ uint32_t panel_addr(int row, int chunk, int rowb) {
  const int i = row & 15, mt = row >> 4;
  return (uint32_t)((i * MT + mt) * rowb + ((chunk ^ i) << 4));
}

// One ring slot: the gate and up fragments of one stream position and their
// input column blocks (dead slots point at the packed zero tile and column 0).
template <int B>
struct GUSlot {
  u32x4 g[1][TileShape<B>::CW], u[1][TileShape<B>::CW];
  int cg, cu;
};
// B = 16: the 8-byte fragments of the 16x16x16 form
template <>
struct GUSlot<16> {
  u32x2 g, u;
  int cg, cu;
};
// B = 16 with one panel stream (a shared gate/up topology, or the plain product): a position is
// a pair of slots (2p, 2p + 1) of a row, one 16x16x32 MFMA per product.  Lanes g < 2 hold
// k = 8 (g & 1) .. + 7 of slot 2p's tile, lanes g >= 2 those of slot 2p + 1's (the packed B = 16
// tile stores exactly these 16-byte pieces); cg / cu hold the two slots' gate / up column blocks
// in bytes 0 and 1.  With two panel streams the panel reads, not the MFMAs, bound the kernel
// (16 eight-byte reads per 8 MFMAs), and the pairs measured slower there.
struct GUSlotPair {
  u32x4 g, u;
  int cg, cu;
};

__device__ __forceinline__ u32x2 lds8(const unsigned char* base, uint32_t off) {
  return *reinterpret_cast<const u32x2*>(base + off);
}
// panel byte address of lane (i, g)'s 16x16x16 B = 16 fragment of column block cb (k = 4g .. 4g + 3
// of the block: 16-byte chunk 2 cb + g / 2, its half g & 1)
__device__ __forceinline__ uint32_t k16_addr(uint32_t lbase, int cb, int g, int i) {
  return lbase + ((uint32_t)(((cb * 2 + (g >> 1)) ^ i) << 4) | (uint32_t)((g & 1) << 3));
}
// the same in a stage whose rows with (i & 8) hold their chunk halves swapped: the 16 lanes
// i = 0 .. 15 of one 8-byte read then fall on 16 different bank pairs (with the chunk XOR alone,
// lanes i and i + 8 share them)
__device__ __forceinline__ uint32_t k16s_addr(uint32_t lbase, int cb, int g, int i) {
  return lbase + ((uint32_t)(((cb * 2 + (g >> 1)) ^ i) << 4) | (uint32_t)(((g & 1) ^ ((i >> 3) & 1)) << 3));
}
// a 16-byte chunk of token row `row` as the B = 16 layouts store it (halves swapped when row & 8)
template <int B>
__device__ __forceinline__ u32x4 k16s_chunk(const u32x4& v, int row) {
  if constexpr (B == 16) return (row & 8) ? u32x4{v[2], v[3], v[0], v[1]} : v;
  else return v;
}

// gate/up ring depth (positions in flight + 1)
constexpr int GU_RING = 4;
// column-table entries per thread loaded beside the prologue's other loads (a larger table loads
// the rest in further rounds before the panel barrier)
constexpr int GU_CT_MAX = 8;

// gate/up panel row stride: 2048 bytes (MT = 4, d_model <= 1024) or 4096 (MT = 2)
template <int MT>
struct GUPanel { static constexpr int ROWB = 8192 / MT; };

// gate/up of token block tb (16 * MT tokens), h rows r_lo .. r_lo + nrs - 1, by one workgroup of
// 64 * NW threads; smem holds the panel and the slice's column table (gu_lds bytes).  Waves without rows return after the panel
// barrier, so a caller that synchronises afterwards must do so after the call.
// READY: the panel and the column table are already in LDS (the looped kernel's down phase
// wrote the next iteration's normalised rows; the table stays from the first iteration).
// BIAS: add a.bg / a.bu (either may be null) to the pre-activations; without it the epilogue
// has no bias code at all.
// LIN: one plain product y = x W (+ a.bg) into a.h: the gate stream only (the caller passes
// the gate's weights and columns for up too, with SHARED), no SiLU.
// NW, RING: waves of the workgroup and ring depth (12 waves with a 2-deep ring for the plain
// x-panel path, where three waves per SIMD fit the register budget).
template <int B, int MT, bool NORM, bool INTER, bool SHARED, bool READY = false, bool BIAS = false, bool LIN = false,
          int NW = 8, int RING = GU_RING>
__device__ __forceinline__ void gu_tile(const GUArgs& a, int64_t tb, int r_lo, int nrs, unsigned char* smem,
                                        int tid) {
  constexpr int CW = TileShape<B>::CW;
  constexpr int TM = 16 * MT;
  constexpr int ROWB = GUPanel<MT>::ROWB;
  static_assert(TileShape<B>::NKS == 1, "gate/up kernel handles B <= 32");
  constexpr int NT = 64 * NW;
  static_assert(NW == 8 || !READY, "the looped kernel's gate/up phase runs 8 waves");
  const int d_model = a.d_model;
  const int lane = tid & 63;
  const int w = uniform(tid >> 6);
  const int i = lane & 15, g = lane >> 4;
  const int64_t t0 = tb * TM;
  const int cin = d_model / B;
  const int64_t d_ff = (int64_t)a.R_ff * B;
  const int K = a.Kg;                        // == a.Ku >= 1
  const int64_t ztile = (int64_t)a.R_ff * K; // index of the packed zero tile
  // column table after the panel: (gate col, up col) per (row of the slice, slot) as one byte each
  // (d_model <= 2048, so at most 128 input column blocks); dead -> 0
  uint16_t* ctab = reinterpret_cast<uint16_t*>(smem + (size_t)TM * ROWB);

  // ---- column table: the first GU_CT_MAX entries per thread are loaded (at clamped addresses)
  // with the panel loads and stored after them; a larger table loads the rest in further rounds
  const int nct = nrs * K;
  const int64_t cbase = (int64_t)r_lo * K;
  int2 ctv[GU_CT_MAX];
  auto ctab_fetch_at = [&](int base) {
#pragma unroll
    for (int u = 0; u < GU_CT_MAX; ++u) {
      const int e = base + tid + NT * u;
      const int64_t ec = cbase + (e < nct ? e : 0);
      ctv[u] = make_int2(a.cg[ec], a.cu[ec]);
    }
  };
  auto ctab_store_at = [&](int base) {
#pragma unroll
    for (int u = 0; u < GU_CT_MAX; ++u) {
      const int e = base + tid + NT * u;
      int cg = ctv[u].x, cu = ctv[u].y;
      cg = (cg >= 0 && cg < cin) ? cg : 0;
      cu = (cu >= 0 && cu < cin) ? cu : 0;
      if (e < nct) ctab[e] = (uint16_t)(cg | (cu << 8));
    }
  };
  auto ctab_fetch = [&]() { ctab_fetch_at(0); };
  auto ctab_store = [&]() {
    ctab_store_at(0);
    for (int base = NT * GU_CT_MAX; base < nct; base += NT * GU_CT_MAX) {
      ctab_fetch_at(base);
      ctab_store_at(base);
    }
  };

  // ---- stream this wave's rows r = r_lo + w + NW n through a RING-slot ring of
  // (gate, up) tile pairs.  Each row takes KP positions, K rounded up to a
  // multiple of RING (padding positions read the zero tile), so slot s of the
  // ring always holds position s of a group; every position issues the same
  // loads, so the compiler's memory-counter waits stay exact and RING - 1
  // positions stay in flight across row boundaries.
  const int nrows = (nrs - w + NW - 1) / NW;   // may be <= 0: such a wave only helps fill the panel
  constexpr bool PAIR = B == 16 && (SHARED || LIN);
  using Slot = std::conditional_t<PAIR, GUSlotPair, GUSlot<B>>;
  const int KS = PAIR ? (K + 1) / 2 : K;      // positions of a row: slots, or slot pairs
  const int KP = (KS + RING - 1) / RING * RING;
  const u32x4* pg = static_cast<const u32x4*>(a.pg);
  const u32x4* pu = static_cast<const u32x4*>(a.pu);
  const uint32_t lbase = (uint32_t)(i * MT * ROWB);   // this lane's first panel row

  int rn = 0, rk = 0;   // next position to fetch
  // weight loads of the next position (the column table is not needed yet)
  // byte offsets in a packed B = 16 tile of this lane's 8-byte 16x16x16 fragment and (slot pairs)
  // of its 16-byte piece (row i, k = 8 (g & 1) .. + 7)
  const uint32_t f16 = pfrag16_off(lane);
  const uint32_t f32 = (uint32_t)(16 * (i + 16 * (g & 1)));
  auto fetch_w = [&](Slot& S) {
    if constexpr (PAIR) {
      // slots 2 rk and 2 rk + 1 of the row (past the row's slots: the zero tile)
      const int k0 = 2 * rk;
      const bool la = rn < nrows && k0 < K, lb = rn < nrows && k0 + 1 < K;
      const int el = (w + NW * rn) * K + k0;   // entry of the slice's column table
      const int64_t ea = la ? cbase + el : ztile, eb = lb ? cbase + el + 1 : ztile;
      const int64_t e = g < 2 ? ea : eb;
      S.g = *reinterpret_cast<const u32x4*>(reinterpret_cast<const unsigned char*>(pg + e * PackedTile<B>::U32X4) + f32);
      if constexpr (!LIN)
        S.u = *reinterpret_cast<const u32x4*>(reinterpret_cast<const unsigned char*>(pu + e * PackedTile<B>::U32X4) + f32);
      S.cg = la ? el : -1;   // table entries until fetch_c replaces them by columns
      S.cu = lb ? el + 1 : -1;
    } else {
      const bool live = rn < nrows && rk < K;
      const int el = (w + NW * rn) * K + rk;   // entry of the slice's column table
      const int64_t e = live ? cbase + el : ztile;
      if constexpr (B == 16) {
        S.g = load_pfrag16(pg + e * PackedTile<B>::U32X4, f16);
        if constexpr (!LIN) S.u = load_pfrag16(pu + e * PackedTile<B>::U32X4, f16);
      } else {
        load_pfrag<B>(pg + e * PackedTile<B>::U32X4, lane, S.g);
        if constexpr (!LIN) load_pfrag<B>(pu + e * PackedTile<B>::U32X4, lane, S.u);
      }
      S.cg = live ? el : -1;   // table entry until fetch_c replaces it by columns
    }
  };
  auto fetch_c = [&](Slot& S) {
    if constexpr (PAIR) {
      const uint32_t ca = ctab[S.cg >= 0 ? S.cg : 0], cb = ctab[S.cu >= 0 ? S.cu : 0];
      S.cg = (int)((ca & 0xffu) | ((cb & 0xffu) << 8));
      S.cu = (int)((ca >> 8) | ((cb >> 8) << 8));
    } else {
      const uint32_t c = ctab[S.cg >= 0 ? S.cg : 0];
      S.cg = (int)(c & 0xffu);
      S.cu = (int)(c >> 8);
    }
    if (++rk == KP) {
      rk = 0;
      ++rn;
    }
  };
  auto fetch = [&](Slot& S) {
    fetch_w(S);
    fetch_c(S);
  };
  Slot P[RING];
  auto prefetch_ring = [&]() {
    int sn = 0, sk = 0;
#pragma unroll
    for (int sl = 0; sl < RING; ++sl) {
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

  f32x4 ag[MT][CW], au[MT][CW];
  // A fragments of a position's gate and up column blocks (shared topology: gate and up
  // read the same column list, so one panel read feeds both products)
  using AF = std::conditional_t<B == 16 && !PAIR, u32x2, u32x4>;
  struct AFrags {
    AF g[MT], u[SHARED ? 1 : MT];
  };
  auto load_a = [&](const Slot& S, AFrags& A) {
    const int cg = uniform(S.cg), cu = uniform(S.cu);
    if constexpr (B == 16 && !PAIR) {
      const uint32_t ag0 = k16s_addr(lbase, cg, g, i), au0 = k16s_addr(lbase, cu, g, i);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        A.g[mt] = lds8(smem, ag0 + mt * ROWB);
        if constexpr (!SHARED) A.u[mt] = lds8(smem, au0 + mt * ROWB);
      }
    } else if constexpr (PAIR) {
      // lane (i, g): token row i, k = 8 (g & 1) .. + 7 of its slot's column block: the 16-byte
      // chunk 2 c + (g & 1), whose halves rows with (i & 8) store swapped, read as two 8-byte
      // halves in order
      const int lcg = g < 2 ? (cg & 0xff) : (cg >> 8), lcu = g < 2 ? (cu & 0xff) : (cu >> 8);
      const uint32_t sw = (uint32_t)((i >> 3) & 1) << 3;
      const uint32_t ag0 = lbase + ((uint32_t)((lcg * 2 + (g & 1)) ^ i) << 4);
      const uint32_t au0 = lbase + ((uint32_t)((lcu * 2 + (g & 1)) ^ i) << 4);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const u32x2 glo = lds8(smem, ag0 + sw + mt * ROWB), ghi = lds8(smem, ag0 + (sw ^ 8) + mt * ROWB);
        A.g[mt] = u32x4{glo[0], glo[1], ghi[0], ghi[1]};
        if constexpr (!SHARED) {
          const u32x2 ulo = lds8(smem, au0 + sw + mt * ROWB), uhi = lds8(smem, au0 + (sw ^ 8) + mt * ROWB);
          A.u[mt] = u32x4{ulo[0], ulo[1], uhi[0], uhi[1]};
        }
      }
    } else {
      const uint32_t ag0 = lbase + (((cg * (B / 8) + g) ^ i) << 4);
      const uint32_t au0 = lbase + (((cu * (B / 8) + g) ^ i) << 4);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        A.g[mt] = lds16(smem, ag0 + mt * ROWB);
        if constexpr (!SHARED) A.u[mt] = lds16(smem, au0 + mt * ROWB);
      }
    }
  };
  // The weight tile is the A operand and the panel rows the B operand, so an accumulator
  // holds h transposed: lane (n, g) of ag[mt][m] has token 16 mt + n and h columns
  // 8 g + 4 m + v (B = 32, with the gate/up tile packing) or 4 g + v (B = 16, from one slot or a
  // slot pair), v < 4.
  // FIRST: the row's first position, whose MFMAs start from zero (an inline constant, where
  // clearing the accumulators would take 64 moves per row at B = 32).
  auto compute = [&](const Slot& S, const AFrags& A, auto first) {
    constexpr bool FIRST = decltype(first)::value;
    const f32x4 z = {0.f, 0.f, 0.f, 0.f};
    if constexpr (PAIR) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        ag[mt][0] = mfma_bf16(S.g, A.g[mt], FIRST ? z : ag[mt][0]);
        if constexpr (!LIN) au[mt][0] = mfma_bf16(S.u, SHARED ? A.g[mt] : A.u[mt], FIRST ? z : au[mt][0]);
      }
    } else if constexpr (B == 16) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        ag[mt][0] = mfma_bf16_k16(S.g, A.g[mt], FIRST ? z : ag[mt][0]);
        if constexpr (!LIN) au[mt][0] = mfma_bf16_k16(S.u, SHARED ? A.g[mt] : A.u[mt], FIRST ? z : au[mt][0]);
      }
    } else {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int m = 0; m < CW; ++m) ag[mt][m] = mfma_bf16(S.g[0][m], A.g[mt], FIRST ? z : ag[mt][m]);
      if constexpr (!LIN) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int m = 0; m < CW; ++m)
            au[mt][m] = mfma_bf16(S.u[0][m], SHARED ? A.g[mt] : A.u[mt], FIRST ? z : au[mt][m]);
      }
    }
  };

  // ---- input panel: all of this thread's loads are issued before any store,
  // and the first ring positions' weight loads go out before the barrier
  if constexpr (READY) {
    // the column table stays in LDS from the first phase unless the phases alternate between
    // core blocks (each with its own table)
    if (a.reload_table) {
      ctab_fetch();
      if (nrows > 0) prefetch_ring();
      ctab_store();
    } else if (nrows > 0) {
      prefetch_ring();
    }
  } else if constexpr (!NORM) {
    constexpr int CPR = ROWB / 16;                 // chunk capacity of a panel row
    constexpr int NCH = TM * CPR;                  // chunks of the panel
    constexpr int PIT = (NCH + NT - 1) / NT;       // chunks per thread
    const int cpr = d_model / 8;
    // every load at a clamped address (row t0, chunk 0 stand in for the padding), so no
    // load sits under a branch and the waits before the stores stay exact
    u32x4 pv[PIT];
#pragma unroll
    for (int it = 0; it < PIT; ++it) {
      const int e0 = tid + NT * it;
      const int e = (NCH % NT == 0 || e0 < NCH) ? e0 : 0;
      const int row = e / CPR, cc = e % CPR;
      const int64_t t = t0 + row;
      const bool ok = cc < cpr && t < a.N;
      pv[it] = *reinterpret_cast<const u32x4*>(a.x + (ok ? t : t0) * d_model + 8 * (ok ? cc : 0));
    }
    ctab_fetch();
    if (nrows > 0) prefetch_ring();
    ctab_store();
#pragma unroll
    for (int it = 0; it < PIT; ++it) {
      const int e = tid + NT * it;
      const int row = e / CPR, cc = e % CPR;
      const bool ok = cc < cpr && t0 + row < a.N;
      if ((NCH % NT == 0 || e < NCH) && cc < cpr)
        *reinterpret_cast<u32x4*>(smem + panel_addr<MT>(row, cc, ROWB)) = k16s_chunk<B>(ok ? pv[it] : u32x4{0, 0, 0, 0}, row);
    }
  } else {
    // fp32 state rows -> RMSNorm -> bf16 panel; wave w owns rows w, w+NW, ...;
    // lane holds 8 contiguous values per 512-column step of each row
    constexpr int RW = (TM + NW - 1) / NW;         // rows per wave
    constexpr int SPR = ROWB / 1024;               // 512-column steps of the widest row
    // rows in registers at once: all of a wave's rows with 8 waves (their loads go out with the
    // other prologue loads), two at a time with more waves (a smaller register budget)
    constexpr int RB = NW == 8 ? RW : 2;
    f32x4 xv[RB][SPR][2];
    auto load_rows = [&](int rr0) {
#pragma unroll
      for (int b = 0; b < RB; ++b) {
        const int row = w + NW * (rr0 + b);
        const bool rok = (TM % NW == 0 || row < TM) && rr0 + b < RW;
        const int64_t t = t0 + row;
#pragma unroll
        for (int j = 0; j < SPR; ++j) {
          const int col = 8 * lane + 512 * j;
          // clamped address (row t0, column 0) for padding, zeroed after the load
          const bool ok = rok && col < d_model && t < a.N;
          const float* src = a.xf + (ok ? t : t0) * d_model + (ok ? col : 0);
          const f32x4 v0 = *reinterpret_cast<const f32x4*>(src);
          const f32x4 v1 = *reinterpret_cast<const f32x4*>(src + 4);
          xv[b][j][0] = ok ? v0 : f32x4{0.f, 0.f, 0.f, 0.f};
          xv[b][j][1] = ok ? v1 : f32x4{0.f, 0.f, 0.f, 0.f};
        }
      }
    };
    // the norm scale of this lane's columns, loaded once for all rows
    f32x4 sc[SPR][2];
    auto load_scale = [&]() {
#pragma unroll
      for (int j = 0; j < SPR; ++j) {
        const int col = 8 * lane + 512 * j;
        const float* src = a.norm_scale + (col < d_model ? col : 0);
        sc[j][0] = *reinterpret_cast<const f32x4*>(src);
        sc[j][1] = *reinterpret_cast<const f32x4*>(src + 4);
      }
    };
    auto norm_rows = [&](int rr0) {
#pragma unroll
      for (int b = 0; b < RB; ++b) {
        const int row = w + NW * (rr0 + b);
        if (rr0 + b >= RW || (TM % NW != 0 && row >= TM)) break;
        float ss = 0.f;
#pragma unroll
        for (int j = 0; j < SPR; ++j)
#pragma unroll
          for (int h2 = 0; h2 < 2; ++h2)
#pragma unroll
            for (int q = 0; q < 4; ++q) ss += xv[b][j][h2][q] * xv[b][j][h2][q];
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o, 64);
        const float rs = 1.0f / sqrtf(ss / (float)d_model + a.eps);
#pragma unroll
        for (int j = 0; j < SPR; ++j) {
          const int col = 8 * lane + 512 * j;
          // col < ROWB / 2 always: the padding columns of the panel row get zeros (no branch)
          const f32x4 s0 = sc[j][0], s1 = sc[j][1];
          const f32x4 v0 = xv[b][j][0], v1 = xv[b][j][1];
          const u32x4 o = {pack2_bf16(v0[0] * rs * s0[0], v0[1] * rs * s0[1]),
                           pack2_bf16(v0[2] * rs * s0[2], v0[3] * rs * s0[3]),
                           pack2_bf16(v1[0] * rs * s1[0], v1[1] * rs * s1[1]),
                           pack2_bf16(v1[2] * rs * s1[2], v1[3] * rs * s1[3])};
          *reinterpret_cast<u32x4*>(smem + panel_addr<MT>(row, col / 8, ROWB)) =
              k16s_chunk<B>(col < d_model ? o : u32x4{0, 0, 0, 0}, row);
        }
      }
    };
    if constexpr (RB == RW) {
      load_rows(0);
      load_scale();
      ctab_fetch();
      if (nrows > 0) prefetch_ring();
      ctab_store();
      norm_rows(0);
    } else {
      load_scale();
      ctab_fetch();
      if (nrows > 0) prefetch_ring();
      ctab_store();
      for (int rr0 = 0; rr0 < RW; rr0 += RB) {
        load_rows(rr0);
        norm_rows(rr0);
      }
    }
  }
  __syncthreads();
  if (nrows <= 0) return;
#pragma unroll
  for (int sl = 0; sl < RING; ++sl) fetch_c(P[sl]);

  // The A fragments of position p + 1 are read from the panel while position p's MFMAs
  // run (two register sets, alternating with the slot parity; RING is even), so the
  // LDS latency stays off the MFMA chain.
  static_assert(RING % 2 == 0, "A-fragment double buffer alternates with the slot parity");
  AFrags A0, A1;
  load_a(P[0], A0);
  __builtin_amdgcn_sched_barrier(0);
  // one group of RING positions (slot sl holds position sl of the group); the scheduling
  // barriers keep each slot's use after the previous slot's refill, so the wait before it
  // covers only that slot's loads
  auto ring_group = [&](auto first_group) {
#pragma unroll
    for (int sl = 0; sl < RING; ++sl) {
      const auto first = std::integral_constant<bool, decltype(first_group)::value>{};
      const std::integral_constant<bool, false> later{};
      if (sl % 2 == 0) {
        load_a(P[(sl + 1) % RING], A1);
        if (sl == 0) compute(P[sl], A0, first);
        else compute(P[sl], A0, later);
      } else {
        load_a(P[(sl + 1) % RING], A0);
        compute(P[sl], A1, later);
      }
      fetch(P[sl]);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  for (int n = 0; n < nrows; ++n) {
    // a row takes KP >= RING positions, so its first group always exists
    ring_group(std::true_type{});
    for (int k = RING; k < KP; k += RING) ring_group(std::false_type{});
    // epilogue of row r: h = silu(g) * u (and the pre-activations); each lane stores the
    // 4 * CW consecutive columns it holds of one token with one store
    const int r = r_lo + w + NW * n;
    const int64_t col0 = (int64_t)r * B + 4 * CW * g;
    // biases of this lane's 4 * CW columns
    float bgv[4 * CW], buv[4 * CW];
    if constexpr (BIAS) {
#pragma unroll
      for (int q = 0; q < 4 * CW; ++q) {
        bgv[q] = a.bg ? a.bg[col0 + q] : 0.f;
        buv[q] = a.bu ? a.bu[col0 + q] : 0.f;
      }
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int64_t t = t0 + 16 * mt + i;
      float o[4 * CW], gv[4 * CW], uv[4 * CW];
#pragma unroll
      for (int m = 0; m < CW; ++m)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          gv[4 * m + v] = ag[mt][m][v];
          uv[4 * m + v] = au[mt][m][v];
          if constexpr (BIAS) {
            gv[4 * m + v] += bgv[4 * m + v];
            uv[4 * m + v] += buv[4 * m + v];
          }
          o[4 * m + v] = LIN ? gv[4 * m + v] : silu_f(gv[4 * m + v]) * uv[4 * m + v];
        }
      if (t < a.N) {
        store_bf16x<4 * CW>(a.h + t * d_ff + col0, o);
        if constexpr (INTER) {
          if (a.gpre) store_bf16x<4 * CW>(a.gpre + t * d_ff + col0, gv);
          if (a.uout) store_bf16x<4 * CW>(a.uout + t * d_ff + col0, uv);
        }
      }
    }
  }
}

// Looped core: true when some token of [t0, t0 + tm) below N runs iteration `it` (tdepth[t] > it).
// tm <= 64: every wave reads the block's depths and takes the same ballot, so the answer is
// uniform over the workgroup without a barrier (or the LDS word a workgroup-wide vote would take,
// which would no longer leave the kernels their full 160 KB of dynamic LDS).
__device__ __forceinline__ bool block_runs(const int32_t* tdepth, int it, int64_t t0, int tm, int64_t N, int tid) {
  const int lane = tid & 63;
  bool p = false;
  if (lane < tm && t0 + lane < N) p = it < tdepth[t0 + lane];
  return __ballot(p) != 0;
}

// workgroup b -> (token block b / H, row slice b % H); the slices' rows split R_ff evenly, and
// with H a multiple of 8 every workgroup of one slice runs on the same XCD (workgroups are dealt
// to the 8 XCDs round robin), so each XCD's L2 holds the weights of its slices only
__device__ __forceinline__ void gu_slice(const GUArgs& a, int64_t& tb, int& r_lo, int& nrs) {
  const int64_t b = blockIdx.x;
  const int H = a.H, hs = (int)(b % H);
  tb = b / H;
  r_lo = (int)((int64_t)hs * a.R_ff / H);
  nrs = (int)((int64_t)(hs + 1) * a.R_ff / H) - r_lo;
}

template <int B, int MT, bool NORM, bool INTER, bool SHARED, bool BIAS>
__global__ __launch_bounds__(512, 1) void gu_kernel(GUArgs a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  int64_t tb;
  int r_lo, nrs;
  gu_slice(a, tb, r_lo, nrs);
  if (a.tdepth && !block_runs(a.tdepth, a.it, tb * 16 * MT, 16 * MT, a.N, (int)threadIdx.x)) return;
  gu_tile<B, MT, NORM, INTER, SHARED, false, BIAS>(a, tb, r_lo, nrs, smem, (int)threadIdx.x);
}

// gate/up with distinct gate/up topologies, without exported pre-activations or biases, one row
// slice, with 12 waves and a 2-deep
// ring: at most 168 VGPRs fit three waves per SIMD, and the extra waves hide more of the
// panel-read and weight-load latency than the shallower ring gives up.  B = 16 with a shared
// topology (slot pairs, so a 2-deep ring keeps four slots in flight) takes the same shape; B = 16
// with distinct topologies, with a quarter of the accumulators and 8-byte fragments (113 VGPRs),
// runs 16 waves with a 4-deep ring (forward at d_model 1024, d_ff 4096, 25 %, 16384 tokens:
// 0.2490 ms with 12 waves, 0.2467 with 16).
template <int B, bool SHARED> constexpr int gu_w12_waves() { return B == 16 && !SHARED ? 16 : 12; }
template <int B, bool SHARED> constexpr int gu_w12_ring() { return B == 16 && !SHARED ? 4 : 2; }
// (B = 16 also takes shared topologies and biases here)
template <int B, int MT, bool NORM, bool SHARED = false, bool BIAS = false>
__global__ __launch_bounds__((64 * gu_w12_waves<B, SHARED>()), 1) void gu_kernel_w12(GUArgs a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  if (a.tdepth && !block_runs(a.tdepth, a.it, (int64_t)blockIdx.x * 16 * MT, 16 * MT, a.N, (int)threadIdx.x)) return;
  gu_tile<B, MT, NORM, false, SHARED, false, BIAS, false, gu_w12_waves<B, SHARED>(), gu_w12_ring<B, SHARED>()>(
      a, (int64_t)blockIdx.x, 0, a.R_ff, smem, (int)threadIdx.x);
}

// plain Block-ELL product y = x W (+ bias) over an LDS panel of x (the gate/up kernel's gate
// stream alone).  With one stream the accumulators and fragments fit 16 waves at a 2-deep ring
// (at most 92 VGPRs); at the headline gate shape (16384 x 1024 -> 4096, B = 32) a call with
// per-call packing took 0.0535 ms against 0.0615 with 8 waves and a 4-deep ring (12 waves:
// 0.0551 with a 2-deep ring, 0.0535 with a 4-deep one)
constexpr int LIN_WAVES = 16;
template <int B, int MT, bool BIAS>
__global__ __launch_bounds__(64 * LIN_WAVES, 1) void lin_kernel(GUArgs a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  int64_t tb;
  int r_lo, nrs;
  gu_slice(a, tb, r_lo, nrs);
  gu_tile<B, MT, false, false, true, false, BIAS, true, LIN_WAVES, 2>(a, tb, r_lo, nrs, smem, (int)threadIdx.x);
}

// ===========================================================================
// down
// ===========================================================================
// h column blocks per LDS stage: 512 bytes of each token row (32 chunks)
// down kernel shape: DN_WAVES waves (one down row each) per workgroup; a stage holds
// DN_STAGE_COLS h columns of the workgroup's tokens
constexpr int DN_WAVES = 16;
constexpr int DN_STAGE_COLS = 512;
template <int B, int SC>
struct DnStage { static constexpr int G = SC / B; };

// The looped core's injection o = decay * o + dt * e on the CW state columns col .. col + CW - 1
// of the element at off (coef: decay [d], then dt [d])
template <int CW>
__device__ __forceinline__ void inject_cw(float (&o)[CW], const uint16_t* __restrict__ e,
                                          const float* __restrict__ coef, int64_t off, int col, int d) {
#pragma unroll
  for (int m = 0; m < CW; ++m) o[m] = coef[col + m] * o[m] + coef[d + col + m] * bf2f(e[off + m]);
}

// Per-wave fetch list of one stage: position q (lane q % 64 of v[q / 64]) holds
// desc = tile << 6 | cb -- the packed down tile (row * Kd + slot) and its column
// block within the stage.  Positions run over the wave's rows in order, hits of
// a row in slot order; a row with an odd hit count gets one padding position on
// the packed zero tile, so a two-slot ring consumes every row with the same
// slot parity.  pcnt[rho] is the padded count of row rho, tot their sum (even).
// A stage holds at most RPW * (Kd + 1) <= 64 * NV positions: NV = 4 for up to 64 slots per row
// (RPW <= 2, or RPW = 4 with Kd <= 63), 5 for up to 128 (RPW <= 2).
template <int KC> constexpr int dn_list_words() { return KC == 1 ? 4 : 5; }
template <int RPW, int NV>
struct FetchList {
  int v[NV];
  int pcnt[RPW];
  int tot;
};

__device__ __forceinline__ int lanes_below(uint64_t m) {
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0));
}

// write `val` of the lanes in `m` (in lane order) to positions base, base+1, ...
// of the list; positions outside [base, base + popcount(m)) keep their values
template <int NV>
__device__ __forceinline__ void list_scatter(int (&v)[NV], uint64_t m, int base, int val, int lane) {
  const int cnt = __builtin_popcountll(m);
  if (cnt == 0) return;
  const int rank = lanes_below(m);
  const bool src = (m >> lane) & 1;
#pragma unroll
  for (int t = 0; t < NV; ++t) {
    const int lo = base - 64 * t, hi = base + cnt - 64 * t;   // range of this target, in its lanes
    if (hi <= 0 || lo >= 64) continue;
    const int clo = lo > 0 ? lo : 0, chi = hi < 64 ? hi : 64;
    // participants: source lanes whose position lands in this target
    const int pos = base + rank - 64 * t;
    const bool part = src && pos >= 0 && pos < 64;
    const uint64_t pm = __ballot(part);
    // a full permutation: participants -> their lanes, the others -> the lanes outside [clo, chi)
    const int orank = lanes_below(~pm);
    const int dst = part ? pos : (orank < clo ? orank : orank + (chi - clo));
    const int got = __builtin_amdgcn_ds_permute(dst << 2, val);
    if (lane >= clo && lane < chi) v[t] = got;
  }
}

template <int NV>
__device__ __forceinline__ void list_set(int (&v)[NV], int q, int val, int lane) {
  const int t = q >> 6, l = q & 63;
#pragma unroll
  for (int u = 0; u < NV; ++u)
    if (t == u && lane == l) v[u] = val;
}

template <int NV>
__device__ __forceinline__ int list_get(const int (&v)[NV], int q) {
  const int l = q & 63, t = q >> 6;
  int r = __builtin_amdgcn_readlane(v[0], l);
#pragma unroll
  for (int u = 1; u < NV; ++u) {
    const int e = __builtin_amdgcn_readlane(v[u], l);
    r = t == u ? e : r;
  }
  return r;
}

// the fetch list of the stage covering column blocks c0 .. c0 + ncb - 1: lane l of colreg[rho][kc]
// holds the column of slot 64 kc + l of the wave's row rho (-1 beyond Kd)
template <int RPW, int KC, int NV>
__device__ __forceinline__ void dn_build(FetchList<RPW, NV>& L, int c0, int ncb, const int (&colreg)[RPW][KC],
                                         int wrow0, int Kd, int ztile, int lane) {
  int tot = 0;
#pragma unroll
  for (int t = 0; t < NV; ++t) L.v[t] = 0;
#pragma unroll
  for (int rho = 0; rho < RPW; ++rho) {
    int cnt = 0;
#pragma unroll
    for (int kc = 0; kc < KC; ++kc) {
      const int cb = colreg[rho][kc] - c0;
      const uint64_t m = __ballot(cb >= 0 && cb < ncb);
      list_scatter(L.v, m, tot + cnt, (((wrow0 + rho) * Kd + 64 * kc + lane) << 6) | (cb & 63), lane);
      cnt += __builtin_popcountll(m);
    }
    if (cnt & 1) list_set(L.v, tot + cnt, ztile << 6, lane);
    L.pcnt[rho] = cnt + (cnt & 1);
    tot += L.pcnt[rho];
  }
  L.tot = tot;
}

// down projection of token block tb for the down rows of row group rg (NW * RPW rows) by one
// workgroup of NW waves; dn_smem holds two h stages (2 * 16 * MT * DN_STAGE_COLS * 2 bytes).
// Every wave reaches every barrier (a workgroup whose tokens are all past N returns at once).
// NORMOUT (fp32 state mode, all down rows in this one group): the epilogue also writes the
// RMSNorm of the new state rows (norm_scale, eps), as bf16, into the gate/up panel at the start
// of dn_smem (row stride GUPanel<MT>::ROWB), for the next iteration's gate/up phase; red holds
// (NW + 1) * 16 * MT floats for the per-token sums of squares.
template <int B, int MT, int RPW, int NW, bool NORMOUT = false, bool BIAS = false, int SC = DN_STAGE_COLS,
          bool CORE = false, int KC = 1>
__device__ __forceinline__ void dn_tile(const DNArgs& a, int64_t tb, int rg, unsigned char* dn_smem,
                                        uint16_t* out, int tid, const float* norm_scale = nullptr,
                                        float eps = 0.f, float* red = nullptr) {
  constexpr int CW = TileShape<B>::CW;
  constexpr int TM = 16 * MT;
  constexpr int G = DnStage<B, SC>::G;
  constexpr int SROWB = G * B * 2;                   // bytes per token row of a stage (512)
  constexpr int SBYTES = TM * SROWB;                 // bytes per stage
  constexpr int CHUNKS = SBYTES / 16;                // 16-byte chunks per stage
  constexpr int NT = 64 * NW;                        // threads
  constexpr int PER_T = (CHUNKS + NT - 1) / NT;      // chunks per thread per stage
  static_assert(TileShape<B>::NKS == 1, "down kernel handles B <= 32");
  static_assert(SROWB % 256 == 0, "stage rows must cover multiples of 16 chunks");
  static_assert(G <= 64, "a list entry holds the column block of its stage in 6 bits");

  const int lane = tid & 63;
  const int w = uniform(tid >> 6);
  const int i = lane & 15, g = lane >> 4;
  const int64_t t0 = tb * TM;
  if (t0 >= a.N) return;   // the whole workgroup, before any barrier
  const int row0 = rg * NW * RPW;   // first down row of this workgroup
  const int d_model = a.d_model;
  const int64_t d_ff = a.d_ff;
  const int C = a.C_d;
  const int nstages = (C + G - 1) / G;
  const u32x4* pd = static_cast<const u32x4*>(a.pd);
  const int ztile = a.R_m * a.Kd;   // packed zero tile

  // lane l of colreg[rho][kc]: the column of slot 64 kc + l of row rho (-1 beyond the row's slots)
  int colreg[RPW][KC];
#pragma unroll
  for (int rho = 0; rho < RPW; ++rho) {
    const int rm = row0 + w * RPW + rho;
#pragma unroll
    for (int kc = 0; kc < KC; ++kc)
      colreg[rho][kc] = (rm < a.R_m && 64 * kc + lane < a.Kd) ? a.cd[(int64_t)rm * a.Kd + 64 * kc + lane] : -1;
  }

  f32x4 acc[RPW][MT][CW];
#pragma unroll
  for (int rho = 0; rho < RPW; ++rho)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int m = 0; m < CW; ++m) acc[rho][mt][m] = f32x4{0.f, 0.f, 0.f, 0.f};

  // stage loader: chunk e of stage s -> (token row, 16-byte chunk within the row)
  u32x4 sreg[PER_T];
  auto stage_fetch = [&](int s) {
#pragma unroll
    for (int u = 0; u < PER_T; ++u) {
      const int e = tid + NT * u;
      sreg[u] = u32x4{0, 0, 0, 0};
      if (e < CHUNKS) {
        const int row = e / (SROWB / 16), c = e - row * (SROWB / 16);
        const int64_t t = t0 + row;
        const int64_t col = (int64_t)s * G * B + 8 * c;
        if (t < a.N && col < d_ff) sreg[u] = *reinterpret_cast<const u32x4*>(a.h + t * d_ff + col);
      }
    }
  };
  auto stage_store = [&](int buf) {
#pragma unroll
    for (int u = 0; u < PER_T; ++u) {
      const int e = tid + NT * u;
      if (e < CHUNKS) {
        const int row = e / (SROWB / 16), c = e - row * (SROWB / 16);
        *reinterpret_cast<u32x4*>(dn_smem + buf * SBYTES + panel_addr<MT>(row, c, SROWB)) = k16s_chunk<B>(sreg[u], row);
      }
    }
  };

  // ring slots: weight fragments and column block
  struct Slot {
    std::conditional_t<B == 16, u32x2, u32x4> f[1][CW];   // B = 16: 16x16x16 fragments
    int cb;
  };
  const uint32_t f16 = pfrag16_off(lane);
  constexpr int NV = dn_list_words<KC>();
  FetchList<RPW, NV> cur, nxt;
  // position q of the stream made of the current stage's list followed by the
  // next stage's; beyond both, the zero tile
  auto fetch = [&](Slot& S, int q) {
    int d = ztile << 6;
    if (q < cur.tot) d = list_get(cur.v, q);
    else if (q - cur.tot < nxt.tot) d = list_get(nxt.v, q - cur.tot);
    if constexpr (B == 16) S.f[0][0] = load_pfrag16(pd + (int64_t)(d >> 6) * PackedTile<B>::U32X4, f16);
    else load_pfrag<B>(pd + (int64_t)(d >> 6) * PackedTile<B>::U32X4, lane, S.f);
    S.cb = d & 63;
  };
  const uint32_t lbase = (uint32_t)(i * MT * SROWB);
  auto compute = [&](const Slot& S, const unsigned char* sb, f32x4 (&ac)[MT][CW]) {
    const int cb = uniform(S.cb);
    if constexpr (B == 16) {
      const uint32_t a0 = k16s_addr(lbase, cb, g, i);
      u32x2 av[MT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) av[mt] = lds8(sb, a0 + mt * SROWB);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) ac[mt][0] = mfma_bf16_k16(av[mt], S.f[0][0], ac[mt][0]);
    } else {
      const uint32_t a0 = lbase + (((cb * (B / 8) + g) ^ i) << 4);
      u32x4 av[MT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) av[mt] = lds16(sb, a0 + mt * SROWB);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int m = 0; m < CW; ++m) ac[mt][m] = mfma_bf16(av[mt], S.f[0][m], ac[mt][m]);
    }
  };

  const bool any_rows = (row0 + w * RPW < a.R_m) && a.Kd > 0;
  Slot S0, S1;
  nxt.tot = 0;
  dn_build<RPW, KC, NV>(cur, 0, (C < G ? C : G), colreg, row0 + w * RPW, a.Kd, ztile, lane);
  if (nstages > 1) dn_build<RPW, KC, NV>(nxt, G, (C - G) < G ? (C - G) : G, colreg, row0 + w * RPW, a.Kd, ztile, lane);
  stage_fetch(0);
  stage_store(0);
  bool ring_ok = false;   // S0/S1 hold positions 0 and 1 of the current stage
  __syncthreads();
  for (int s = 0; s < nstages; ++s) {
    const int buf = s & 1;
    const unsigned char* sb = dn_smem + buf * SBYTES;
    if (s + 1 < nstages) stage_fetch(s + 1);
    if (any_rows && cur.tot > 0) {
      if (!ring_ok) {
        __builtin_amdgcn_sched_barrier(0);
        fetch(S0, 0);
        __builtin_amdgcn_sched_barrier(0);
        fetch(S1, 1);
        __builtin_amdgcn_sched_barrier(0);
      }
      int q = 0;
#pragma unroll
      for (int rr = 0; rr < RPW; ++rr) {
        for (int j = 0; j < cur.pcnt[rr]; j += 2) {
          compute(S0, sb, acc[rr]);
          fetch(S0, q + 2);
          __builtin_amdgcn_sched_barrier(0);
          compute(S1, sb, acc[rr]);
          fetch(S1, q + 3);
          __builtin_amdgcn_sched_barrier(0);
          q += 2;
        }
      }
    }
    // the ring now holds positions 0 and 1 of the next stage iff this stage ran and the next has hits
    ring_ok = any_rows && cur.tot > 0 && nxt.tot > 0;
    if (s + 1 < nstages) stage_store(buf ^ 1);
    cur = nxt;
    nxt.tot = 0;
    if (s + 2 < nstages) {
      const int c2 = (s + 2) * G;
      dn_build<RPW, KC, NV>(nxt, c2, (C - c2) < G ? (C - c2) : G, colreg, row0 + w * RPW, a.Kd, ztile, lane);
    }
    __syncthreads();
  }

  if constexpr (NORMOUT) {
    // ---- epilogue with the next iteration's normalised panel: new state = acc + state
    // (written back, kept in acc), per-token sums of squares over the lanes, the waves, then
    // bf16(state * rs * scale) into the panel
    constexpr int ROWB = GUPanel<MT>::ROWB;
    float ssq[MT][4];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int v = 0; v < 4; ++v) ssq[mt][v] = 0.f;
#pragma unroll
    for (int rho = 0; rho < RPW; ++rho) {
      const int rm = row0 + w * RPW + rho;
      if (rm >= a.R_m) continue;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int64_t t = t0 + 16 * mt + 4 * g + v;
          const bool ok = t < a.N;
          const int64_t off = (ok ? t : t0) * d_model + rm * B + CW * i;
          // looped core: a row past its depth keeps its state; one that runs the next iteration
          // takes that iteration's injection
          bool run = ok, inj = CORE && ok && a.inj_e;
          if (CORE && a.tdepth) {
            const int dep = ok ? a.tdepth[t] : 0;
            run = a.it < dep;
            inj = inj && a.it + 1 < dep;
          }
          float o[CW];
#pragma unroll
          for (int m = 0; m < CW; ++m) {
            float av = acc[rho][mt][m][v];
            if constexpr (BIAS) {
              if (a.bd) av += a.bd[rm * B + CW * i + m];
            }
            const float sv = ok ? a.state[off + m] : 0.f;
            o[m] = run ? av + sv : sv;
          }
          if (inj) inject_cw<CW>(o, a.inj_e, a.inj_coef, off, rm * B + CW * i, d_model);
#pragma unroll
          for (int m = 0; m < CW; ++m) {
            acc[rho][mt][m][v] = o[m];
            ssq[mt][v] += o[m] * o[m];
          }
          if (run) {
#pragma unroll
            for (int m = 0; m < CW; ++m) a.state[off + m] = o[m];
          }
          if (ok && out) store_bf16<CW>(out + off, o);
        }
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
#pragma unroll
        for (int o = 1; o < 16; o <<= 1) ssq[mt][v] += __shfl_xor(ssq[mt][v], o, 64);
        if (i == 0) red[w * TM + 16 * mt + 4 * g + v] = ssq[mt][v];
      }
    __syncthreads();
    if (tid < TM) {
      float ss = 0.f;
#pragma unroll
      for (int ww = 0; ww < NW; ++ww) ss += red[ww * TM + tid];
      red[NW * TM + tid] = 1.0f / sqrtf(ss / (float)d_model + eps);
    }
    __syncthreads();
#pragma unroll
    for (int rho = 0; rho < RPW; ++rho) {
      const int rm = row0 + w * RPW + rho;
      if (rm >= a.R_m) continue;
      const int col = rm * B + CW * i;
      float sc[CW];
#pragma unroll
      for (int m = 0; m < CW; ++m) sc[m] = norm_scale[col + m];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int row = 16 * mt + 4 * g + v;
          const float rs = red[NW * TM + row];
          // (B = 16: the element's half of the chunk swapped in rows with row & 8, as k16s_chunk)
          unsigned char* dst = dn_smem + panel_addr<MT>(row, col / 8, ROWB) +
                               ((2 * (col % 8)) ^ (B == 16 ? ((row >> 3) & 1) << 3 : 0));
          if constexpr (CW == 2) {
            *reinterpret_cast<uint32_t*>(dst) =
                pack2_bf16(acc[rho][mt][0][v] * rs * sc[0], acc[rho][mt][1][v] * rs * sc[1]);
          } else {
            *reinterpret_cast<uint16_t*>(dst) = f2bf(acc[rho][mt][0][v] * rs * sc[0]);
          }
        }
    }
    return;
  }

  // ---- epilogue: + residual (bf16) or + fp32 state; store bf16 (and the state)
#pragma unroll
  for (int rho = 0; rho < RPW; ++rho) {
    const int rm = row0 + w * RPW + rho;
    if (rm >= a.R_m) continue;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int64_t t = t0 + 16 * mt + 4 * g + v;
        if (t >= a.N) continue;
        const int64_t off = t * d_model + rm * B + CW * i;
        float o[CW];
#pragma unroll
        for (int m = 0; m < CW; ++m) {
          o[m] = acc[rho][mt][m][v];
          if constexpr (BIAS) {
            if (a.bd) o[m] += a.bd[rm * B + CW * i + m];
          }
        }
        if (a.state) {
          // looped core: a row past its depth keeps its state (and its output is that state);
          // one that runs the next iteration takes that iteration's injection
          bool run = true, inj = CORE && a.inj_e != nullptr;
          if (CORE && a.tdepth) {
            const int dep = a.tdepth[t];
            run = a.it < dep;
            inj = inj && a.it + 1 < dep;
          }
          if (run) {
#pragma unroll
            for (int m = 0; m < CW; ++m) o[m] += a.state[off + m];
            if (inj) inject_cw<CW>(o, a.inj_e, a.inj_coef, off, rm * B + CW * i, d_model);
#pragma unroll
            for (int m = 0; m < CW; ++m) a.state[off + m] = o[m];
          } else {
            if (!out) continue;
#pragma unroll
            for (int m = 0; m < CW; ++m) o[m] = a.state[off + m];
          }
        } else if (a.resid) {
          float rv[CW];
          load_bf16<CW>(a.resid + off, rv);
#pragma unroll
          for (int m = 0; m < CW; ++m) o[m] += rv[m];
        }
        if (out) store_bf16<CW>(out + off, o);
      }
  }
}

// CORE: the looped core's state update (depth mask, fused injection); the other instantiations
// carry none of its code
template <int B, int MT, int RPW, int NW, int SC, bool BIAS, bool CORE, int KC>
__global__ __launch_bounds__(64 * NW, 1) void dn_kernel(DNArgs a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char dn_smem[];   // two stages
  // workgroup -> (token block, row group).  With several row groups, the groups of one token
  // block get workgroup ids that agree mod 8, i.e. one XCD (workgroups are dealt to the 8
  // XCDs round robin), so the h stages every group reads come from that XCD's L2.
  int tb = (int)blockIdx.x, rg = 0;
  if (a.nrg > 1) {
    const int b = (int)blockIdx.x, rest = b >> 3;
    rg = rest % a.nrg;
    tb = 8 * (rest / a.nrg) + (b & 7);
  }
  constexpr int TM = 16 * MT;
  if (CORE && a.tdepth && !block_runs(a.tdepth, a.it, (int64_t)tb * TM, TM, a.N, (int)threadIdx.x)) {
    // looped core: every row of the block is past its depth; only the last application's
    // output (the kept state, as bf16) remains to be written
    if (a.out) {
      const int row0 = rg * NW * RPW;
      const int nrm = a.R_m - row0 < NW * RPW ? a.R_m - row0 : NW * RPW;
      const int c8 = nrm * B / 8;   // 8-column groups of this workgroup's down rows
      for (int idx = (int)threadIdx.x; idx < TM * c8; idx += 64 * NW) {
        const int64_t t = (int64_t)tb * TM + idx / c8;
        if (t >= a.N) break;
        const int64_t off = t * a.d_model + row0 * B + 8 * (idx % c8);
        const f32x4 v0 = *reinterpret_cast<const f32x4*>(a.state + off);
        const f32x4 v1 = *reinterpret_cast<const f32x4*>(a.state + off + 4);
        *reinterpret_cast<u32x4*>(a.out + off) = u32x4{pack2_bf16(v0[0], v0[1]), pack2_bf16(v0[2], v0[3]),
                                                       pack2_bf16(v1[0], v1[1]), pack2_bf16(v1[2], v1[3])};
      }
    }
    return;
  }
  dn_tile<B, MT, RPW, NW, false, BIAS, SC, CORE, KC>(a, tb, rg, dn_smem, a.out, (int)threadIdx.x);
}

// ===========================================================================
// down projection with a deep ring (the plain forward)
// ===========================================================================
// dnf_kernel<B, D>: the dn_kernel workgroup (16 waves, 64 tokens, one down row per wave, h staged
// through LDS 512 columns at a time, next stage fetched into registers while the current one is
// consumed), but each wave streams its tiles through a D-slot ring that runs over its whole row:
// lane k of a wave holds the column of the row's slot k, the entries of stage s are the lanes
// whose column lies in it (ballot), taken in lane order, so the ring's positions follow the
// stages with no padding and no restart, and a stage change is a workgroup barrier taken inline
// when the next position belongs to a later stage.  The tile loads a wave keeps in flight (D) hide
// the L2 latency that the two-slot pairs of dn_kernel could not.
template <int B, int D, bool BIAS>
__global__ __launch_bounds__(64 * DN_WAVES, 1) void dnf_kernel(DNArgs a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char dn_smem[];   // two stages
  constexpr int MT = 4, NW = DN_WAVES;
  constexpr int CW = TileShape<B>::CW;
  constexpr int TM = 16 * MT;
  constexpr int G = DnStage<B, DN_STAGE_COLS>::G;    // column blocks per stage
  constexpr int SROWB = G * B * 2;                   // bytes per token row of a stage
  constexpr int SBYTES = TM * SROWB;                 // bytes per stage
  constexpr int CHUNKS = SBYTES / 16;
  constexpr int NT = 64 * NW;
  constexpr int PER_T = (CHUNKS + NT - 1) / NT;
  static_assert(TileShape<B>::NKS == 1, "B <= 32");
  const int tid = (int)threadIdx.x;
  const int lane = tid & 63;
  const int w = uniform(tid >> 6);
  const int i = lane & 15, g = lane >> 4;
  int tb = (int)blockIdx.x, rg = 0;
  if (a.nrg > 1) {   // the row groups of one token block on one XCD (ids equal mod 8)
    const int b = (int)blockIdx.x, rest = b >> 3;
    rg = rest % a.nrg;
    tb = 8 * (rest / a.nrg) + (b & 7);
  }
  const int64_t t0 = (int64_t)tb * TM;
  if (t0 >= a.N) return;   // the whole workgroup, before any barrier
  const int rm = rg * NW + w;   // this wave's down row
  const int d_model = a.d_model;
  const int64_t d_ff = a.d_ff;
  const int C = a.C_d;
  const int nstages = (C + G - 1) / G;
  const u32x4* pd = static_cast<const u32x4*>(a.pd);
  const int ztile = a.R_m * a.Kd;

  // lane k: slot k of the row (dead slots and lanes beyond Kd take no part)
  int ecol = -1;
  if (rm < a.R_m && lane < a.Kd) ecol = a.cd[(int64_t)rm * a.Kd + lane];
  const bool live = ecol >= 0 && ecol < C;
  const int est = live ? ecol / G : 0;

  f32x4 acc[MT][CW];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int m = 0; m < CW; ++m) acc[mt][m] = f32x4{0.f, 0.f, 0.f, 0.f};

  // stage loads: unconditional (clamped address), zeros selected at the LDS store
  u32x4 sreg[PER_T];
  int sok = 0;
  auto stage_fetch = [&](int s) {
    sok = 0;
#pragma unroll
    for (int u = 0; u < PER_T; ++u) {
      const int e = tid + NT * u;
      const int ec = e < CHUNKS ? e : CHUNKS - 1;
      const int row = ec / (SROWB / 16), c = ec - row * (SROWB / 16);
      const int64_t t = t0 + row;
      const int64_t col = (int64_t)s * G * B + 8 * c;
      sok |= (e < CHUNKS && t < a.N && col < d_ff) ? 1 << u : 0;
      sreg[u] = *reinterpret_cast<const u32x4*>(a.h + (t < a.N ? t : a.N - 1) * d_ff + (col < d_ff ? col : 0));
    }
  };
  auto stage_store = [&](int buf) {
#pragma unroll
    for (int u = 0; u < PER_T; ++u) {
      const int e = tid + NT * u;
      if (e < CHUNKS) {
        const int row = e / (SROWB / 16), c = e - row * (SROWB / 16);
        *reinterpret_cast<u32x4*>(dn_smem + buf * SBYTES + panel_addr<MT>(row, c, SROWB)) =
            (sok >> u) & 1 ? sreg[u] : u32x4{0, 0, 0, 0};
      }
    }
  };

  struct Slot {
    std::conditional_t<B == 16, u32x2, u32x4> f[1][CW];
    int el;   // entry lane (-1: none left)
    int st;   // stage
    int cb;   // column block within the stage
  };
  const uint32_t f16 = pfrag16_off(lane);
  // fetch cursor: stage fs and the entries of it not yet fetched
  int fs = 0;
  uint64_t fmask = __builtin_amdgcn_ballot_w64(live && est == 0);
  auto fetch = [&](Slot& S) {
    while (fmask == 0 && fs + 1 < nstages) {
      ++fs;
      fmask = __builtin_amdgcn_ballot_w64(live && est == fs);
    }
    int el = -1;
    if (fmask) {
      el = (int)__builtin_ctzll(fmask);
      fmask &= fmask - 1;
    }
    const int tile = el >= 0 ? rm * a.Kd + el : ztile;
    if constexpr (B == 16) S.f[0][0] = load_pfrag16(pd + (int64_t)tile * PackedTile<B>::U32X4, f16);
    else load_pfrag<B>(pd + (int64_t)tile * PackedTile<B>::U32X4, lane, S.f);
    S.el = el;
    S.st = fs;
    S.cb = __builtin_amdgcn_readlane(ecol, el >= 0 ? el : 0) - fs * G;
  };
  const uint32_t lbase = (uint32_t)(i * MT * SROWB);
  auto compute = [&](const Slot& S, const unsigned char* sb) {
    const int cb = S.cb;
    if constexpr (B == 16) {
      const uint32_t a0 = k16_addr(lbase, cb, g, i);
      u32x2 av[MT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) av[mt] = lds8(sb, a0 + mt * SROWB);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) acc[mt][0] = mfma_bf16_k16(av[mt], S.f[0][0], acc[mt][0]);
    } else {
      const uint32_t a0 = lbase + (((cb * (B / 8) + g) ^ i) << 4);
      u32x4 av[MT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) av[mt] = lds16(sb, a0 + mt * SROWB);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int m = 0; m < CW; ++m) acc[mt][m] = mfma_bf16(av[mt], S.f[0][m], acc[mt][m]);
    }
  };

  Slot R[D];
#pragma unroll
  for (int sl = 0; sl < D; ++sl) fetch(R[sl]);
  stage_fetch(0);
  stage_store(0);
  __syncthreads();
  if (nstages > 1) stage_fetch(1);
  // stage cs -> cs + 1: the registers fetched at the start of stage cs go to the other buffer;
  // after the barrier every wave is past stage cs, whose buffer takes the stage after next
  int cs = 0;
  auto transition = [&]() {
    stage_store((cs + 1) & 1);
    __syncthreads();
    ++cs;
    if (cs + 1 < nstages) stage_fetch(cs + 1);
  };
  // Every slot is refetched on every pass, also past the row's last entry (the zero tile), so the
  // tile loads are never skipped and the compiler's memory-counter waits stay exact; the entries
  // are consumed in fetch order, so once slot 0 comes back empty every slot is.
  for (;;) {
#pragma unroll
    for (int sl = 0; sl < D; ++sl) {
      Slot& S = R[sl];
      if (S.el >= 0) {
        while (cs < S.st) transition();
        compute(S, dn_smem + (cs & 1) * SBYTES);
      }
      fetch(S);
    }
    if (R[0].el < 0) break;
  }
  while (cs + 1 < nstages) transition();

  // ---- epilogue: (+ down bias) + residual; store bf16
  if (rm >= a.R_m) return;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int64_t t = t0 + 16 * mt + 4 * g + v;
      if (t >= a.N) continue;
      const int64_t off = t * d_model + rm * B + CW * i;
      float o[CW];
#pragma unroll
      for (int m = 0; m < CW; ++m) {
        o[m] = acc[mt][m][v];
        if constexpr (BIAS) o[m] += a.bd[rm * B + CW * i + m];
      }
      if (a.resid) {
        float rv[CW];
        load_bf16<CW>(a.resid + off, rv);
#pragma unroll
        for (int m = 0; m < CW; ++m) o[m] += rv[m];
      }
      store_bf16<CW>(a.out + off, o);
    }
}

// ===========================================================================
// looped block in one persistent launch
// ===========================================================================
// LDS of the looped kernel: gate/up panel (or the two down stages) | column table | per-token
// sums of squares of the down phase's normalisation (9 * 16 * MT floats)
template <int MT>
__host__ __device__ inline size_t looped_red_offset(int R_ff, int K) {
  return (size_t)16 * MT * GUPanel<MT>::ROWB + (((size_t)R_ff * K * 2 + 255) & ~(size_t)255);
}
// looped_kernel<B, MT, SHARED, RPW>: workgroup tb owns token block tb (16 * MT tokens) for all L
// iterations of the looped core: it copies its rows of h_in into the fp32 state (with the first
// iteration's injection, state = decay * state + dt * e, when e is given), then per iteration runs
// the n_core blocks in order, each h <- h + SwiGLU(RMSNorm(h)) as a gate/up tile (RMSNorm of its
// state rows into the LDS panel, h of its tokens to the h buffer) and the down tile of every row
// group (h staged back through LDS, state += down product), with workgroup barriers between the
// phases.  The last block's down phase also applies the next iteration's injection.  With
// per-token depths a row stops once it has run its depth (its state is kept: the reference's
// where(active, h_new, h_agg)), and the block stops after its deepest row.  Only this workgroup
// reads or writes its state and h rows, so no grid-wide barrier is needed; the weights are read by
// every workgroup in every iteration (the packed tiles stay in L2 / the memory-side cache across
// iterations).  The block's last phase also writes the bf16 output.
template <int B, int MT, bool SHARED, int RPW, bool BIAS>
__global__ __launch_bounds__(512, 1) void looped_kernel(LoopArgs la) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  constexpr int TM = 16 * MT;
  const int tid = threadIdx.x;
  const int64_t tb = blockIdx.x;
  const int64_t t0 = tb * TM;
  const int64_t N = la.gu.N;
  if (t0 >= N) return;
  const int d_model = la.gu.d_model;
  const int rows = (int)(N - t0 < TM ? N - t0 : TM);
  float* red = reinterpret_cast<float*>(smem + la.red_off);
  // iterations this block runs: L, or its deepest row's depth when that is smaller
  int lrun = la.L;
  if (la.tdepth) {
    if (tid < 64) {
      int dmax = 0;
      for (int r = tid; r < rows; r += 64) {
        const int dp = la.tdepth[t0 + r];
        dmax = dp > dmax ? dp : dmax;
      }
#pragma unroll
      for (int o = 32; o >= 1; o >>= 1) {
        const int v = __shfl_xor(dmax, o, 64);
        dmax = v > dmax ? v : dmax;
      }
      if (tid == 0) reinterpret_cast<int*>(red)[0] = dmax;
    }
    __syncthreads();
    const int dmax = reinterpret_cast<const int*>(red)[0];
    __syncthreads();
    lrun = dmax < lrun ? dmax : lrun;
  }
  // state rows <- float(h_in rows) (+ the first injection on the rows that run it): 8 elements per
  // thread per step (d_model % 8 == 0); a block that runs no iteration copies h_in to the output
  {
    const int n = rows * d_model;
    const int64_t base = t0 * d_model;
    for (int e = 8 * tid; e < n; e += 8 * 512) {
      const u32x4 v = *reinterpret_cast<const u32x4*>(la.h_in + base + e);
      if (lrun <= 0) {
        *reinterpret_cast<u32x4*>(la.dn.out + base + e) = v;
        continue;
      }
      float sv[8];
      unpack8_bf16(v, sv);
      if (la.e) {
        const int r = e / d_model;
        if (!la.tdepth || la.tdepth[t0 + r] > 0) inject8(sv, la.e, la.inj_coef, base + e, e - r * d_model, d_model);
      }
      float* y = la.dn.state + base + e;
      *reinterpret_cast<f32x4*>(y) = f32x4{sv[0], sv[1], sv[2], sv[3]};
      *reinterpret_cast<f32x4*>(y + 4) = f32x4{sv[4], sv[5], sv[6], sv[7]};
    }
  }
  if (lrun <= 0) return;
  __syncthreads();
  const int nrg = (la.dn.R_m + 8 * RPW - 1) / (8 * RPW);
  // with every down row in one group, the down phase writes the next phase's normalised panel
  // itself (the gate/up phase then reads the state no more)
  const bool fuse = nrg == 1;
  const int nc = la.n_core;
  for (int l = 0; l < lrun; ++l) {
    for (int c = 0; c < nc; ++c) {
      // The thread and token-block indices pass through an opaque copy in every phase:
      // otherwise the compiler hoists the phases' address arithmetic (derived from them) out
      // of the iteration loop, and the registers it then keeps live across both phases spill.
      int tg = tid;
      int64_t tbg = tb;
      asm volatile("" : "+v"(tg), "+s"(tbg));
      const CoreW& cw = la.core[c];
      GUArgs gu = la.gu;
      gu.pg = cw.pg; gu.cg = cw.cg; gu.Kg = cw.Kg;
      gu.pu = cw.pu; gu.cu = cw.cu; gu.Ku = cw.Kg;
      gu.norm_scale = cw.norm_scale; gu.bg = cw.bg; gu.bu = cw.bu;
      gu.reload_table = nc > 1;
      if (fuse && (l > 0 || c > 0)) gu_tile<B, MT, true, false, SHARED, true, BIAS>(gu, tbg, 0, gu.R_ff, smem, tg);
      else gu_tile<B, MT, true, false, SHARED, false, BIAS>(gu, tbg, 0, gu.R_ff, smem, tg);
      __syncthreads();
      const bool last = l == lrun - 1 && c == nc - 1;
      uint16_t* out = last ? la.dn.out : nullptr;
      DNArgs dn = la.dn;
      dn.pd = cw.pd; dn.cd = cw.cd; dn.Kd = cw.Kd; dn.bd = cw.bd;
      dn.tdepth = la.tdepth; dn.it = l;
      dn.inj_e = (c == nc - 1 && l + 1 < lrun) ? la.e : nullptr;
      dn.inj_coef = la.inj_coef;
      const float* next_scale = la.core[c + 1 < nc ? c + 1 : 0].norm_scale;
      for (int rg = 0; rg < nrg; ++rg) {
        int td = tid;
        int64_t tbd = tb;
        asm volatile("" : "+v"(td), "+s"(tbd));
        if (fuse && !last)
          dn_tile<B, MT, RPW, 8, true, BIAS, DN_STAGE_COLS, true>(dn, tbd, rg, smem, out, td, next_scale, la.gu.eps,
                                                                 red);
        else
          dn_tile<B, MT, RPW, 8, false, BIAS, DN_STAGE_COLS, true>(dn, tbd, rg, smem, out, td);
        __syncthreads();
      }
    }
  }
}

// state <- float(x), fp32 copy of a bf16 tensor
// 8 elements per thread (one 16-byte load, two 16-byte stores) when x and y are 16-byte
// aligned; the last partial group element by element
__global__ __launch_bounds__(256) void bf16_to_f32_kernel(const uint16_t* __restrict__ x, int64_t n,
                                                          float* __restrict__ y) {
  const int64_t e0 = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 8;
  if (e0 + 8 <= n) {
    const u32x4 v = *reinterpret_cast<const u32x4*>(x + e0);
    *reinterpret_cast<f32x4*>(y + e0) = f32x4{bf_lo(v[0]), bf_hi(v[0]), bf_lo(v[1]), bf_hi(v[1])};
    *reinterpret_cast<f32x4*>(y + e0 + 4) = f32x4{bf_lo(v[2]), bf_hi(v[2]), bf_lo(v[3]), bf_hi(v[3])};
  } else {
    for (int64_t e = e0; e < n; ++e) y[e] = bf2f(x[e]);
  }
}

// ===========================================================================
// host side
// ===========================================================================
static int gu_mt(int d_model) { return d_model <= 1024 ? 4 : (d_model <= 2048 ? 2 : 0); }

static size_t gu_lds(int R_ff, int K, int mt) {
  // panel (128 KB) + column table (two bytes per entry: up to 16384 entries)
  return (size_t)16 * mt * (8192 / mt) + (((size_t)R_ff * K * 2 + 15) & ~(size_t)15);
}

// Row slices per token block for the gate/up kernels: with fewer token blocks than CUs, each
// block's h rows are split so that about 256 workgroups run (a workgroup streams the weights of
// its rows only), keeping at least 8 rows (one per wave) per slice; above 4 slices the count is
// a multiple of 8, so that one slice's workgroups share an XCD.
static int gu_slices(int64_t ntb, int R_ff) {
  if (ntb >= 256) return 1;
  const int hmax = R_ff / 8 > 1 ? R_ff / 8 : 1;
  int H = (int)((256 + ntb - 1) / ntb);
  if (H > 4) H = (H + 7) / 8 * 8;
  return H < hmax ? H : hmax;
}

bool split_supported(int B, int d_model, int R_ff, int R_m, int Kg, int Ku, int Kd) {
  if (B != 16 && B != 32) return false;
  if (Kg != Ku || Kg < 1) return false;               // gate and up stream in lockstep
  if (Kd > 128) return false;                         // one or two slot chunks of 64 lanes per down row
  if (d_model % 128) return false;                    // swizzled panel rows
  const int mt = gu_mt(d_model);
  if (mt == 0 || gu_lds(R_ff, Kg, mt) > 163840) return false;
  if (R_m < 1 || R_m * B != d_model) return false;
  if ((R_ff * B) % 8) return false;
  return true;
}

template <int B, int MT, bool NORM, bool INTER, bool SHARED, bool BIAS>
static int launch_gu_b(const GUArgs& a, hipStream_t st) {
  auto kern = gu_kernel<B, MT, NORM, INTER, SHARED, BIAS>;
  static std::atomic<uint64_t> configured{0};
  if (set_lds_limit_once((const void*)kern, 163840, configured)) return -1;
  const int TM = 16 * MT;
  const size_t lds = gu_lds(a.R_ff, a.Kg, MT);
  hipLaunchKernelGGL(kern, dim3((unsigned)((a.N + TM - 1) / TM * a.H)), dim3(512), lds, st, a);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

template <int B, int MT, bool NORM, bool SHARED = false, bool BIAS = false>
static int launch_gu_w12(const GUArgs& a, hipStream_t st) {
  auto kern = gu_kernel_w12<B, MT, NORM, SHARED, BIAS>;
  static std::atomic<uint64_t> configured{0};
  if (set_lds_limit_once((const void*)kern, 163840, configured)) return -1;
  hipLaunchKernelGGL(kern, dim3((unsigned)((a.N + 16 * MT - 1) / (16 * MT))), dim3(64 * gu_w12_waves<B, SHARED>()),
                     gu_lds(a.R_ff, a.Kg, MT), st, a);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

// the bias-free kernels carry no bias code (a bias is an epilogue add and two loads per column)
template <int B, int MT, bool NORM, bool INTER, bool SHARED>
static int launch_gu_t(const GUArgs& a, hipStream_t st) {
  return (a.bg || a.bu) ? launch_gu_b<B, MT, NORM, INTER, SHARED, true>(a, st)
                        : launch_gu_b<B, MT, NORM, INTER, SHARED, false>(a, st);
}

int launch_gu(int B, bool norm, const GUArgs& a0, hipStream_t st) {
  if (a0.N == 0) return 0;
  const int mt = gu_mt(a0.d_model);
  if (mt == 0) return -2;
  GUArgs a = a0;
  a.H = gu_slices((a.N + 16 * mt - 1) / (16 * mt), a.R_ff);
  const bool inter = a.gpre || a.uout;
  // gate and up passing the same column-index buffer share their topology (the reference
  // layer initialises both from the same seed)
  const bool shared = a.cg == a.cu;
  // 12 waves for distinct gate/up topologies at B = 32 with one row slice, no exports and no
  // biases (interleaved runs: headline forward 0.1455 -> 0.1434 ms, looped launches at L = 8
  // 1.305 -> 1.283 ms with the normalising kernel; with a shared topology 8 waves measured as
  // fast or faster, 0.1378 against 0.1381-0.1429 ms)
  if (B == 32 && mt == 4 && a.H == 1 && !inter && !shared && !a.bg && !a.bu)
    return norm ? launch_gu_w12<32, 4, true>(a, st) : launch_gu_w12<32, 4, false>(a, st);
  // B = 16 with one row slice and no exports: 16 waves for every topology and bias combination
  // (at most 113 VGPRs; reference-default layer forward 0.2615 -> 0.2408 ms against 8 waves)
  // the same at 32-token panels (d_model 2048), bias-free or not, shared or not; the normalising
  // fill of 2048-wide rows would spill at 16 waves (the reference's large tile-16 layer, d_ff 8192,
  // 25 %, biases, shared topology, 16384 tokens: 1.276 -> 1.198 ms per forward)
  if (B == 16 && mt == 2 && a.H == 1 && !inter && !norm) {
    const int sel = (shared ? 2 : 0) | ((a.bg || a.bu) ? 1 : 0);
    switch (sel) {
      case 0: return launch_gu_w12<16, 2, false, false, false>(a, st);
      case 1: return launch_gu_w12<16, 2, false, false, true>(a, st);
      case 2: return launch_gu_w12<16, 2, false, true, false>(a, st);
      default: return launch_gu_w12<16, 2, false, true, true>(a, st);
    }
  }
  if (B == 16 && mt == 4 && a.H == 1 && !inter) {
    const int sel = (norm ? 4 : 0) | (shared ? 2 : 0) | ((a.bg || a.bu) ? 1 : 0);
    switch (sel) {
      case 0: return launch_gu_w12<16, 4, false, false, false>(a, st);
      case 1: return launch_gu_w12<16, 4, false, false, true>(a, st);
      case 2: return launch_gu_w12<16, 4, false, true, false>(a, st);
      case 3: return launch_gu_w12<16, 4, false, true, true>(a, st);
      case 4: return launch_gu_w12<16, 4, true, false, false>(a, st);
      case 5: return launch_gu_w12<16, 4, true, false, true>(a, st);
      case 6: return launch_gu_w12<16, 4, true, true, false>(a, st);
      default: return launch_gu_w12<16, 4, true, true, true>(a, st);
    }
  }
#define LBK_GU2(BB, MM, SH)                                                                          \
  if (norm) return launch_gu_t<BB, MM, true, false, SH>(a, st);                                     \
  return inter ? launch_gu_t<BB, MM, false, true, SH>(a, st) : launch_gu_t<BB, MM, false, false, SH>(a, st);
#define LBK_GU(BB, MM)                                                                          \
  if (B == BB && mt == MM) {                                                                    \
    if (shared) { LBK_GU2(BB, MM, true) }                                                       \
    LBK_GU2(BB, MM, false)                                                                      \
  }
  LBK_GU(16, 4) LBK_GU(16, 2) LBK_GU(32, 4) LBK_GU(32, 2)
#undef LBK_GU
#undef LBK_GU2
  return -2;
}

template <int B, int MT, bool BIAS>
static int launch_lin_t(const GUArgs& a, hipStream_t st) {
  auto kern = lin_kernel<B, MT, BIAS>;
  static std::atomic<uint64_t> configured{0};
  if (set_lds_limit_once((const void*)kern, 163840, configured)) return -1;
  const int TM = 16 * MT;
  const size_t lds = gu_lds(a.R_ff, a.Kg, MT);
  hipLaunchKernelGGL(kern, dim3((unsigned)((a.N + TM - 1) / TM * a.H)), dim3(64 * LIN_WAVES), lds, st, a);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

bool lin_supported(int B, int in_features, int R, int K) {
  if (B != 16 && B != 32) return false;
  if (K < 1 || in_features % 128) return false;
  const int mt = gu_mt(in_features);
  if (mt == 0 || gu_lds(R, K, mt) > 163840) return false;
  return (R * B) % 8 == 0;
}

int launch_lin(int B, const GUArgs& a0, hipStream_t st) {
  if (a0.N == 0) return 0;
  GUArgs a = a0;   // the up operands are the gate's (never read as weights)
  a.pu = a.pg;
  a.cu = a.cg;
  a.Ku = a.Kg;
  const int mt = gu_mt(a.d_model);
  if (mt == 0) return -2;
  a.H = gu_slices((a.N + 16 * mt - 1) / (16 * mt), a.R_ff);
#define LBK_LIN(BB, MM)                                                                     \
  if (B == BB && mt == MM) return a.bg ? launch_lin_t<BB, MM, true>(a, st) : launch_lin_t<BB, MM, false>(a, st);
  LBK_LIN(16, 4) LBK_LIN(16, 2) LBK_LIN(32, 4) LBK_LIN(32, 2)
#undef LBK_LIN
  return -2;
}

template <int B, int MT, int RPW, int NW, int SC, int KC>
static int launch_dn_k(const DNArgs& a0, hipStream_t st) {
  const int TM = 16 * MT;
  constexpr size_t lds = 2 * (size_t)TM * SC * 2;   // two stages
  DNArgs a = a0;
  const int64_t ntb = (a.N + TM - 1) / TM;
  a.nrg = (a.R_m + NW * RPW - 1) / (NW * RPW);
  const int64_t grid = a.nrg == 1 ? ntb : 8 * a.nrg * ((ntb + 7) / 8);
  const bool core = a.tdepth || a.inj_e;
  auto kern = a.bd ? (core ? dn_kernel<B, MT, RPW, NW, SC, true, true, KC>
                           : dn_kernel<B, MT, RPW, NW, SC, true, false, KC>)
                   : (core ? dn_kernel<B, MT, RPW, NW, SC, false, true, KC>
                           : dn_kernel<B, MT, RPW, NW, SC, false, false, KC>);
  if (lds > 65536 && hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                         hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess)
    return -1;
  hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(64 * NW), lds, st, a);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

// rows with up to 64 slots take one lane per slot; up to 128 (the reference's tile-16 layers at
// density 1.0 and d_ff 2048) two slot chunks per lane
template <int B, int MT, int RPW, int NW, int SC>
static int launch_dn_t(const DNArgs& a, hipStream_t st) {
  return a.Kd > 64 ? launch_dn_k<B, MT, RPW, NW, SC, 2>(a, st) : launch_dn_k<B, MT, RPW, NW, SC, 1>(a, st);
}

// One down row per wave (a workgroup covers DN_WAVES rows; the row groups of one token block
// share an XCD): few accumulator registers per wave, four waves per SIMD.  (128-token
// workgroups, which halve the weight bytes each CU streams, measured slower at the headline
// geometry: 154 us with 8 waves of two rows and 256-column stages, 161 us with 16 waves of one
// row, against 144 us; the smaller stages add padding and per-stage imbalance.)
// the deep-ring down kernel on 64-token blocks, rows of at most 64 slots
constexpr int DNF_RING = 4;
template <int B>
static int launch_dnf(const DNArgs& a0, hipStream_t st) {
  constexpr int TM = 64;
  constexpr size_t lds = 2 * (size_t)TM * DN_STAGE_COLS * 2;   // two stages
  DNArgs a = a0;
  const int64_t ntb = (a.N + TM - 1) / TM;
  a.nrg = (a.R_m + DN_WAVES - 1) / DN_WAVES;
  const int64_t grid = a.nrg == 1 ? ntb : 8 * a.nrg * ((ntb + 7) / 8);
  auto kern = a.bd ? dnf_kernel<B, DNF_RING, true> : dnf_kernel<B, DNF_RING, false>;
  if (hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                          (int)lds) != hipSuccess)
    return -1;
  hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(64 * DN_WAVES), lds, st, a);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_dn(int B, const DNArgs& a, hipStream_t st) {
  if (a.N == 0) return 0;
  // the deep-ring kernel takes the plain forward (with an fp32 state, as the looped block's
  // iterations run it, it measured slower: L = 8 at the headline geometry 1.270 -> 1.281 ms)
  const bool plain = !a.state && !a.tdepth && !a.inj_e && a.out && a.Kd <= 64;
  // Fewer 64-token blocks than the 16-row groups need to fill the CUs: smaller workgroups with
  // longer stages, so that more of them run and each walks fewer stages -- 16 tokens and 4 rows
  // per workgroup with 2048-column stages (1024 for B = 16) while they number at most 128, else
  // 32 tokens and 8 rows with 1024-column stages.  Measured at d_model 1024, d_ff 4096, B = 32
  // (forward per N = 64 / 256 / 1024 / 2048 / 4096): 20.0 / 21.0 / 28.6 / 37.3 / 62.3 us, against
  // 38.4 / 40.3 / 44.4 / 50.9 / 61.9 with 64 tokens and 4 rows at 256-column stages.
  if ((a.N + 63) / 64 * ((a.R_m + 15) / 16) < 256) {
    if ((a.N + 15) / 16 * ((a.R_m + 3) / 4) <= 128) {
      if (B == 16) return launch_dn_t<16, 1, 1, 4, 1024>(a, st);
      if (B == 32) return launch_dn_t<32, 1, 1, 4, 2048>(a, st);
    }
    if (B == 16) return launch_dn_t<16, 2, 1, 8, 1024>(a, st);
    if (B == 32) return launch_dn_t<32, 2, 1, 8, 1024>(a, st);
  }
  // B = 16 (half the accumulators) with more than 16 down rows: two rows per wave, so half the
  // row groups re-read h (d_model 1024, d_ff 4096: forward 0.301 -> 0.293 ms)
  if (B == 16 && a.R_m > DN_WAVES) return launch_dn_t<16, 4, 2, DN_WAVES, DN_STAGE_COLS>(a, st);
  if (B == 16) return launch_dn_t<16, 4, 1, DN_WAVES, DN_STAGE_COLS>(a, st);
  if (B == 32 && plain) return launch_dnf<32>(a, st);
  if (B == 32) return launch_dn_t<32, 4, 1, DN_WAVES, DN_STAGE_COLS>(a, st);
  return -2;
}

template <int B, int MT, bool SHARED, int RPW, bool BIAS>
static int launch_looped_b(const LoopArgs& a0, hipStream_t st) {
  auto kern = looped_kernel<B, MT, SHARED, RPW, BIAS>;
  static std::atomic<uint64_t> configured{0};
  if (set_lds_limit_once((const void*)kern, 163840, configured)) return -1;
  LoopArgs a = a0;
  int kmax = 0;
  for (int c = 0; c < a.n_core; ++c) kmax = a.core[c].Kg > kmax ? a.core[c].Kg : kmax;
  const int TM = 16 * MT;
  const size_t dn_lds = 2 * (size_t)TM * DN_STAGE_COLS * 2;
  const size_t g_lds = gu_lds(a.gu.R_ff, kmax, MT);
  size_t lds = g_lds > dn_lds ? g_lds : dn_lds;
  a.red_off = looped_red_offset<MT>(a.gu.R_ff, kmax);
  const size_t r_end = a.red_off + (size_t)9 * TM * 4;
  lds = lds > r_end ? lds : r_end;
  if (lds > 163840) return -2;
  hipLaunchKernelGGL(kern, dim3((unsigned)((a.gu.N + TM - 1) / TM)), dim3(512), lds, st, a);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

template <int B, int MT, bool SHARED, int RPW>
static int launch_looped_t(const LoopArgs& a, hipStream_t st) {
  bool bias = false;
  for (int c = 0; c < a.n_core; ++c) bias = bias || a.core[c].bg || a.core[c].bu || a.core[c].bd;
  return bias ? launch_looped_b<B, MT, SHARED, RPW, true>(a, st) : launch_looped_b<B, MT, SHARED, RPW, false>(a, st);
}

// The persistent looped block takes the shapes of the two-kernel path with MT = 4
// (d_model <= 1024): its LDS holds either the gate/up panel or the two down stages.
bool looped_persistent_supported(int B, int d_model, int R_ff, int R_m, int Kg, int Ku, int Kd) {
  // four down rows per wave: a stage's hit list holds up to 4 * (Kd + 1) <= 256 entries
  return split_supported(B, d_model, R_ff, R_m, Kg, Ku, Kd) && Kd <= 63 && gu_mt(d_model) == 4 &&
         looped_red_offset<4>(R_ff, Kg) + (size_t)9 * 64 * 4 <= 163840;
}

int launch_looped(int B, const LoopArgs& a, hipStream_t st) {
  if (a.gu.N == 0 || a.L <= 0) return 0;
  if (gu_mt(a.gu.d_model) != 4 || a.n_core < 1 || a.n_core > kMaxCore) return -2;
  // one kernel shape for all core blocks: either every block shares its gate/up topology or none
  const bool shared = a.core[0].cg == a.core[0].cu;
  for (int c = 1; c < a.n_core; ++c)
    if ((a.core[c].cg == a.core[c].cu) != shared) return -2;
  // four down rows per wave: the 32 rows of a 1024-wide model in one group, h staged once
  // (measured at the looped-block geometry: 1.50 ms against 1.58 with two rows per wave in
  // two groups and 1.87 with one row per wave in four)
#define LBK_LOOP(BB)                                                                        \
  if (B == BB) return shared ? launch_looped_t<BB, 4, true, 4>(a, st) : launch_looped_t<BB, 4, false, 4>(a, st);
  LBK_LOOP(16)
  LBK_LOOP(32)
#undef LBK_LOOP
  return -2;
}

int launch_bf16_to_f32(const uint16_t* x, int64_t n, float* y, hipStream_t st) {
  if (n == 0) return 0;
  if ((reinterpret_cast<uintptr_t>(x) & 15) || (reinterpret_cast<uintptr_t>(y) & 15)) return -2;
  hipLaunchKernelGGL(bf16_to_f32_kernel, dim3((unsigned)((n + 2047) / 2048)), dim3(256), 0, st, x, n, y);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace lbk
