// lbk_internal.h — launcher interfaces shared between the kernel files and the C ABI.
#pragma once
#include <atomic>

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace lbk {

struct RowblockLaunch {
  const uint16_t* x;   // [N, ldx] activations
  int64_t N;
  int64_t ldx;
  int C;               // input column blocks (in_features / B)
  int R;               // block rows (output features / B)
  const uint16_t* v0; const int32_t* c0; int K0;   // weight (gate for MODE 1)
  const uint16_t* v1; const int32_t* c1; int K1;   // up weight (MODE 1 only)
  const float* bias;                                // optional: the product's (MODE 0, 2) or gate's (MODE 1)
  const float* bias1;                               // optional: up's bias (MODE 1)
  const uint16_t* resid; int64_t ldr;              // MODE 2, optional
  uint16_t* y; int64_t ldy;
  uint16_t* aux0; uint16_t* aux1; int64_t ldaux;    // MODE 1 optional pre-activations
};

// mode: 0 = product (+bias), 1 = gate/up with SiLU*mul, 2 = down (+residual)
int launch_rowblock(int B, int mode, const RowblockLaunch& a, hipStream_t st);

// bf16 tiles -> fragment-major packed tiles (PackedTile<B> in lbk_device.h); dead
// slots (col < 0 or >= C) become zero tiles and one zero tile is appended at index ntiles
int launch_pack_bf16(const uint16_t* values, const int32_t* col, int64_t ntiles, int C, int B, uint32_t* packed,
                     hipStream_t st);
size_t packed_bf16_bytes(int64_t ntiles, int B);   // includes the appended zero tile
// up to three weights packed by one launch (ndw is filled in by the launcher)
// Raises a kernel's dynamic LDS limit once per device: the attribute belongs to the device that
// is current at the call (the device of the stream the kernel is then launched on).
inline int set_lds_limit_once(const void* kern, int bytes, std::atomic<uint64_t>& done) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return -1;
  const uint64_t bit = (dev >= 0 && dev < 64) ? (1ull << dev) : 0ull;
  if (bit && (done.load(std::memory_order_acquire) & bit)) return 0;
  if (hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, bytes) != hipSuccess) return -1;
  done.fetch_or(bit, std::memory_order_release);
  return 0;
}

struct PackJob {
  const uint16_t* values; const int32_t* col; int64_t ntiles; int C; uint32_t* packed; int64_t ndw;
  int gu_layout;   // 1: column order of the gate/up kernel's swapped product (B = 32)
};
struct PackJobs {
  static constexpr int kMax = 3;
  PackJob job[kMax];
  int64_t first[kMax];   // first workgroup of each job
  int n;
};
int launch_pack_bf16_multi(const PackJob* jobs, int n, int B, hipStream_t st);


// two-kernel SwiGLU: gate/up (+optional RMSNorm prologue) -> h, then down (+residual / fp32 state)
struct GUArgs {
  const uint16_t* x;        // [N, d_model] bf16 input (plain mode)
  const float* xf;          // [N, d_model] fp32 state (RMSNorm mode)
  int64_t N;
  int d_model;
  const float* norm_scale;  // RMSNorm mode: [d_model]
  float eps;
  const void* pg; const int32_t* cg; int Kg;   // packed gate tiles
  const void* pu; const int32_t* cu; int Ku;   // packed up tiles
  int R_ff;
  uint16_t* h;              // [N, d_ff] silu(g) * u
  uint16_t* gpre;           // [N, d_ff] optional gate pre-activation
  uint16_t* uout;           // [N, d_ff] optional up output
  const float* bg; const float* bu;   // optional [d_ff] gate / up biases (added before SiLU*mul)
  int H;                    // row slices per token block (set by the launcher)
  // looped core: per-token depths; a token block whose rows all have tdepth[t] <= it is skipped
  const int32_t* tdepth; int it;
  int reload_table;         // looped kernel: a gate/up phase on a ready panel re-reads the column table
};
struct DNArgs {
  const uint16_t* h;        // [N, d_ff]
  int64_t N;
  int64_t d_ff;
  int d_model;
  const void* pd; const int32_t* cd; int Kd;   // packed down tiles
  int R_m;
  int C_d;                  // d_ff / B
  const uint16_t* resid;    // optional bf16 residual [N, d_model]
  float* state;             // optional fp32 state [N, d_model]: read as residual, written back
  uint16_t* out;            // optional bf16 output [N, d_model]
  int nrg;                  // row groups per token block (set by the launcher)
  const float* bd;          // optional [d_model] down bias
  // looped core (state mode): rows with tdepth[t] <= it keep their state; when inj_e is set the
  // rows that run the next iteration (it + 1 < tdepth[t]) then take its injection
  // state = decay * state + dt * e (inj_coef: decay [d_model], then dt [d_model])
  const int32_t* tdepth; int it;
  const uint16_t* inj_e; const float* inj_coef;
};
bool split_supported(int B, int d_model, int R_ff, int R_m, int Kg, int Ku, int Kd);
// plain product y[N, R*B] = x[N, in] W (+ bias in a.bg) on packed tiles (a.pg, a.cg, a.Kg, a.R_ff,
// a.d_model = in, output in a.h with row stride R*B): the gate/up kernel's gate stream alone
bool lin_supported(int B, int in_features, int R, int K);
int launch_lin(int B, const GUArgs& a, hipStream_t st);
// looped block in one launch: gate/up (RMSNorm of the fp32 state) and down per token block
// for all L iterations; gu.xf == dn.state == the fp32 state, gu.h == dn.h
// one core block of the persistent looped kernel (packed tiles, columns, norm scale, biases)
struct CoreW {
  const void* pg; const void* pu; const void* pd;
  const int32_t* cg; const int32_t* cu; const int32_t* cd;
  int Kg, Kd;
  const float* norm_scale;
  const float* bg; const float* bu; const float* bd;
};
constexpr int kMaxCore = 8;
struct LoopArgs {
  GUArgs gu;                 // shared fields (the per-block ones come from core[])
  DNArgs dn;                 // dn.out: bf16 result, written by the last iteration
  const uint16_t* h_in;      // [N, d_model] bf16 initial state
  int L;
  int n_core;                // core blocks applied in order per iteration (core[0] only: gu/dn as given)
  CoreW core[kMaxCore];
  const int32_t* tdepth;     // optional [N] per-token depths (iterations a row runs)
  const uint16_t* e;         // optional [N, d_model] injection input, applied at every iteration's start
  const float* inj_coef;     // decay [d_model], dt [d_model] (with e)
  size_t red_off;            // LDS byte offset of the reduction area (after the widest column table)
};
bool looped_persistent_supported(int B, int d_model, int R_ff, int R_m, int Kg, int Ku, int Kd);
int launch_looped(int B, const LoopArgs& a, hipStream_t st);
int launch_gu(int B, bool norm, const GUArgs& a, hipStream_t st);
int launch_dn(int B, const DNArgs& a, hipStream_t st);
int launch_bf16_to_f32(const uint16_t* x, int64_t n, float* y, hipStream_t st);
// looped core helpers (lbk_bf16.hip): injection coefficients (decay, dt per feature, when log_A)
// and per-token depths (tdepth[t] = depths[t / seq_len], when depths), in one launch
int launch_core_prep(const float* log_A, const float* log_dt, int d, float* coef, const int32_t* depths,
                     int64_t seq_len, int64_t N, int32_t* tdepth, hipStream_t st);
// state = float(h_in), then the first iteration's injection on the rows that run it (e optional)
int launch_core_init(const uint16_t* h_in, const uint16_t* e, const float* coef, const int32_t* tdepth, int L,
                     int64_t N, int d, float* state, hipStream_t st);
// state update of a core block computed outside the split kernels (y bf16): rows running
// iteration it add y (the others keep their state), then with e the next iteration's injection
// on rows that run it; out (optional) = bf16(state)
int launch_core_update(float* state, const uint16_t* y, const int32_t* tdepth, int it, const uint16_t* e,
                       const float* coef, int64_t N, int d, uint16_t* out, hipStream_t st);

// decode-shaped SwiGLU FFN (N <= 16): gate/up kernel, then down kernel
struct DecodeArgs {
  const uint16_t* x; int N; int d_model;
  const uint16_t* vg; const int32_t* cg; int Kg;
  const uint16_t* vu; const int32_t* cu; int Ku;
  int R_ff;
  const uint16_t* vd; const int32_t* cd; int Kd;
  int R_m;
  const uint16_t* resid;     // optional [N, d_model]
  uint16_t* out;             // [N, d_model]
  uint16_t* h;               // [N, d_ff] workspace (or the caller's h)
  const float* bg; const float* bu; const float* bd;   // optional biases
  float* state;              // optional fp32 [N, d_model]: added to the product and written back
                             // (resid is then ignored; out, if given, gets the bf16 of the sum)
};
bool decode_supported(int Kg, int Ku, int Kd);
int launch_decode(int B, const DecodeArgs& a, hipStream_t st);

int launch_rmsnorm(const uint16_t* x, int64_t N, int d, const float* scale, float eps, uint16_t* out,
                   hipStream_t st);
// fp32 rows -> bf16 RMSNorm (d % 8 == 0, 16-byte aligned operands)
int launch_rmsnorm_f32(const float* x, int64_t N, int d, const float* scale, float eps, uint16_t* out,
                       hipStream_t st);
size_t rmsnorm_bwd_bytes(int64_t N, int d);   // fp32 dscale partials of the workgroups
// fp32 column sums out[C] of a bf16 [N, C] matrix (deterministic: per-64-row partials in part)
size_t colsum_bytes(int64_t N, int C);
int launch_colsum(const uint16_t* a, int64_t N, int C, int64_t lda, float* part, float* out, hipStream_t st);
int launch_rmsnorm_bwd(const uint16_t* x, const uint16_t* dy, int64_t N, int d, const float* scale, float eps,
                       uint16_t* dx, float* dscale, float* part, hipStream_t st);
int launch_injection(const uint16_t* h, const uint16_t* e, const float* log_A, const float* log_dt, int64_t N,
                     int d, uint16_t* out, hipStream_t st);
size_t injection_bwd_bytes(int64_t N, int d);   // fp32 column partials (two per row block)
int launch_injection_bwd(const uint16_t* g, const uint16_t* h, const uint16_t* e, const float* log_A,
                         const float* log_dt, int64_t N, int d, uint16_t* dh, uint16_t* de, float* d_log_A,
                         float* d_log_dt, float* part, hipStream_t st);

// ---- ternary / int8
int launch_quantize_act(const uint16_t* x, int64_t N, int F, int64_t ldx, int8_t* xq, float* sx, hipStream_t st);
int launch_pack_ternary(const int8_t* t, int R, int K, int B, uint32_t* packed, hipStream_t st);
int launch_ternary_quantize_weights(const uint16_t* values, int R, int K, int B, uint32_t* packed, float* scales,
                                    hipStream_t st);

struct TernaryLaunch {
  const int8_t* xq; const float* sx; int64_t N; int C;   // activations [N, C*B] int8
  const uint32_t* p0; const float* s0; const int32_t* c0; int K0;
  const uint32_t* p1; const float* s1; const int32_t* c1; int K1;   // gate/up mode only
  int R;
  const uint16_t* resid;      // [N, R*B] bf16, optional (product mode)
  uint16_t* y;                // [N, R*B] bf16
  int32_t* partials;          // [N, R, K0, B] int32, optional (product mode)
  // optional accumulators before scaling, [N, R*B]: acc = sum_k m * P of weight 0 (and of
  // weight 1 in gate/up mode), pre = f32(f32(acc) * 2^-e) * sx
  int32_t* acc0; int32_t* acc1; float* pre0; float* pre1;
};
// mode: 0 = product, 1 = gate/up with SiLU*mul (y = h bf16)
int launch_ternary(int B, int mode, const TernaryLaunch& a, hipStream_t st);

// two-kernel ternary SwiGLU (B = 64) on prepared weights (launch_tprep)
typedef uint32_t tu32x4 __attribute__((ext_vector_type(4)));
struct TGUArgs {
  const int8_t* xq; const float* sx; int64_t N; int d_model;
  const tu32x4* twg; const int32_t* mg; const float* rmg; const int32_t* cg;   // gate
  const tu32x4* twu; const int32_t* mu; const float* rmu; const int32_t* cu;   // up
  int K;                    // slots per row (gate and up alike)
  int R_ff;
  int H;                    // block-row slices per token block
  uint16_t* h;              // [N, d_ff] bf16
  float* hmax;              // [H, N] max |h| of each slice
  // optional [N, d_ff]: integer accumulators sum_k m * P and pre-activations f32(f32(acc) * 2^-e) * sx
  int32_t* acc_g; int32_t* acc_u; float* g_pre; float* u_pre;
};
struct TDNArgs {
  const uint16_t* h; const float* hmax; int H; int64_t N; int d_ff; int d_model;
  const tu32x4* twd; const int32_t* md; const float* rmd; const int32_t* cd; int Kd;
  int R_m; int C_d;
  const uint16_t* resid;    // optional [N, d_model]
  uint16_t* out;            // [N, d_model]
  int8_t* hq_out;           // optional [N, d_ff]
  float* sh_out;            // optional [N]
  int32_t* acc_d;           // optional [N, d_model]: integer accumulators sum_k m * P
  int G;                    // down row groups per token block (set by the launcher)
};
// bytes of one prepared tile of weight `which` (0 gate, 1 up: int8 MFMA fragments; 2 down:
// 2-bit t + 1 words)
constexpr int tprep_tile_bytes(int which) { return which < 2 ? 4096 : 1024; }
size_t tprep_bytes(int64_t ntiles, int R, int which);
struct TPrepWeight {
  const uint32_t* packed; const float* s; const int32_t* col; int R, K, C;
};
struct TPrepJob {
  const uint32_t* packed; const float* s; const int32_t* col; int R, K, C;
  bool int8;
  tu32x4* tw; int32_t* mval; float* rmul;
};
struct TPrepJobs {
  TPrepJob job[3];
  int64_t first[3];   // first workgroup of each weight
};
// prepares gate, up and down (w[0..2]) into out[0..2] (tprep_bytes each) in one launch; with
// run = false only the pointers into out are returned (weights prepared earlier)
int launch_tprep(const TPrepWeight (&w)[3], void* const (&out)[3], const tu32x4* (&tw)[3],
                 const int32_t* (&mval)[3], const float* (&rmul)[3], hipStream_t st,
                 bool run = true);
bool tsplit_supported(int B, int d_model, int R_ff, int R_m, int Kg, int Ku, int Kd);
int tgu_slices(int64_t N, int R_ff);
int launch_tgu(const TGUArgs& a, hipStream_t st);
int launch_tdn(const TDNArgs& a, hipStream_t st);

// ---- backward of the SwiGLU FFN (lbk_bwd.hip)
// transposed topology: for input column block c, cnt[c] slots e = r*K + k with col[e] == c at
// list[c*R*K ...], ascending
struct TListJob {
  const int32_t* col; int R, K, C;
  int32_t* cnt; int32_t* list;   // [C], [C, R*K]
};
struct TListJobs {
  static constexpr int kMax = 3;
  TListJob job[kMax];
  int64_t first[kMax];
  int n;
};
int launch_tlist(const TListJob* jobs, int n, hipStream_t st);
// out[:, c*B ..] = sum over sources and their slots of column block c of A[:, r*B ..] W[e]^T
struct TProdSrc {
  const uint16_t* a; int64_t lda;   // activations [N, R*B]
  const uint16_t* w; int K;         // raw tiles [R, K, B, B]
  const int32_t* cnt; const int32_t* list; int64_t cap;
  // e / K = (umulhi(e, kmul) + e) >> ksh for 0 <= e < 2^31 (set by the launchers that use it)
  uint32_t kmul; int ksh;
};
struct TProdArgs {
  TProdSrc src[2]; int nsrc;
  int64_t N; int C; int64_t ldo;    // output [N, C*B], row stride ldo (also of g, u, resid)
  const uint16_t* g; const uint16_t* u; uint16_t* dg; uint16_t* du;   // mode 0
  const uint16_t* resid; uint16_t* out;                               // mode 1 (resid optional)
  int nsl;                          // output column slices per token block (set by the launcher)
};
// mode 0: dh -> dg, du (SiLU*mul backward); mode 1: out = product + resid
int launch_tprod(int B, int mode, const TProdArgs& a, hipStream_t st);
// tile gradients dW[e] = X[:, col(e)]^T G[:, row(e)] through fp32 per-chunk partials
struct DWJob {
  const uint16_t* x; int64_t ldx;    // [N, C*B]
  const uint16_t* gy; int64_t ldg;   // [N, R*B]
  const int32_t* col; int R, K, C;
  float* part;                       // [nchunk, R*K, B, B]
  uint16_t* dw;                      // [R, K, B, B] bf16
  // optional transposed topology of launch_tlist (per column block c: tcnt[c] slots e at
  // tlist[c * R * K ..]); lets a weight with wide input rows and narrow output rows (the down
  // projection) stage its G rows whole and walk the slots of each input column block
  const int32_t* tcnt; const int32_t* tlist;
  int chunk, nchunk;                 // tokens per partial tile and their count (set by launch_dw)
};
struct DWJobs {
  static constexpr int kMax = 3;
  DWJob job[kMax];
  int64_t first[kMax], rfirst[kMax];
  int n; int64_t N; int chunk; int nchunk;
};
constexpr int DW_CHUNK = 2048;   // tokens per partial tile
// tokens per partial tile of a weight [R, K, B, B] with C input column blocks, G rows of ldg
// elements and N tokens: DW_CHUNK / 2 where the tile gradients take the transposed-list kernel
// (input rows too wide to stage whole, output rows at most 1024 wide, and at least 256 of its
// workgroups at that chunk), else DW_CHUNK
int dw_job_chunk(int B, int R, int C, int64_t ldg, int64_t N);
// per job: chunk = dw_job_chunk(...) (a multiple of 64), partials [ceil(N / chunk), R*K, B, B]
int launch_dw(int B, const DWJob* jobs, int n, int64_t N, hipStream_t st);

// ---- topology transforms (lbk_topo.hip)
int launch_topo_count(const uint8_t* alive, int R, int K, int32_t* counts, int32_t* mx, hipStream_t st);
int launch_topo_compact(const uint16_t* values, const int32_t* col, const uint8_t* alive, int R, int K, int B,
                        int K_new, uint16_t* ov, int32_t* oc, uint8_t* oa, hipStream_t st);
int launch_topo_importance(const int32_t* c1, const uint8_t* a1, int64_t n1, const uint8_t* a2, int R2, int K2,
                           int C_ff, float* imp, hipStream_t st);
int launch_topo_perm(const float* imp, int C, int32_t* perm, hipStream_t st);
int launch_topo_apply(const uint16_t* values, const int32_t* col, const uint8_t* alive, int R, int K, int B,
                      const int32_t* perm, int C_ff, int column, uint16_t* ov, int32_t* oc, uint8_t* oa,
                      hipStream_t st);
int launch_topo_kactive(const int32_t* col, const uint8_t* alive, int64_t n, int tpm, int32_t* out, hipStream_t st);
int launch_topo_gather(const void* src, int64_t row_bytes, const int32_t* perm, int n_src, int n_dst, void* dst,
                       hipStream_t st);
int launch_topo_csc(const int32_t* col, int R, int K, int C, int32_t* col_ptr, int32_t* entries, hipStream_t st);

// storage-format bridges (lbk_format.hip); elem_bytes 2 = bf16, 4 = fp32
int launch_fmt_from_dense(const void* dense, int64_t ld, int elem_bytes, int R, int C, int B, const int32_t* col,
                          int K, void* values, hipStream_t st);
int launch_fmt_to_dense(const void* values, const int32_t* col, int R, int K, int B, int C, int elem_bytes,
                        void* dense, int64_t ld, hipStream_t st);
int launch_fmt_topk(const void* dense, int64_t ld, int elem_bytes, int R, int C, int B, int K, int32_t* col_out,
                    hipStream_t st);
int launch_fmt_ternary_check(const uint32_t* words, int64_t n, int32_t* bad, hipStream_t st);

int launch_check_columns(const int32_t* col, int64_t count, int C, int32_t* bad, hipStream_t st);

}  // namespace lbk
