// lbk_internal.h — launcher interfaces shared between the kernel files and the C ABI.
#pragma once

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
  const float* bias;                                // MODE 0, optional
  const uint16_t* resid; int64_t ldr;              // MODE 2, optional
  uint16_t* y; int64_t ldy;
  uint16_t* aux0; uint16_t* aux1; int64_t ldaux;    // MODE 1 optional pre-activations
};

// mode: 0 = product (+bias), 1 = gate/up with SiLU*mul, 2 = down (+residual)
int launch_rowblock(int B, int mode, const RowblockLaunch& a, hipStream_t st);

struct PanelArgs {
  const uint16_t* x;       // [N, d_model]
  int64_t N;
  int d_model;
  const uint16_t* vg; const int32_t* cg; int Kg;
  const uint16_t* vu; const int32_t* cu; int Ku;
  int R_ff;
  const uint16_t* vd; const int32_t* cd; int Kd;
  int R_m;
  int add_residual;        // forward only: accumulate on top of x
  const float* norm_scale; // looped only: [d_model]
  float eps;
  int L;                   // looped only: number of applications
  uint16_t* out;           // [N, d_model]
};

size_t panel_lds_bytes(int B, int d_model, int R_ff, int R_m);
bool panel_supported(int B, int d_model, int R_ff, int R_m, int Kd);
int launch_panel(int B, bool norm, const PanelArgs& p, hipStream_t st);

int launch_rmsnorm(const uint16_t* x, int64_t N, int d, const float* scale, float eps, uint16_t* out,
                   hipStream_t st);
int launch_injection(const uint16_t* h, const uint16_t* e, const float* log_A, const float* log_dt, int64_t N,
                     int d, uint16_t* out, hipStream_t st);

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
};
// mode: 0 = product, 1 = gate/up with SiLU*mul (y = h bf16)
int launch_ternary(int B, int mode, const TernaryLaunch& a, hipStream_t st);
int launch_check_columns(const int32_t* col, int64_t count, int C, int32_t* bad, hipStream_t st);

}  // namespace lbk
