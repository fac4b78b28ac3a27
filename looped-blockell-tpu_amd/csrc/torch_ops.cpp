// torch_ops.cpp — thin PyTorch-ROCm extension: registers the titan:: operators
// over the C ABI of liblbk.so (include/lbk.h).
//
// The reference registers the same schemas for its CUDA kernels
// (csrc/block_ell/block_ell_ops.cpp:49-98, csrc/loop/loop_ops.cpp:36-67); the
// schemas below keep those names, arguments and return types, and add the ops
// this library exposes beyond them (block_ell_matmul, looped_swiglu, rmsnorm,
// diagonal_injection and the ternary family).  PyTorch on ROCm dispatches HIP
// tensors under the CUDA key.  Every op checks its inputs with TORCH_CHECK
// (a Python RuntimeError), makes inputs contiguous, allocates its outputs and
// queues the work on the current stream; C ABI status codes become errors.
#include <ATen/ATen.h>
#include <ATen/hip/impl/HIPGuardImplMasqueradingAsCUDA.h>
#include <ATen/hip/impl/HIPStreamMasqueradingAsCUDA.h>
#include <torch/csrc/autograd/autograd_not_implemented_fallback.h>
#include <torch/library.h>

#include <vector>

#include "lbk.h"

namespace {

void* cur_stream(const at::Tensor& t) {
  return (void*)c10::hip::getCurrentHIPStreamMasqueradingAsCUDA(t.device().index()).stream();
}

#define LBK_CALL(opname, expr)                                                                    \
  do {                                                                                            \
    const int _st = (expr);                                                                       \
    TORCH_CHECK(_st == LBK_OK, "titan::" opname ": ", lbk_status_string(_st), " (status ", _st, ")"); \
  } while (0)

const uint16_t* bf(const at::Tensor& t) { return reinterpret_cast<const uint16_t*>(t.data_ptr()); }
uint16_t* bfm(at::Tensor& t) { return reinterpret_cast<uint16_t*>(t.data_ptr()); }

void check_gpu(const at::Tensor& t, const char* op, const char* name) {
  TORCH_CHECK(t.is_cuda(), "titan::", op, ": ", name, " must be a GPU (HIP) tensor");
}

// values [R,K,B,B] bf16 + col_idx [R,K] int32 -> lbk_bell (tensors made contiguous in place)
lbk_bell make_bell(at::Tensor& v, at::Tensor& c, const char* op, const char* name) {
  check_gpu(v, op, name);
  check_gpu(c, op, name);
  TORCH_CHECK(v.scalar_type() == at::kBFloat16, "titan::", op, ": ", name, " values must be bf16");
  TORCH_CHECK(c.scalar_type() == at::kInt, "titan::", op, ": ", name, " col_indices must be int32");
  TORCH_CHECK(v.dim() == 4 && v.size(2) == v.size(3), "titan::", op, ": ", name,
              " values must be [R, K, B, B], got ", v.sizes());
  TORCH_CHECK(c.dim() == 2 && c.size(0) == v.size(0) && c.size(1) == v.size(1), "titan::", op, ": ", name,
              " col_indices must be [R, K] matching values, got ", c.sizes());
  v = v.contiguous();
  c = c.contiguous();
  return lbk_bell{bf(v), c.data_ptr<int32_t>(), (int32_t)v.size(0), (int32_t)v.size(1), (int32_t)v.size(2)};
}

lbk_bell_ternary make_tern(at::Tensor& p, at::Tensor& s, at::Tensor& c, const char* op, const char* name) {
  check_gpu(p, op, name);
  check_gpu(s, op, name);
  check_gpu(c, op, name);
  TORCH_CHECK(p.scalar_type() == at::kInt || p.scalar_type() == at::kUInt32, "titan::", op, ": ", name,
              " packed must be int32/uint32 words");
  TORCH_CHECK(s.scalar_type() == at::kFloat, "titan::", op, ": ", name, " scales must be fp32");
  TORCH_CHECK(c.scalar_type() == at::kInt, "titan::", op, ": ", name, " col_indices must be int32");
  TORCH_CHECK(p.dim() == 4 && p.size(3) * 16 == p.size(2), "titan::", op, ": ", name,
              " packed must be [R, K, B, B/16], got ", p.sizes());
  TORCH_CHECK(s.dim() == 2 && s.size(0) == p.size(0) && s.size(1) == p.size(1), "titan::", op, ": ", name,
              " scales must be [R, K]");
  TORCH_CHECK(c.dim() == 2 && c.size(0) == p.size(0) && c.size(1) == p.size(1), "titan::", op, ": ", name,
              " col_indices must be [R, K]");
  p = p.contiguous();
  s = s.contiguous();
  c = c.contiguous();
  return lbk_bell_ternary{reinterpret_cast<const uint32_t*>(p.data_ptr()), s.data_ptr<float>(),
                          c.data_ptr<int32_t>(), (int32_t)p.size(0), (int32_t)p.size(1), (int32_t)p.size(2)};
}

at::Tensor check_x2d(const at::Tensor& x, const char* op) {
  check_gpu(x, op, "x");
  TORCH_CHECK(x.scalar_type() == at::kBFloat16, "titan::", op, ": x must be bf16");
  TORCH_CHECK(x.dim() == 2, "titan::", op, ": x must be 2D [N, d_model], got ", x.sizes());
  return x.contiguous();
}

at::Tensor workspace(size_t bytes, const at::Tensor& like) {
  return at::empty({(int64_t)std::max<size_t>(bytes, 1)}, like.options().dtype(at::kByte));
}

// ------------------------------------------------------------------ bf16 SwiGLU
// optional fp32 bias of `n` elements on x's device (made contiguous), or undefined
at::Tensor opt_bias(const c10::optional<at::Tensor>& b, int64_t n, const at::Tensor& x, const char* op,
                    const char* name) {
  if (!b.has_value() || !b->defined()) return at::Tensor();
  check_gpu(*b, op, name);
  TORCH_CHECK(b->numel() == n, "titan::", op, ": ", name, " must have ", n, " elements, got ", b->numel());
  return b->to(x.device(), at::kFloat).contiguous();
}
const float* fptr(const at::Tensor& t) { return t.defined() ? t.data_ptr<float>() : nullptr; }

std::vector<at::Tensor> swiglu_impl(const at::Tensor& x_, at::Tensor vg, at::Tensor cg, at::Tensor vu,
                                    at::Tensor cu, at::Tensor vd, at::Tensor cd, bool add_residual,
                                    bool intermediates, const c10::optional<at::Tensor>& bg_ = c10::nullopt,
                                    const c10::optional<at::Tensor>& bu_ = c10::nullopt,
                                    const c10::optional<at::Tensor>& bd_ = c10::nullopt,
                                    const char* opname = nullptr, const at::Tensor* packed = nullptr) {
  const char* op = opname ? opname
                          : (intermediates ? "block_ell_swiglu_fwd_with_intermediate" : "block_ell_swiglu_fwd");
  at::Tensor x = check_x2d(x_, op);
  const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(x.device());
  lbk_bell g = make_bell(vg, cg, op, "gate"), u = make_bell(vu, cu, op, "up"), d = make_bell(vd, cd, op, "down");
  const int64_t N = x.size(0), d_model = x.size(1);
  TORCH_CHECK((int64_t)d.R * d.B == d_model, "titan::", op, ": values_down R_model=", d.R,
              " inconsistent with d_model=", d_model);
  TORCH_CHECK(g.R == u.R, "titan::", op, ": gate and up must have same R_ff");
  const int64_t d_ff = (int64_t)g.R * g.B;
  at::Tensor out = at::empty({N, d_model}, x.options());
  std::vector<at::Tensor> res{out};
  uint16_t *h = nullptr, *gp = nullptr, *uo = nullptr;
  if (intermediates) {
    at::Tensor th = at::empty({N, d_ff}, x.options()), tg = at::empty({N, d_ff}, x.options()),
               tu = at::empty({N, d_ff}, x.options());
    h = bfm(th);
    gp = bfm(tg);
    uo = bfm(tu);
    res.push_back(th);
    res.push_back(tg);
    res.push_back(tu);
  }
  const at::Tensor bg = opt_bias(bg_, d_ff, x, op, "b_gate"), bu = opt_bias(bu_, d_ff, x, op, "b_up"),
                   bd = opt_bias(bd_, d_model, x, op, "b_down");
  if (packed) {
    check_gpu(*packed, op, "packed");
    TORCH_CHECK(packed->scalar_type() == at::kByte && packed->dim() == 1 && packed->is_contiguous(), "titan::", op,
                ": packed must be the contiguous uint8 tensor of block_ell_swiglu_prepack");
    const size_t need = lbk_swiglu_prepacked_bytes((int32_t)d_model, &g, &u, &d);
    TORCH_CHECK((size_t)packed->numel() >= need, "titan::", op, ": packed holds ", packed->numel(),
                " bytes, this geometry needs ", need, " (pack these weights with block_ell_swiglu_prepack)");
    const size_t wsb = lbk_swiglu_prepacked_workspace_bytes(N, (int32_t)d_model, &g, &u, &d, intermediates ? 1 : 0);
    at::Tensor ws = wsb ? workspace(wsb, x) : at::Tensor();
    LBK_CALL("block_ell_swiglu_fwd_prepacked",
             lbk_swiglu_fwd_prepacked_bf16(bf(x), N, (int32_t)d_model, &g, &u, &d,
                                           need ? packed->data_ptr() : nullptr, (size_t)packed->numel(), fptr(bg),
                                           fptr(bu), fptr(bd), add_residual ? 1 : 0, bfm(out), h, gp, uo,
                                           wsb ? ws.data_ptr() : nullptr, wsb, cur_stream(x)));
    return res;
  }
  const size_t wsb = lbk_swiglu_workspace_bytes(N, (int32_t)d_model, &g, &u, &d, intermediates ? 1 : 0);
  at::Tensor ws = wsb ? workspace(wsb, x) : at::Tensor();
  LBK_CALL("block_ell_swiglu_fwd",
           lbk_swiglu_fwd_bias_bf16(bf(x), N, (int32_t)d_model, &g, &u, &d, fptr(bg), fptr(bu), fptr(bd),
                                    add_residual ? 1 : 0, bfm(out), h, gp, uo, wsb ? ws.data_ptr() : nullptr, wsb,
                                    cur_stream(x)));
  return res;
}

// SwiGLU with the projections' biases: (out, h, gate_pre_act, up_out); the intermediates are
// empty tensors unless asked for
std::tuple<at::Tensor, at::Tensor, at::Tensor, at::Tensor> swiglu_fwd_bias(
    const at::Tensor& x, const at::Tensor& vg, const at::Tensor& cg, const c10::optional<at::Tensor>& bg,
    const at::Tensor& vu, const at::Tensor& cu, const c10::optional<at::Tensor>& bu, const at::Tensor& vd,
    const at::Tensor& cd, const c10::optional<at::Tensor>& bd, bool add_residual, bool intermediates) {
  auto r = swiglu_impl(x, vg, cg, vu, cu, vd, cd, add_residual, intermediates, bg, bu, bd,
                       "block_ell_swiglu_fwd_bias");
  if (!intermediates) {
    at::Tensor e = at::empty({0}, x.options());
    return {r[0], e, e, e};
  }
  return {r[0], r[1], r[2], r[3]};
}

// The fragment-major packed copy of gate/up/down that the two-kernel forward reads, built once
// (uint8; empty when the geometry has no packed form): block_ell_swiglu_fwd_prepacked then
// skips the per-call pack.  It reflects the values and column indices at the time of the call.
at::Tensor swiglu_prepack(const at::Tensor& vg_, const at::Tensor& cg_, const at::Tensor& vu_, const at::Tensor& cu_,
                          const at::Tensor& vd_, const at::Tensor& cd_) {
  const char* op = "block_ell_swiglu_prepack";
  at::Tensor vg = vg_, cg = cg_, vu = vu_, cu = cu_, vd = vd_, cd = cd_;
  check_gpu(vg, op, "gate");
  const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(vg.device());
  lbk_bell g = make_bell(vg, cg, op, "gate"), u = make_bell(vu, cu, op, "up"), d = make_bell(vd, cd, op, "down");
  const int32_t d_model = d.R * d.B;
  const size_t bytes = lbk_swiglu_prepacked_bytes(d_model, &g, &u, &d);
  at::Tensor packed = at::empty({(int64_t)bytes}, vg.options().dtype(at::kByte));
  if (bytes)
    LBK_CALL("block_ell_swiglu_prepack",
             lbk_swiglu_prepack_bf16(d_model, &g, &u, &d, packed.data_ptr(), bytes, cur_stream(vg)));
  return packed;
}

at::Tensor swiglu_fwd_prepacked(const at::Tensor& x, const at::Tensor& packed, const at::Tensor& vg,
                                const at::Tensor& cg, const c10::optional<at::Tensor>& bg, const at::Tensor& vu,
                                const at::Tensor& cu, const c10::optional<at::Tensor>& bu, const at::Tensor& vd,
                                const at::Tensor& cd, const c10::optional<at::Tensor>& bd, bool add_residual) {
  return swiglu_impl(x, vg, cg, vu, cu, vd, cd, add_residual, false, bg, bu, bd, "block_ell_swiglu_fwd_prepacked",
                     &packed)[0];
}

at::Tensor swiglu_fwd(const at::Tensor& x, const at::Tensor& vg, const at::Tensor& cg, const at::Tensor& vu,
                      const at::Tensor& cu, const at::Tensor& vd, const at::Tensor& cd, bool add_residual) {
  return swiglu_impl(x, vg, cg, vu, cu, vd, cd, add_residual, false)[0];
}

std::tuple<at::Tensor, at::Tensor, at::Tensor, at::Tensor> swiglu_fwd_inter(
    const at::Tensor& x, const at::Tensor& vg, const at::Tensor& cg, const at::Tensor& vu, const at::Tensor& cu,
    const at::Tensor& vd, const at::Tensor& cd, bool add_residual) {
  auto r = swiglu_impl(x, vg, cg, vu, cu, vd, cd, add_residual, true);
  return {r[0], r[1], r[2], r[3]};
}

at::Tensor block_ell_matmul(const at::Tensor& x_, const at::Tensor& v_, const at::Tensor& c_,
                            const c10::optional<at::Tensor>& bias) {
  const char* op = "block_ell_matmul";
  at::Tensor v = v_, c = c_;
  at::Tensor x = check_x2d(x_, op);
  const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(x.device());
  lbk_bell w = make_bell(v, c, op, "weight");
  TORCH_CHECK(x.size(1) % w.B == 0, "titan::block_ell_matmul: in_features ", x.size(1), " not a multiple of B=", w.B);
  const int64_t N = x.size(0), out_f = (int64_t)w.R * w.B;
  const at::Tensor b = opt_bias(bias, out_f, x, op, "bias");
  at::Tensor y = at::empty({N, out_f}, x.options());
  const size_t wsb = lbk_block_ell_matmul_workspace_bytes(N, (int32_t)x.size(1), &w);
  at::Tensor ws = wsb ? workspace(wsb, x) : at::Tensor();
  LBK_CALL("block_ell_matmul", lbk_block_ell_matmul_ws_bf16(bf(x), N, (int32_t)x.size(1), &w, fptr(b), bfm(y),
                                                            wsb ? ws.data_ptr() : nullptr, wsb, cur_stream(x)));
  return y;
}

// block_ell_matmul's packed tiles for weights fixed across calls (uint8; empty when the shape takes
// the row-block kernel), and the product from them
at::Tensor block_ell_matmul_prepack(const at::Tensor& v_, const at::Tensor& c_, int64_t in_features) {
  const char* op = "block_ell_matmul_prepack";
  at::Tensor v = v_, c = c_;
  check_gpu(v, op, "values");
  const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(v.device());
  lbk_bell w = make_bell(v, c, op, "weight");
  TORCH_CHECK(in_features > 0 && in_features % w.B == 0, "titan::block_ell_matmul_prepack: in_features ",
              in_features, " not a positive multiple of B=", w.B);
  const size_t bytes = lbk_block_ell_matmul_prepacked_bytes((int32_t)in_features, &w);
  at::Tensor packed = at::empty({(int64_t)bytes}, v.options().dtype(at::kByte));
  if (bytes)
    LBK_CALL("block_ell_matmul_prepack",
             lbk_block_ell_matmul_prepack_bf16((int32_t)in_features, &w, packed.data_ptr(), bytes, cur_stream(v)));
  return packed;
}

at::Tensor block_ell_matmul_prepacked(const at::Tensor& x_, const at::Tensor& packed, const at::Tensor& v_,
                                      const at::Tensor& c_, const c10::optional<at::Tensor>& bias) {
  const char* op = "block_ell_matmul_prepacked";
  at::Tensor v = v_, c = c_;
  at::Tensor x = check_x2d(x_, op);
  const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(x.device());
  lbk_bell w = make_bell(v, c, op, "weight");
  TORCH_CHECK(x.size(1) % w.B == 0, "titan::block_ell_matmul_prepacked: in_features ", x.size(1),
              " not a multiple of B=", w.B);
  check_gpu(packed, op, "packed");
  TORCH_CHECK(packed.scalar_type() == at::kByte && packed.dim() == 1 && packed.is_contiguous(),
              "titan::block_ell_matmul_prepacked: packed must be the uint8 tensor of block_ell_matmul_prepack");
  const size_t need = lbk_block_ell_matmul_prepacked_bytes((int32_t)x.size(1), &w);
  TORCH_CHECK((size_t)packed.numel() >= need, "titan::block_ell_matmul_prepacked: packed holds ", packed.numel(),
              " bytes, this shape needs ", need);
  const int64_t N = x.size(0), out_f = (int64_t)w.R * w.B;
  const at::Tensor b = opt_bias(bias, out_f, x, op, "bias");
  at::Tensor y = at::empty({N, out_f}, x.options());
  LBK_CALL("block_ell_matmul_prepacked",
           lbk_block_ell_matmul_prepacked_bf16(bf(x), N, (int32_t)x.size(1), &w, need ? packed.data_ptr() : nullptr,
                                               (size_t)packed.numel(), fptr(b), bfm(y), cur_stream(x)));
  return y;
}

// backward of block_ell_matmul (bias gradient excluded): (dx, d_values)
std::tuple<at::Tensor, at::Tensor> block_ell_matmul_bwd(const at::Tensor& dy_, const at::Tensor& x_,
                                                        const at::Tensor& v_, const at::Tensor& c_) {
  const char* op = "block_ell_matmul_bwd";
  at::Tensor v = v_, c = c_;
  at::Tensor x = check_x2d(x_, op);
  const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(x.device());
  lbk_bell w = make_bell(v, c, op, "weight");
  TORCH_CHECK(x.size(1) % w.B == 0, "titan::block_ell_matmul_bwd: in_features ", x.size(1),
              " not a multiple of B=", w.B);
  const int64_t N = x.size(0), out_f = (int64_t)w.R * w.B;
  at::Tensor dy = check_x2d(dy_, op);
  TORCH_CHECK(dy.size(0) == N && dy.size(1) == out_f, "titan::block_ell_matmul_bwd: grad_out must be [", N, ", ",
              out_f, "], got ", dy.sizes());
  at::Tensor dx = at::empty({N, x.size(1)}, x.options());
  at::Tensor dv = at::empty_like(v);
  const size_t wsb = lbk_block_ell_matmul_bwd_workspace_bytes(N, (int32_t)x.size(1), &w);
  at::Tensor ws = workspace(wsb, x);
  LBK_CALL("block_ell_matmul_bwd", lbk_block_ell_matmul_bwd_bf16(bf(dy), bf(x), N, (int32_t)x.size(1), &w, bfm(dx),
                                                                 bfm(dv), ws.data_ptr(), wsb, cur_stream(x)));
  return {dx, dv};
}

// ------------------------------------------------------------------ norm / loop
at::Tensor rmsnorm(const at::Tensor& x_, const at::Tensor& scale_, double eps) {
  at::Tensor x = check_x2d(x_, "rmsnorm");
  const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(x.device());
  at::Tensor s = scale_.to(x.device(), at::kFloat).contiguous();
  TORCH_CHECK(s.numel() == x.size(1), "titan::rmsnorm: scale must have d elements");
  at::Tensor out = at::empty_like(x);
  LBK_CALL("rmsnorm", lbk_rmsnorm_bf16(bf(x), x.size(0), (int32_t)x.size(1), s.data_ptr<float>(), (float)eps,
                                       bfm(out), cur_stream(x)));
  return out;
}

std::tuple<at::Tensor, at::Tensor> rmsnorm_bwd(const at::Tensor& dy_, const at::Tensor& x_, const at::Tensor& scale_,
                                               double eps) {
  at::Tensor x = check_x2d(x_, "rmsnorm_bwd");
  at::Tensor dy = check_x2d(dy_, "rmsnorm_bwd");
  TORCH_CHECK(dy.sizes() == x.sizes(), "titan::rmsnorm_bwd: grad_out must match x");
  const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(x.device());
  at::Tensor s = scale_.to(x.device(), at::kFloat).contiguous();
  TORCH_CHECK(s.numel() == x.size(1), "titan::rmsnorm_bwd: scale must have d elements");
  at::Tensor dx = at::empty_like(x);
  at::Tensor ds = at::empty({x.size(1)}, x.options().dtype(at::kFloat));
  const size_t wsb = lbk_rmsnorm_bwd_workspace_bytes(x.size(0), (int32_t)x.size(1));
  at::Tensor ws = workspace(wsb, x);
  LBK_CALL("rmsnorm_bwd", lbk_rmsnorm_bwd_bf16(bf(x), bf(dy), x.size(0), (int32_t)x.size(1), s.data_ptr<float>(),
                                               (float)eps, bfm(dx), ds.data_ptr<float>(), ws.data_ptr(), wsb,
                                               cur_stream(x)));
  return {dx, ds};
}

at::Tensor diagonal_injection(const at::Tensor& h_, const at::Tensor& e_, const at::Tensor& log_A,
                              const at::Tensor& log_dt) {
  at::Tensor h = check_x2d(h_, "diagonal_injection");
  at::Tensor e = check_x2d(e_, "diagonal_injection");
  TORCH_CHECK(e.sizes() == h.sizes(), "titan::diagonal_injection: e must match h");
  const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(h.device());
  at::Tensor la = log_A.to(h.device(), at::kFloat).contiguous(), ld = log_dt.to(h.device(), at::kFloat).contiguous();
  TORCH_CHECK(la.numel() == h.size(1) && ld.numel() == h.size(1), "titan::diagonal_injection: log_A/log_dt must be [d_model]");
  at::Tensor out = at::empty_like(h);
  LBK_CALL("diagonal_injection", lbk_diagonal_injection_bf16(bf(h), bf(e), la.data_ptr<float>(), ld.data_ptr<float>(),
                                                             h.size(0), (int32_t)h.size(1), bfm(out), cur_stream(h)));
  return out;
}

// (dh, de, d_log_A, d_log_dt) of diagonal_injection for grad_out
std::tuple<at::Tensor, at::Tensor, at::Tensor, at::Tensor> diagonal_injection_bwd(
    const at::Tensor& dy_, const at::Tensor& h_, const at::Tensor& e_, const at::Tensor& log_A,
    const at::Tensor& log_dt) {
  const char* op = "diagonal_injection_bwd";
  at::Tensor dy = check_x2d(dy_, op), h = check_x2d(h_, op), e = check_x2d(e_, op);
  TORCH_CHECK(e.sizes() == h.sizes() && dy.sizes() == h.sizes(), "titan::diagonal_injection_bwd: grad_out, h and e "
              "must have one shape");
  const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(h.device());
  at::Tensor la = log_A.to(h.device(), at::kFloat).contiguous(), ld = log_dt.to(h.device(), at::kFloat).contiguous();
  TORCH_CHECK(la.numel() == h.size(1) && ld.numel() == h.size(1),
              "titan::diagonal_injection_bwd: log_A/log_dt must be [d_model]");
  at::Tensor dh = at::empty_like(h), de = at::empty_like(h);
  at::Tensor dla = at::empty({h.size(1)}, h.options().dtype(at::kFloat)), dld = at::empty_like(dla);
  const size_t wsb = lbk_diagonal_injection_bwd_workspace_bytes(h.size(0), (int32_t)h.size(1));
  at::Tensor ws = workspace(wsb, h);
  LBK_CALL("diagonal_injection_bwd",
           lbk_diagonal_injection_bwd_bf16(bf(dy), bf(h), bf(e), la.data_ptr<float>(), ld.data_ptr<float>(), h.size(0),
                                           (int32_t)h.size(1), bfm(dh), bfm(de), dla.data_ptr<float>(),
                                           dld.data_ptr<float>(), ws.data_ptr(), wsb, cur_stream(h)));
  return {dh, de, dla, dld};
}

at::Tensor looped_impl(const at::Tensor& h, const at::Tensor& scale_, at::Tensor vg, at::Tensor cg, at::Tensor vu,
                       at::Tensor cu, at::Tensor vd, at::Tensor cd, int64_t L, double eps, const char* op,
                       int path = 0) {
  at::Tensor x = check_x2d(h, op);
  const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(x.device());
  lbk_bell g = make_bell(vg, cg, op, "gate"), u = make_bell(vu, cu, op, "up"), d = make_bell(vd, cd, op, "down");
  at::Tensor s = scale_.to(x.device(), at::kFloat).contiguous();
  TORCH_CHECK(s.numel() == x.size(1), "titan::", op, ": norm scale must have d_model elements");
  TORCH_CHECK(L >= 0, "titan::", op, ": L must be >= 0");
  at::Tensor out = at::empty_like(x);
  const size_t wsb = lbk_looped_workspace_bytes(x.size(0), (int32_t)x.size(1), &g, &u, &d);
  at::Tensor ws = wsb ? workspace(wsb, x) : at::Tensor();
  // path 0: the library's choice, 1: one persistent launch, 2: launches per iteration
  auto fn = path == 1 ? lbk_looped_swiglu_persistent_bf16
                      : (path == 2 ? lbk_looped_swiglu_launches_bf16 : lbk_looped_swiglu_bf16);
  LBK_CALL("looped_swiglu", fn(bf(x), x.size(0), (int32_t)x.size(1), s.data_ptr<float>(), (float)eps, (int32_t)L,
                               &g, &u, &d, bfm(out), wsb ? ws.data_ptr() : nullptr, wsb, cur_stream(x)));
  return out;
}

at::Tensor looped_swiglu_bias(const at::Tensor& h_, const at::Tensor& scale_, const at::Tensor& vg_,
                              const at::Tensor& cg_, const c10::optional<at::Tensor>& bg_, const at::Tensor& vu_,
                              const at::Tensor& cu_, const c10::optional<at::Tensor>& bu_, const at::Tensor& vd_,
                              const at::Tensor& cd_, const c10::optional<at::Tensor>& bd_, int64_t L, double eps) {
  const char* op = "looped_swiglu_bias";
  at::Tensor x = check_x2d(h_, op);
  const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(x.device());
  at::Tensor vg = vg_, cg = cg_, vu = vu_, cu = cu_, vd = vd_, cd = cd_;
  lbk_bell g = make_bell(vg, cg, op, "gate"), u = make_bell(vu, cu, op, "up"), d = make_bell(vd, cd, op, "down");
  at::Tensor s = scale_.to(x.device(), at::kFloat).contiguous();
  TORCH_CHECK(s.numel() == x.size(1), "titan::", op, ": norm scale must have d_model elements");
  TORCH_CHECK(L >= 0, "titan::", op, ": L must be >= 0");
  const int64_t d_ff = (int64_t)g.R * g.B;
  const at::Tensor bg = opt_bias(bg_, d_ff, x, op, "b_gate"), bu = opt_bias(bu_, d_ff, x, op, "b_up"),
                   bd = opt_bias(bd_, x.size(1), x, op, "b_down");
  at::Tensor out = at::empty_like(x);
  const size_t wsb = lbk_looped_workspace_bytes(x.size(0), (int32_t)x.size(1), &g, &u, &d);
  at::Tensor ws = wsb ? workspace(wsb, x) : at::Tensor();
  LBK_CALL("looped_swiglu_bias",
           lbk_looped_swiglu_bias_bf16(bf(x), x.size(0), (int32_t)x.size(1), s.data_ptr<float>(), (float)eps,
                                       (int32_t)L, &g, &u, &d, fptr(bg), fptr(bu), fptr(bd), bfm(out),
                                       wsb ? ws.data_ptr() : nullptr, wsb, cur_stream(x)));
  return out;
}

at::Tensor looped_swiglu_persistent(const at::Tensor& h, const at::Tensor& scale, const at::Tensor& vg,
                                    const at::Tensor& cg, const at::Tensor& vu, const at::Tensor& cu,
                                    const at::Tensor& vd, const at::Tensor& cd, int64_t L, double eps) {
  return looped_impl(h, scale, vg, cg, vu, cu, vd, cd, L, eps, "looped_swiglu_persistent", 1);
}

at::Tensor looped_swiglu_launches(const at::Tensor& h, const at::Tensor& scale, const at::Tensor& vg,
                                  const at::Tensor& cg, const at::Tensor& vu, const at::Tensor& cu,
                                  const at::Tensor& vd, const at::Tensor& cd, int64_t L, double eps) {
  return looped_impl(h, scale, vg, cg, vu, cu, vd, cd, L, eps, "looped_swiglu_launches", 2);
}

at::Tensor looped_swiglu(const at::Tensor& h, const at::Tensor& scale, const at::Tensor& vg, const at::Tensor& cg,
                         const at::Tensor& vu, const at::Tensor& cu, const at::Tensor& vd, const at::Tensor& cd,
                         int64_t L, double eps) {
  return looped_impl(h, scale, vg, cg, vu, cu, vd, cd, L, eps, "looped_swiglu");
}

// Reference semantics (csrc/loop/persistent_core.cu:273-338): injection once,
// then for each core block: h = h + SwiGLU(RMSNorm(h, eps=1e-6)).
at::Tensor persistent_mlp_step(const at::Tensor& h, const at::Tensor& e, const at::Tensor& log_A,
                               const at::Tensor& log_dt, at::TensorList norm_scales, at::TensorList gate_values,
                               at::TensorList gate_col_idx, at::TensorList up_values, at::TensorList up_col_idx,
                               at::TensorList down_values, at::TensorList down_col_idx) {
  const size_t n_core = norm_scales.size();
  TORCH_CHECK(n_core > 0, "persistent_mlp_step: n_core must be > 0");
  TORCH_CHECK(gate_values.size() == n_core && gate_col_idx.size() == n_core && up_values.size() == n_core &&
                  up_col_idx.size() == n_core && down_values.size() == n_core && down_col_idx.size() == n_core,
              "persistent_mlp_step: all weight vector sizes must equal n_core");
  TORCH_CHECK(h.dim() == 2, "persistent_mlp_step: h must be 2D [N, d_model], got shape ", h.sizes());
  TORCH_CHECK(h.scalar_type() == at::kBFloat16, "persistent_mlp_step: h must be bf16");
  at::Tensor cur = diagonal_injection(h, e, log_A, log_dt);
  for (size_t i = 0; i < n_core; ++i)
    cur = looped_impl(cur, norm_scales[i], gate_values[i], gate_col_idx[i], up_values[i], up_col_idx[i],
                      down_values[i], down_col_idx[i], 1, 1e-6, "persistent_mlp_step");
  return cur;
}

// The looped application of the FFN core (looped_blockell/looping/looped_model.py:293-340 on its
// FFN path): per iteration the injection (when e is given), the n_core blocks in order, then the
// depth freeze (when depths is given, one entry per seq_len rows).  biases: empty, or
// (b_gate, b_up, b_down) per block, each optional.
at::Tensor looped_core(const at::Tensor& h_, const c10::optional<at::Tensor>& e_, const c10::optional<at::Tensor>& la_,
                       const c10::optional<at::Tensor>& ld_, at::TensorList norm_scales, at::TensorList gate_values,
                       at::TensorList gate_col_idx, at::TensorList up_values, at::TensorList up_col_idx,
                       at::TensorList down_values, at::TensorList down_col_idx,
                       const c10::List<c10::optional<at::Tensor>>& biases, int64_t L,
                       const c10::optional<at::Tensor>& depths_, int64_t seq_len, double eps, bool persistent) {
  const char* op = "looped_core";
  at::Tensor x = check_x2d(h_, op);
  const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(x.device());
  const size_t n_core = norm_scales.size();
  TORCH_CHECK(n_core >= 1 && n_core <= LBK_MAX_CORE_BLOCKS, "titan::looped_core: n_core must be in [1, ",
              LBK_MAX_CORE_BLOCKS, "], got ", n_core);
  TORCH_CHECK(gate_values.size() == n_core && gate_col_idx.size() == n_core && up_values.size() == n_core &&
                  up_col_idx.size() == n_core && down_values.size() == n_core && down_col_idx.size() == n_core,
              "titan::looped_core: all weight lists must have n_core entries");
  TORCH_CHECK(biases.size() == 0 || biases.size() == 3 * n_core,
              "titan::looped_core: biases must be empty or hold (b_gate, b_up, b_down) per core block");
  TORCH_CHECK(L >= 0, "titan::looped_core: L must be >= 0");
  const int64_t N = x.size(0), d_model = x.size(1);
  std::vector<at::Tensor> keep;   // contiguous copies alive until the call is queued
  std::vector<lbk_core_block> blocks(n_core);
  for (size_t c = 0; c < n_core; ++c) {
    at::Tensor vg = gate_values[c], cg = gate_col_idx[c], vu = up_values[c], cu = up_col_idx[c],
               vd = down_values[c], cd = down_col_idx[c];
    lbk_core_block& b = blocks[c];
    b.gate = make_bell(vg, cg, op, "gate");
    b.up = make_bell(vu, cu, op, "up");
    b.down = make_bell(vd, cd, op, "down");
    at::Tensor sc = norm_scales[c].to(x.device(), at::kFloat).contiguous();
    TORCH_CHECK(sc.numel() == d_model, "titan::looped_core: norm scale ", c, " must have d_model elements");
    b.norm_scale = sc.data_ptr<float>();
    const int64_t d_ff = (int64_t)b.gate.R * b.gate.B;
    at::Tensor bt[3];
    if (biases.size()) {
      bt[0] = opt_bias(biases.get(3 * c), d_ff, x, op, "b_gate");
      bt[1] = opt_bias(biases.get(3 * c + 1), d_ff, x, op, "b_up");
      bt[2] = opt_bias(biases.get(3 * c + 2), d_model, x, op, "b_down");
    }
    b.b_gate = fptr(bt[0]);
    b.b_up = fptr(bt[1]);
    b.b_down = fptr(bt[2]);
    for (at::Tensor* t : {&vg, &cg, &vu, &cu, &vd, &cd, &sc, &bt[0], &bt[1], &bt[2]})
      if (t->defined()) keep.push_back(*t);
  }
  at::Tensor e, la, ld, dep;
  if (e_.has_value() && e_->defined()) {
    e = check_x2d(*e_, op);
    TORCH_CHECK(e.sizes() == x.sizes(), "titan::looped_core: e must match h, got ", e.sizes());
    TORCH_CHECK(la_.has_value() && la_->defined() && ld_.has_value() && ld_->defined(),
                "titan::looped_core: the injection needs log_A and log_dt");
    la = la_->to(x.device(), at::kFloat).contiguous();
    ld = ld_->to(x.device(), at::kFloat).contiguous();
    TORCH_CHECK(la.numel() == d_model && ld.numel() == d_model,
                "titan::looped_core: log_A and log_dt must have d_model elements");
  }
  if (depths_.has_value() && depths_->defined()) {
    TORCH_CHECK(seq_len >= 1, "titan::looped_core: seq_len must be >= 1");
    dep = depths_->to(x.device(), at::kInt).contiguous();
    TORCH_CHECK(dep.numel() * seq_len >= N, "titan::looped_core: depths must cover every row (",
                dep.numel(), " x seq_len ", seq_len, " < N = ", N, ")");
  }
  at::Tensor out = at::empty_like(x);
  const size_t wsb = lbk_looped_core_workspace_bytes(N, (int32_t)d_model, (int32_t)n_core, blocks.data());
  at::Tensor ws = wsb ? workspace(wsb, x) : at::Tensor();
  auto fn = persistent ? lbk_looped_core_persistent_bf16 : lbk_looped_core_bf16;
  LBK_CALL("looped_core",
           fn(bf(x), e.defined() ? bf(e) : nullptr, la.defined() ? la.data_ptr<float>() : nullptr,
              ld.defined() ? ld.data_ptr<float>() : nullptr, N, (int32_t)d_model, (int32_t)n_core, blocks.data(),
              (float)eps, (int32_t)L, dep.defined() ? dep.data_ptr<int32_t>() : nullptr, seq_len, bfm(out),
              wsb ? ws.data_ptr() : nullptr, wsb, cur_stream(x)));
  return out;
}

// ------------------------------------------------------------------ ternary
std::tuple<at::Tensor, at::Tensor> quantize_act_int8(const at::Tensor& x_) {
  at::Tensor x = check_x2d(x_, "quantize_act_int8");
  const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(x.device());
  at::Tensor q = at::empty(x.sizes(), x.options().dtype(at::kChar));
  at::Tensor s = at::empty({x.size(0)}, x.options().dtype(at::kFloat));
  LBK_CALL("quantize_act_int8", lbk_quantize_act_int8(bf(x), x.size(0), (int32_t)x.size(1), x.size(1),
                                                      q.data_ptr<int8_t>(), s.data_ptr<float>(), cur_stream(x)));
  return {q, s};
}

at::Tensor pack_ternary(const at::Tensor& t_) {
  check_gpu(t_, "pack_ternary", "t");
  TORCH_CHECK(t_.scalar_type() == at::kChar, "titan::pack_ternary: t must be int8");
  TORCH_CHECK(t_.dim() == 4 && t_.size(2) == t_.size(3), "titan::pack_ternary: t must be [R, K, B, B]");
  at::Tensor t = t_.contiguous();
  const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(t.device());
  const int64_t B = t.size(2);
  TORCH_CHECK(B == 16 || B == 32 || B == 64, "titan::pack_ternary: B must be 16, 32 or 64");
  at::Tensor p = at::empty({t.size(0), t.size(1), B, B / 16}, t.options().dtype(at::kInt));
  LBK_CALL("pack_ternary", lbk_pack_ternary(t.data_ptr<int8_t>(), (int32_t)t.size(0), (int32_t)t.size(1),
                                            (int32_t)B, reinterpret_cast<uint32_t*>(p.data_ptr()), cur_stream(t)));
  return p;
}

std::tuple<at::Tensor, at::Tensor> ternary_quantize_weights(const at::Tensor& v_) {
  check_gpu(v_, "ternary_quantize_weights", "values");
  TORCH_CHECK(v_.dim() == 4 && v_.size(2) == v_.size(3), "titan::ternary_quantize_weights: values must be [R,K,B,B]");
  at::Tensor v = v_.to(at::kBFloat16).contiguous();
  const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(v.device());
  const int64_t B = v.size(2);
  at::Tensor p = at::empty({v.size(0), v.size(1), B, B / 16}, v.options().dtype(at::kInt));
  at::Tensor s = at::empty({v.size(0), v.size(1)}, v.options().dtype(at::kFloat));
  LBK_CALL("ternary_quantize_weights",
           lbk_ternary_quantize_weights_bf16(bf(v), (int32_t)v.size(0), (int32_t)v.size(1), (int32_t)B,
                                             reinterpret_cast<uint32_t*>(p.data_ptr()), s.data_ptr<float>(),
                                             cur_stream(v)));
  return {p, s};
}

at::Tensor check_int8_x(const at::Tensor& xq_, const at::Tensor& sx, const char* op) {
  check_gpu(xq_, op, "xq");
  check_gpu(sx, op, "sx");
  TORCH_CHECK(xq_.scalar_type() == at::kChar, "titan::", op, ": xq must be int8");
  TORCH_CHECK(xq_.dim() == 2, "titan::", op, ": xq must be 2D [N, features]");
  TORCH_CHECK(sx.scalar_type() == at::kFloat && sx.numel() == xq_.size(0), "titan::", op,
              ": sx must be fp32 [N]");
  return xq_.contiguous();
}

std::tuple<at::Tensor, at::Tensor> ternary_matmul(const at::Tensor& xq_, const at::Tensor& sx_, const at::Tensor& p_,
                                                  const at::Tensor& s_, const at::Tensor& c_, bool want_partials) {
  const char* op = "ternary_matmul";
  at::Tensor p = p_, s = s_, c = c_;
  at::Tensor xq = check_int8_x(xq_, sx_, op);
  at::Tensor sx = sx_.contiguous();
  const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(xq.device());
  lbk_bell_ternary w = make_tern(p, s, c, op, "weight");
  const int64_t N = xq.size(0), out_f = (int64_t)w.R * w.B;
  at::Tensor y = at::empty({N, out_f}, xq.options().dtype(at::kBFloat16));
  at::Tensor part = want_partials ? at::empty({N, w.R, w.K, w.B}, xq.options().dtype(at::kInt))
                                  : at::empty({0}, xq.options().dtype(at::kInt));
  LBK_CALL("ternary_matmul", lbk_ternary_matmul(xq.data_ptr<int8_t>(), sx.data_ptr<float>(), N, (int32_t)xq.size(1),
                                                &w, bfm(y), want_partials ? part.data_ptr<int32_t>() : nullptr,
                                                cur_stream(xq)));
  return {y, part};
}

std::vector<at::Tensor> tern_swiglu_impl(const at::Tensor& xq_, const at::Tensor& sx_, at::Tensor pg, at::Tensor sg,
                                         at::Tensor cg, at::Tensor pu, at::Tensor su, at::Tensor cu, at::Tensor pd,
                                         at::Tensor sd, at::Tensor cd, const c10::optional<at::Tensor>& x_resid,
                                         bool inter, bool accs = false, const at::Tensor* prepared = nullptr) {
  const char* op = prepared ? "block_ell_swiglu_fwd_ternary_prepared"
                   : accs   ? "block_ell_swiglu_fwd_ternary_accumulators"
                   : inter  ? "block_ell_swiglu_fwd_ternary_with_intermediate"
                            : "block_ell_swiglu_fwd_ternary";
  inter = inter || accs;
  at::Tensor xq = check_int8_x(xq_, sx_, op);
  at::Tensor sx = sx_.contiguous();
  const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(xq.device());
  lbk_bell_ternary g = make_tern(pg, sg, cg, op, "gate"), u = make_tern(pu, su, cu, op, "up"),
                   d = make_tern(pd, sd, cd, op, "down");
  const int64_t N = xq.size(0), d_model = xq.size(1), d_ff = (int64_t)g.R * g.B;
  TORCH_CHECK((int64_t)d.R * d.B == d_model, "titan::", op, ": down R inconsistent with d_model");
  at::Tensor xr;
  const uint16_t* xrp = nullptr;
  if (x_resid.has_value() && x_resid->defined()) {
    xr = check_x2d(*x_resid, op);
    TORCH_CHECK(xr.size(0) == N && xr.size(1) == d_model, "titan::", op, ": x_resid must be [N, d_model]");
    xrp = bf(xr);
  }
  at::Tensor out = at::empty({N, d_model}, xq.options().dtype(at::kBFloat16));
  std::vector<at::Tensor> res{out};
  uint16_t* h = nullptr;
  int8_t* hq = nullptr;
  float* sh = nullptr;
  at::Tensor ws;
  size_t wsb = 0;
  if (inter) {
    at::Tensor th = at::empty({N, d_ff}, xq.options().dtype(at::kBFloat16));
    at::Tensor tq = at::empty({N, d_ff}, xq.options().dtype(at::kChar));
    at::Tensor ts = at::empty({N}, xq.options().dtype(at::kFloat));
    h = bfm(th);
    hq = tq.data_ptr<int8_t>();
    sh = ts.data_ptr<float>();
    res.push_back(th);
    res.push_back(tq);
    res.push_back(ts);
  }
  lbk_ternary_acc acc{};
  if (accs) {
    at::Tensor ag = at::empty({N, d_ff}, xq.options().dtype(at::kInt));
    at::Tensor au = at::empty({N, d_ff}, xq.options().dtype(at::kInt));
    at::Tensor ad = at::empty({N, d_model}, xq.options().dtype(at::kInt));
    at::Tensor gp = at::empty({N, d_ff}, xq.options().dtype(at::kFloat));
    at::Tensor up = at::empty({N, d_ff}, xq.options().dtype(at::kFloat));
    acc = lbk_ternary_acc{ag.data_ptr<int32_t>(), au.data_ptr<int32_t>(), ad.data_ptr<int32_t>(),
                          gp.data_ptr<float>(), up.data_ptr<float>()};
    for (const at::Tensor& t : {ag, au, ad, gp, up}) res.push_back(t);
  }
  if (prepared) {
    check_gpu(*prepared, op, "prepared");
    TORCH_CHECK(prepared->scalar_type() == at::kByte && prepared->dim() == 1 && prepared->is_contiguous(), "titan::",
                op, ": prepared must be the contiguous uint8 tensor of ternary_prepare");
    const size_t need = lbk_ternary_prepared_bytes((int32_t)d_model, &g, &u, &d);
    TORCH_CHECK((size_t)prepared->numel() >= need, "titan::", op, ": prepared holds ", prepared->numel(),
                " bytes, this geometry needs ", need, " (prepare these weights with ternary_prepare)");
    wsb = lbk_ternary_prepared_workspace_bytes(N, (int32_t)d_model, &g, &u, &d);
    if (wsb) ws = workspace(wsb, xq);
    LBK_CALL("block_ell_swiglu_fwd_ternary_prepared",
             lbk_swiglu_fwd_ternary_prepared(xq.data_ptr<int8_t>(), sx.data_ptr<float>(), N, (int32_t)d_model, &g, &u,
                                             &d, need ? prepared->data_ptr() : nullptr, (size_t)prepared->numel(), xrp,
                                             bfm(out), h, hq, sh, accs ? &acc : nullptr,
                                             wsb ? ws.data_ptr() : nullptr, wsb, cur_stream(xq)));
    return res;
  }
  wsb = lbk_ternary_swiglu_workspace_bytes(N, (int32_t)d_model, &g, &u, &d);
  if (wsb) ws = workspace(wsb, xq);
  LBK_CALL("block_ell_swiglu_fwd_ternary",
           lbk_swiglu_fwd_ternary_acc(xq.data_ptr<int8_t>(), sx.data_ptr<float>(), N, (int32_t)d_model, &g, &u, &d,
                                      xrp, bfm(out), h, hq, sh, accs ? &acc : nullptr,
                                      wsb ? ws.data_ptr() : nullptr, wsb, cur_stream(xq)));
  return res;
}

at::Tensor tern_swiglu(const at::Tensor& xq, const at::Tensor& sx, const at::Tensor& pg, const at::Tensor& sg,
                       const at::Tensor& cg, const at::Tensor& pu, const at::Tensor& su, const at::Tensor& cu,
                       const at::Tensor& pd, const at::Tensor& sd, const at::Tensor& cd,
                       const c10::optional<at::Tensor>& x_resid) {
  return tern_swiglu_impl(xq, sx, pg, sg, cg, pu, su, cu, pd, sd, cd, x_resid, false)[0];
}

std::tuple<at::Tensor, at::Tensor, at::Tensor, at::Tensor> tern_swiglu_inter(
    const at::Tensor& xq, const at::Tensor& sx, const at::Tensor& pg, const at::Tensor& sg, const at::Tensor& cg,
    const at::Tensor& pu, const at::Tensor& su, const at::Tensor& cu, const at::Tensor& pd, const at::Tensor& sd,
    const at::Tensor& cd, const c10::optional<at::Tensor>& x_resid) {
  auto r = tern_swiglu_impl(xq, sx, pg, sg, cg, pu, su, cu, pd, sd, cd, x_resid, true);
  return {r[0], r[1], r[2], r[3]};
}

// out, h, hq, sh, acc_gate, acc_up, acc_down, gate_pre, up_pre
std::tuple<at::Tensor, at::Tensor, at::Tensor, at::Tensor, at::Tensor, at::Tensor, at::Tensor, at::Tensor, at::Tensor>
tern_swiglu_accs(const at::Tensor& xq, const at::Tensor& sx, const at::Tensor& pg, const at::Tensor& sg,
                 const at::Tensor& cg, const at::Tensor& pu, const at::Tensor& su, const at::Tensor& cu,
                 const at::Tensor& pd, const at::Tensor& sd, const at::Tensor& cd,
                 const c10::optional<at::Tensor>& x_resid) {
  auto r = tern_swiglu_impl(xq, sx, pg, sg, cg, pu, su, cu, pd, sd, cd, x_resid, true, true);
  return {r[0], r[1], r[2], r[3], r[4], r[5], r[6], r[7], r[8]};
}

// The B = 64 ternary path's prepared weights (uint8; empty when the geometry has none), built once
// for weights that stay fixed; block_ell_swiglu_fwd_ternary_prepared then skips the per-call
// preparation.  They reflect packed, scales and col_indices at the time of the call.
at::Tensor ternary_prepare(const at::Tensor& pg_, const at::Tensor& sg_, const at::Tensor& cg_, const at::Tensor& pu_,
                           const at::Tensor& su_, const at::Tensor& cu_, const at::Tensor& pd_, const at::Tensor& sd_,
                           const at::Tensor& cd_) {
  const char* op = "ternary_prepare";
  at::Tensor pg = pg_, sg = sg_, cg = cg_, pu = pu_, su = su_, cu = cu_, pd = pd_, sd = sd_, cd = cd_;
  check_gpu(pg, op, "gate");
  const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(pg.device());
  lbk_bell_ternary g = make_tern(pg, sg, cg, op, "gate"), u = make_tern(pu, su, cu, op, "up"),
                   d = make_tern(pd, sd, cd, op, "down");
  const int32_t d_model = d.R * d.B;
  const size_t bytes = lbk_ternary_prepared_bytes(d_model, &g, &u, &d);
  at::Tensor prepared = at::empty({(int64_t)bytes}, pg.options().dtype(at::kByte));
  if (bytes) LBK_CALL("ternary_prepare", lbk_ternary_prepare(d_model, &g, &u, &d, prepared.data_ptr(), bytes,
                                                             cur_stream(pg)));
  return prepared;
}

at::Tensor tern_swiglu_prepared(const at::Tensor& xq, const at::Tensor& sx, const at::Tensor& prepared,
                                const at::Tensor& pg, const at::Tensor& sg, const at::Tensor& cg, const at::Tensor& pu,
                                const at::Tensor& su, const at::Tensor& cu, const at::Tensor& pd, const at::Tensor& sd,
                                const at::Tensor& cd, const c10::optional<at::Tensor>& x_resid) {
  return tern_swiglu_impl(xq, sx, pg, sg, cg, pu, su, cu, pd, sd, cd, x_resid, false, false, &prepared)[0];
}

at::Tensor check_columns(const at::Tensor& c_, int64_t C) {
  check_gpu(c_, "check_columns", "col_indices");
  TORCH_CHECK(c_.scalar_type() == at::kInt, "titan::check_columns: col_indices must be int32");
  at::Tensor c = c_.contiguous();
  const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(c.device());
  at::Tensor bad = at::empty({}, c.options());
  LBK_CALL("check_columns", lbk_check_columns(c.data_ptr<int32_t>(), c.numel(), (int32_t)C, bad.data_ptr<int32_t>(),
                                              cur_stream(c)));
  return bad;
}
// ------------------------------------------------------------------ bf16 SwiGLU backward
std::tuple<at::Tensor, at::Tensor, at::Tensor, at::Tensor> swiglu_bwd_impl(
    const at::Tensor& dy_, const at::Tensor& x_, const at::Tensor& gp_, const at::Tensor& uo_, const at::Tensor& h_,
    const at::Tensor& vg_, const at::Tensor& cg_, const at::Tensor& vu_, const at::Tensor& cu_, const at::Tensor& vd_,
    const at::Tensor& cd_, bool add_residual, const char* op) {
  at::Tensor vg = vg_, cg = cg_, vu = vu_, cu = cu_, vd = vd_, cd = cd_;
  at::Tensor x = check_x2d(x_, op);
  const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(x.device());
  lbk_bell g = make_bell(vg, cg, op, "gate"), u = make_bell(vu, cu, op, "up"), d = make_bell(vd, cd, op, "down");
  const int64_t N = x.size(0), d_model = x.size(1);
  const int64_t d_ff = (int64_t)g.R * g.B;
  auto act = [&](const at::Tensor& t, int64_t cols, const char* name) {
    check_gpu(t, op, name);
    TORCH_CHECK(t.scalar_type() == at::kBFloat16, "titan::", op, ": ", name, " must be bf16");
    TORCH_CHECK(t.dim() == 2 && t.size(0) == N && t.size(1) == cols, "titan::", op, ": ", name, " must be [", N,
                ", ", cols, "], got ", t.sizes());
    return t.contiguous();
  };
  at::Tensor dy = act(dy_, d_model, "grad_out"), gp = act(gp_, d_ff, "gate_pre_act"),
             uo = act(uo_, d_ff, "up_output"), h = act(h_, d_ff, "h");
  at::Tensor dx = at::empty({N, d_model}, x.options());
  at::Tensor dvg = at::empty_like(vg), dvu = at::empty_like(vu), dvd = at::empty_like(vd);
  const size_t wsb = lbk_swiglu_bwd_workspace_bytes(N, (int32_t)d_model, &g, &u, &d);
  at::Tensor ws = workspace(wsb, x);
  LBK_CALL("block_ell_swiglu_bwd",
           lbk_swiglu_bwd_bf16(bf(dy), bf(x), bf(gp), bf(uo), bf(h), N, (int32_t)d_model, &g, &u, &d,
                               add_residual ? 1 : 0, bfm(dx), bfm(dvg), bfm(dvu), bfm(dvd), ws.data_ptr(), wsb,
                               cur_stream(x)));
  return {dx, dvg, dvu, dvd};
}

// backward with the bias gradients (fp32 column sums of dg, du and grad_out)
std::tuple<at::Tensor, at::Tensor, at::Tensor, at::Tensor, at::Tensor, at::Tensor, at::Tensor> swiglu_bwd_bias(
    const at::Tensor& dy_, const at::Tensor& x_, const at::Tensor& gp_, const at::Tensor& uo_, const at::Tensor& h_,
    const at::Tensor& vg_, const at::Tensor& cg_, const at::Tensor& vu_, const at::Tensor& cu_, const at::Tensor& vd_,
    const at::Tensor& cd_, bool add_residual) {
  const char* op = "block_ell_swiglu_bwd_bias";
  at::Tensor vg = vg_, cg = cg_, vu = vu_, cu = cu_, vd = vd_, cd = cd_;
  at::Tensor x = check_x2d(x_, op);
  const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(x.device());
  lbk_bell g = make_bell(vg, cg, op, "gate"), u = make_bell(vu, cu, op, "up"), d = make_bell(vd, cd, op, "down");
  const int64_t N = x.size(0), d_model = x.size(1);
  const int64_t d_ff = (int64_t)g.R * g.B;
  auto act = [&](const at::Tensor& t, int64_t cols, const char* name) {
    check_gpu(t, op, name);
    TORCH_CHECK(t.scalar_type() == at::kBFloat16, "titan::", op, ": ", name, " must be bf16");
    TORCH_CHECK(t.dim() == 2 && t.size(0) == N && t.size(1) == cols, "titan::", op, ": ", name, " must be [", N,
                ", ", cols, "], got ", t.sizes());
    return t.contiguous();
  };
  at::Tensor dy = act(dy_, d_model, "grad_out"), gp = act(gp_, d_ff, "gate_pre_act"),
             uo = act(uo_, d_ff, "up_output"), h = act(h_, d_ff, "h");
  at::Tensor dx = at::empty({N, d_model}, x.options());
  at::Tensor dvg = at::empty_like(vg), dvu = at::empty_like(vu), dvd = at::empty_like(vd);
  at::Tensor dbg = at::empty({d_ff}, x.options().dtype(at::kFloat)), dbu = at::empty({d_ff}, x.options().dtype(at::kFloat)),
             dbd = at::empty({d_model}, x.options().dtype(at::kFloat));
  const size_t wsb = lbk_swiglu_bwd_bias_workspace_bytes(N, (int32_t)d_model, &g, &u, &d);
  at::Tensor ws = workspace(wsb, x);
  LBK_CALL("block_ell_swiglu_bwd_bias",
           lbk_swiglu_bwd_bias_bf16(bf(dy), bf(x), bf(gp), bf(uo), bf(h), N, (int32_t)d_model, &g, &u, &d,
                                    add_residual ? 1 : 0, bfm(dx), bfm(dvg), bfm(dvu), bfm(dvd), dbg.data_ptr<float>(),
                                    dbu.data_ptr<float>(), dbd.data_ptr<float>(), ws.data_ptr(), wsb, cur_stream(x)));
  return {dx, dvg, dvu, dvd, dbg, dbu, dbd};
}

// the reference operator: dx always includes grad_out (the forward's residual)
std::tuple<at::Tensor, at::Tensor, at::Tensor, at::Tensor> swiglu_bwd(
    const at::Tensor& dy, const at::Tensor& x, const at::Tensor& gp, const at::Tensor& uo, const at::Tensor& h,
    const at::Tensor& vg, const at::Tensor& cg, const at::Tensor& vu, const at::Tensor& cu, const at::Tensor& vd,
    const at::Tensor& cd) {
  return swiglu_bwd_impl(dy, x, gp, uo, h, vg, cg, vu, cu, vd, cd, true, "block_ell_swiglu_bwd");
}

std::tuple<at::Tensor, at::Tensor, at::Tensor, at::Tensor> swiglu_bwd_ex(
    const at::Tensor& dy, const at::Tensor& x, const at::Tensor& gp, const at::Tensor& uo, const at::Tensor& h,
    const at::Tensor& vg, const at::Tensor& cg, const at::Tensor& vu, const at::Tensor& cu, const at::Tensor& vd,
    const at::Tensor& cd, bool add_residual) {
  return swiglu_bwd_impl(dy, x, gp, uo, h, vg, cg, vu, cu, vd, cd, add_residual, "block_ell_swiglu_bwd_ex");
}


// HIP has no access-policy window; weight residency comes from the fused
// kernels (LDS panels, L2/MALL reuse).  The ops stay in the schema so callers
// written against the reference keep working (csrc/loop/loop_ops.cpp:39-46).
void pin_weights_l2(at::TensorList) {}
void unpin_weights_l2() {}

}  // namespace

TORCH_LIBRARY(titan, m) {
  // reference schemas (csrc/block_ell/block_ell_ops.cpp:51-97, csrc/loop/loop_ops.cpp:39-66)
  m.def("block_ell_swiglu_fwd(Tensor x, Tensor v_gate, Tensor ci_gate, Tensor v_up, Tensor ci_up, "
        "Tensor v_down, Tensor ci_down, bool add_residual) -> Tensor");
  m.def("block_ell_swiglu_fwd_with_intermediate(Tensor x, Tensor v_gate, Tensor ci_gate, Tensor v_up, "
        "Tensor ci_up, Tensor v_down, Tensor ci_down, bool add_residual) -> (Tensor, Tensor, Tensor, Tensor)");
  m.def("block_ell_swiglu_bwd(Tensor grad_out, Tensor x, Tensor gate_pre_act, Tensor up_out, Tensor h, "
        "Tensor v_gate, Tensor ci_gate, Tensor v_up, Tensor ci_up, Tensor v_down, Tensor ci_down) "
        "-> (Tensor, Tensor, Tensor, Tensor)");
  m.def("pin_weights_l2(Tensor[] weights) -> ()");
  m.def("unpin_weights_l2() -> ()");
  m.def("persistent_mlp_step(Tensor h, Tensor e, Tensor log_A, Tensor log_dt, Tensor[] norm_scales, "
        "Tensor[] gate_values, Tensor[] gate_col_idx, Tensor[] up_values, Tensor[] up_col_idx, "
        "Tensor[] down_values, Tensor[] down_col_idx) -> Tensor");
  // ops beyond the reference's set
  m.def("block_ell_matmul(Tensor x, Tensor values, Tensor col_indices, Tensor? bias=None) -> Tensor");
  m.def("block_ell_matmul_bwd(Tensor grad_out, Tensor x, Tensor values, Tensor col_indices) -> (Tensor, Tensor)");
  m.def("block_ell_matmul_prepack(Tensor values, Tensor col_indices, int in_features) -> Tensor");
  m.def("block_ell_matmul_prepacked(Tensor x, Tensor packed, Tensor values, Tensor col_indices, Tensor? bias=None) "
        "-> Tensor");
  m.def("block_ell_swiglu_fwd_bias(Tensor x, Tensor v_gate, Tensor ci_gate, Tensor? b_gate, Tensor v_up, "
        "Tensor ci_up, Tensor? b_up, Tensor v_down, Tensor ci_down, Tensor? b_down, bool add_residual, "
        "bool intermediates=False) -> (Tensor, Tensor, Tensor, Tensor)");
  m.def("block_ell_swiglu_prepack(Tensor v_gate, Tensor ci_gate, Tensor v_up, Tensor ci_up, Tensor v_down, "
        "Tensor ci_down) -> Tensor");
  m.def("block_ell_swiglu_fwd_prepacked(Tensor x, Tensor packed, Tensor v_gate, Tensor ci_gate, Tensor? b_gate, "
        "Tensor v_up, Tensor ci_up, Tensor? b_up, Tensor v_down, Tensor ci_down, Tensor? b_down, "
        "bool add_residual) -> Tensor");
  m.def("block_ell_swiglu_bwd_bias(Tensor grad_out, Tensor x, Tensor gate_pre_act, Tensor up_out, Tensor h, "
        "Tensor v_gate, Tensor ci_gate, Tensor v_up, Tensor ci_up, Tensor v_down, Tensor ci_down, "
        "bool add_residual) -> (Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor)");
  m.def("looped_swiglu_bias(Tensor h, Tensor norm_scale, Tensor v_gate, Tensor ci_gate, Tensor? b_gate, "
        "Tensor v_up, Tensor ci_up, Tensor? b_up, Tensor v_down, Tensor ci_down, Tensor? b_down, int L, "
        "float eps=1e-05) -> Tensor");
  m.def("block_ell_swiglu_bwd_ex(Tensor grad_out, Tensor x, Tensor gate_pre_act, Tensor up_out, Tensor h, "
        "Tensor v_gate, Tensor ci_gate, Tensor v_up, Tensor ci_up, Tensor v_down, Tensor ci_down, "
        "bool add_residual) -> (Tensor, Tensor, Tensor, Tensor)");
  m.def("looped_swiglu(Tensor h, Tensor norm_scale, Tensor v_gate, Tensor ci_gate, Tensor v_up, Tensor ci_up, "
        "Tensor v_down, Tensor ci_down, int L, float eps=1e-05) -> Tensor");
  m.def("looped_swiglu_persistent(Tensor h, Tensor norm_scale, Tensor v_gate, Tensor ci_gate, Tensor v_up, "
        "Tensor ci_up, Tensor v_down, Tensor ci_down, int L, float eps=1e-05) -> Tensor");
  m.def("looped_swiglu_launches(Tensor h, Tensor norm_scale, Tensor v_gate, Tensor ci_gate, Tensor v_up, "
        "Tensor ci_up, Tensor v_down, Tensor ci_down, int L, float eps=1e-05) -> Tensor");
  m.def("looped_core(Tensor h, Tensor? e, Tensor? log_A, Tensor? log_dt, Tensor[] norm_scales, "
        "Tensor[] gate_values, Tensor[] gate_col_idx, Tensor[] up_values, Tensor[] up_col_idx, "
        "Tensor[] down_values, Tensor[] down_col_idx, Tensor?[] biases, int L, Tensor? depths=None, "
        "int seq_len=1, float eps=1e-05, bool persistent=False) -> Tensor");
  m.def("rmsnorm(Tensor x, Tensor scale, float eps=1e-05) -> Tensor");
  m.def("rmsnorm_bwd(Tensor grad_out, Tensor x, Tensor scale, float eps=1e-05) -> (Tensor, Tensor)");
  m.def("diagonal_injection(Tensor h, Tensor e, Tensor log_A, Tensor log_dt) -> Tensor");
  m.def("diagonal_injection_bwd(Tensor grad_out, Tensor h, Tensor e, Tensor log_A, Tensor log_dt) "
        "-> (Tensor, Tensor, Tensor, Tensor)");
  m.def("quantize_act_int8(Tensor x) -> (Tensor, Tensor)");
  m.def("pack_ternary(Tensor t) -> Tensor");
  m.def("ternary_quantize_weights(Tensor values) -> (Tensor, Tensor)");
  m.def("ternary_matmul(Tensor xq, Tensor sx, Tensor packed, Tensor scales, Tensor col_indices, "
        "bool want_partials=False) -> (Tensor, Tensor)");
  m.def("block_ell_swiglu_fwd_ternary(Tensor xq, Tensor sx, Tensor p_gate, Tensor s_gate, Tensor ci_gate, "
        "Tensor p_up, Tensor s_up, Tensor ci_up, Tensor p_down, Tensor s_down, Tensor ci_down, "
        "Tensor? x_resid=None) -> Tensor");
  m.def("block_ell_swiglu_fwd_ternary_with_intermediate(Tensor xq, Tensor sx, Tensor p_gate, Tensor s_gate, "
        "Tensor ci_gate, Tensor p_up, Tensor s_up, Tensor ci_up, Tensor p_down, Tensor s_down, Tensor ci_down, "
        "Tensor? x_resid=None) -> (Tensor, Tensor, Tensor, Tensor)");
  m.def("block_ell_swiglu_fwd_ternary_accumulators(Tensor xq, Tensor sx, Tensor p_gate, Tensor s_gate, "
        "Tensor ci_gate, Tensor p_up, Tensor s_up, Tensor ci_up, Tensor p_down, Tensor s_down, Tensor ci_down, "
        "Tensor? x_resid=None) -> (Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor)");
  m.def("check_columns(Tensor col_indices, int C) -> Tensor");
  m.def("ternary_prepare(Tensor p_gate, Tensor s_gate, Tensor ci_gate, Tensor p_up, Tensor s_up, Tensor ci_up, "
        "Tensor p_down, Tensor s_down, Tensor ci_down) -> Tensor");
  m.def("block_ell_swiglu_fwd_ternary_prepared(Tensor xq, Tensor sx, Tensor prepared, Tensor p_gate, Tensor s_gate, "
        "Tensor ci_gate, Tensor p_up, Tensor s_up, Tensor ci_up, Tensor p_down, Tensor s_down, Tensor ci_down, "
        "Tensor? x_resid=None) -> Tensor");
}

TORCH_LIBRARY_IMPL(titan, CUDA, m) {
  m.impl("block_ell_swiglu_fwd", &swiglu_fwd);
  m.impl("block_ell_swiglu_fwd_with_intermediate", &swiglu_fwd_inter);
  m.impl("block_ell_swiglu_bwd", &swiglu_bwd);
  m.impl("block_ell_swiglu_bwd_ex", &swiglu_bwd_ex);
  m.impl("block_ell_swiglu_fwd_bias", &swiglu_fwd_bias);
  m.impl("block_ell_swiglu_bwd_bias", &swiglu_bwd_bias);
  m.impl("block_ell_swiglu_prepack", &swiglu_prepack);
  m.impl("block_ell_swiglu_fwd_prepacked", &swiglu_fwd_prepacked);
  m.impl("looped_swiglu_bias", &looped_swiglu_bias);
  m.impl("pin_weights_l2", &pin_weights_l2);
  m.impl("persistent_mlp_step", &persistent_mlp_step);
  m.impl("block_ell_matmul", &block_ell_matmul);
  m.impl("block_ell_matmul_bwd", &block_ell_matmul_bwd);
  m.impl("block_ell_matmul_prepack", &block_ell_matmul_prepack);
  m.impl("block_ell_matmul_prepacked", &block_ell_matmul_prepacked);
  m.impl("looped_swiglu", &looped_swiglu);
  m.impl("looped_swiglu_persistent", &looped_swiglu_persistent);
  m.impl("looped_swiglu_launches", &looped_swiglu_launches);
  m.impl("looped_core", &looped_core);
  m.impl("rmsnorm", &rmsnorm);
  m.impl("rmsnorm_bwd", &rmsnorm_bwd);
  m.impl("diagonal_injection", &diagonal_injection);
  m.impl("diagonal_injection_bwd", &diagonal_injection_bwd);
  m.impl("quantize_act_int8", &quantize_act_int8);
  m.impl("pack_ternary", &pack_ternary);
  m.impl("ternary_quantize_weights", &ternary_quantize_weights);
  m.impl("ternary_matmul", &ternary_matmul);
  m.impl("block_ell_swiglu_fwd_ternary", &tern_swiglu);
  m.impl("block_ell_swiglu_fwd_ternary_with_intermediate", &tern_swiglu_inter);
  m.impl("block_ell_swiglu_fwd_ternary_accumulators", &tern_swiglu_accs);
  m.impl("check_columns", &check_columns);
  m.impl("ternary_prepare", &ternary_prepare);
  m.impl("block_ell_swiglu_fwd_ternary_prepared", &tern_swiglu_prepared);
}

TORCH_LIBRARY_IMPL(titan, CompositeExplicitAutograd, m) { m.impl("unpin_weights_l2", &unpin_weights_l2); }

// No operator here has an autograd formula of its own (the differentiable ones are wrapped by
// torch.autograd.Function in looped_blockell.kernels, which call them with grad mode off).
// Outputs of an op called on inputs that require grad get a node that raises on backward,
// instead of silently carrying no gradient.
TORCH_LIBRARY_IMPL(titan, Autograd, m) {
  for (const char* name :
       {"block_ell_swiglu_fwd", "block_ell_swiglu_fwd_with_intermediate", "block_ell_swiglu_bwd",
        "persistent_mlp_step", "block_ell_matmul", "block_ell_matmul_bwd", "block_ell_swiglu_bwd_ex",
        "block_ell_matmul_prepack", "block_ell_matmul_prepacked",
        "looped_swiglu", "looped_swiglu_persistent", "looped_swiglu_launches", "looped_core", "rmsnorm",
        "rmsnorm_bwd",
        "block_ell_swiglu_fwd_bias", "block_ell_swiglu_bwd_bias", "looped_swiglu_bias",
        "block_ell_swiglu_prepack", "block_ell_swiglu_fwd_prepacked", "diagonal_injection", "diagonal_injection_bwd",
        "quantize_act_int8", "pack_ternary", "ternary_quantize_weights", "ternary_matmul",
        "block_ell_swiglu_fwd_ternary", "block_ell_swiglu_fwd_ternary_with_intermediate",
        "block_ell_swiglu_fwd_ternary_accumulators", "ternary_prepare", "block_ell_swiglu_fwd_ternary_prepared"})
    m.impl(name, torch::autograd::autogradNotImplementedFallback());
}

// Meta (shape-only) implementations, as the reference provides for FakeTensor tracing
// (csrc/block_ell/block_ell_ops.cpp:179-237, csrc/loop/loop_ops.cpp:125-156).
TORCH_LIBRARY_IMPL(titan, Meta, m) {
  m.impl("block_ell_swiglu_fwd", [](const at::Tensor& x, const at::Tensor&, const at::Tensor&, const at::Tensor&,
                                    const at::Tensor&, const at::Tensor&, const at::Tensor&, bool) {
    return at::empty_like(x);
  });
  m.impl("block_ell_swiglu_fwd_with_intermediate",
         [](const at::Tensor& x, const at::Tensor& vg, const at::Tensor&, const at::Tensor&, const at::Tensor&,
            const at::Tensor&, const at::Tensor&, bool) {
           const int64_t N = x.size(0), d_ff = vg.size(0) * vg.size(2);
           return std::make_tuple(at::empty_like(x), at::empty({N, d_ff}, x.options()),
                                  at::empty({N, d_ff}, x.options()), at::empty({N, d_ff}, x.options()));
         });
  m.impl("block_ell_swiglu_bwd",
         [](const at::Tensor&, const at::Tensor& x, const at::Tensor&, const at::Tensor&, const at::Tensor&,
            const at::Tensor& vg, const at::Tensor&, const at::Tensor& vu, const at::Tensor&, const at::Tensor& vd,
            const at::Tensor&) {
           return std::make_tuple(at::empty_like(x), at::empty_like(vg), at::empty_like(vu), at::empty_like(vd));
         });
  m.impl("block_ell_swiglu_bwd_ex",
         [](const at::Tensor&, const at::Tensor& x, const at::Tensor&, const at::Tensor&, const at::Tensor&,
            const at::Tensor& vg, const at::Tensor&, const at::Tensor& vu, const at::Tensor&, const at::Tensor& vd,
            const at::Tensor&, bool) {
           return std::make_tuple(at::empty_like(x), at::empty_like(vg), at::empty_like(vu), at::empty_like(vd));
         });
  m.impl("block_ell_swiglu_fwd_bias",
         [](const at::Tensor& x, const at::Tensor& vg, const at::Tensor&, const c10::optional<at::Tensor>&,
            const at::Tensor&, const at::Tensor&, const c10::optional<at::Tensor>&, const at::Tensor&,
            const at::Tensor&, const c10::optional<at::Tensor>&, bool, bool inter) {
           const int64_t N = x.size(0), d_ff = vg.size(0) * vg.size(2);
           auto mk = [&]() { return inter ? at::empty({N, d_ff}, x.options()) : at::empty({0}, x.options()); };
           return std::make_tuple(at::empty_like(x), mk(), mk(), mk());
         });
  m.impl("block_ell_swiglu_bwd_bias",
         [](const at::Tensor&, const at::Tensor& x, const at::Tensor&, const at::Tensor&, const at::Tensor&,
            const at::Tensor& vg, const at::Tensor&, const at::Tensor& vu, const at::Tensor&, const at::Tensor& vd,
            const at::Tensor&, bool) {
           const int64_t d_ff = vg.size(0) * vg.size(2);
           auto f = x.options().dtype(at::kFloat);
           return std::make_tuple(at::empty_like(x), at::empty_like(vg), at::empty_like(vu), at::empty_like(vd),
                                  at::empty({d_ff}, f), at::empty({d_ff}, f), at::empty({x.size(1)}, f));
         });
  m.impl("block_ell_swiglu_fwd_prepacked",
         [](const at::Tensor& x, const at::Tensor&, const at::Tensor&, const at::Tensor&,
            const c10::optional<at::Tensor>&, const at::Tensor&, const at::Tensor&, const c10::optional<at::Tensor>&,
            const at::Tensor&, const at::Tensor&, const c10::optional<at::Tensor>&, bool) { return at::empty_like(x); });
  m.impl("looped_swiglu_bias",
         [](const at::Tensor& h, const at::Tensor&, const at::Tensor&, const at::Tensor&,
            const c10::optional<at::Tensor>&, const at::Tensor&, const at::Tensor&, const c10::optional<at::Tensor>&,
            const at::Tensor&, const at::Tensor&, const c10::optional<at::Tensor>&, int64_t,
            double) { return at::empty_like(h); });
  m.impl("pin_weights_l2", [](at::TensorList) {});
  m.impl("persistent_mlp_step",
         [](const at::Tensor& h, const at::Tensor&, const at::Tensor&, const at::Tensor&, at::TensorList,
            at::TensorList, at::TensorList, at::TensorList, at::TensorList, at::TensorList,
            at::TensorList) { return at::empty_like(h); });
  m.impl("block_ell_matmul", [](const at::Tensor& x, const at::Tensor& v, const at::Tensor&,
                                const c10::optional<at::Tensor>&) {
    return at::empty({x.size(0), v.size(0) * v.size(2)}, x.options());
  });
  m.impl("block_ell_matmul_prepacked", [](const at::Tensor& x, const at::Tensor&, const at::Tensor& v, const at::Tensor&,
                                          const c10::optional<at::Tensor>&) {
    return at::empty({x.size(0), v.size(0) * v.size(2)}, x.options());
  });
  m.impl("block_ell_matmul_bwd", [](const at::Tensor&, const at::Tensor& x, const at::Tensor& v, const at::Tensor&) {
    return std::make_tuple(at::empty_like(x), at::empty_like(v));
  });
  m.impl("looped_swiglu", [](const at::Tensor& h, const at::Tensor&, const at::Tensor&, const at::Tensor&,
                             const at::Tensor&, const at::Tensor&, const at::Tensor&, const at::Tensor&, int64_t,
                             double) { return at::empty_like(h); });
  m.impl("looped_swiglu_persistent", [](const at::Tensor& h, const at::Tensor&, const at::Tensor&, const at::Tensor&,
                             const at::Tensor&, const at::Tensor&, const at::Tensor&, const at::Tensor&, int64_t,
                             double) { return at::empty_like(h); });
  m.impl("looped_core",
         [](const at::Tensor& h, const c10::optional<at::Tensor>&, const c10::optional<at::Tensor>&,
            const c10::optional<at::Tensor>&, at::TensorList, at::TensorList, at::TensorList, at::TensorList,
            at::TensorList, at::TensorList, at::TensorList, const c10::List<c10::optional<at::Tensor>>&, int64_t,
            const c10::optional<at::Tensor>&, int64_t, double, bool) { return at::empty_like(h); });
  m.impl("looped_swiglu_launches", [](const at::Tensor& h, const at::Tensor&, const at::Tensor&, const at::Tensor&,
                             const at::Tensor&, const at::Tensor&, const at::Tensor&, const at::Tensor&, int64_t,
                             double) { return at::empty_like(h); });
  m.impl("rmsnorm", [](const at::Tensor& x, const at::Tensor&, double) { return at::empty_like(x); });
  m.impl("rmsnorm_bwd", [](const at::Tensor&, const at::Tensor& x, const at::Tensor&, double) {
    return std::make_tuple(at::empty_like(x), at::empty({x.size(1)}, x.options().dtype(at::kFloat)));
  });
  m.impl("diagonal_injection_bwd", [](const at::Tensor&, const at::Tensor& h, const at::Tensor&, const at::Tensor&,
                                      const at::Tensor&) {
    auto f = h.options().dtype(at::kFloat);
    return std::make_tuple(at::empty_like(h), at::empty_like(h), at::empty({h.size(1)}, f), at::empty({h.size(1)}, f));
  });
  m.impl("diagonal_injection", [](const at::Tensor& h, const at::Tensor&, const at::Tensor&, const at::Tensor&) {
    return at::empty_like(h);
  });
  m.impl("quantize_act_int8", [](const at::Tensor& x) {
    return std::make_tuple(at::empty(x.sizes(), x.options().dtype(at::kChar)),
                           at::empty({x.size(0)}, x.options().dtype(at::kFloat)));
  });
  m.impl("pack_ternary", [](const at::Tensor& t) {
    return at::empty({t.size(0), t.size(1), t.size(2), t.size(2) / 16}, t.options().dtype(at::kInt));
  });
  m.impl("ternary_quantize_weights", [](const at::Tensor& v) {
    return std::make_tuple(at::empty({v.size(0), v.size(1), v.size(2), v.size(2) / 16}, v.options().dtype(at::kInt)),
                           at::empty({v.size(0), v.size(1)}, v.options().dtype(at::kFloat)));
  });
  m.impl("ternary_matmul", [](const at::Tensor& xq, const at::Tensor&, const at::Tensor& p, const at::Tensor&,
                              const at::Tensor&, bool want) {
    return std::make_tuple(at::empty({xq.size(0), p.size(0) * p.size(2)}, xq.options().dtype(at::kBFloat16)),
                           want ? at::empty({xq.size(0), p.size(0), p.size(1), p.size(2)}, xq.options().dtype(at::kInt))
                                : at::empty({0}, xq.options().dtype(at::kInt)));
  });
  m.impl("block_ell_swiglu_fwd_ternary",
         [](const at::Tensor& xq, const at::Tensor&, const at::Tensor&, const at::Tensor&, const at::Tensor&,
            const at::Tensor&, const at::Tensor&, const at::Tensor&, const at::Tensor&, const at::Tensor&,
            const at::Tensor&, const c10::optional<at::Tensor>&) {
           return at::empty(xq.sizes(), xq.options().dtype(at::kBFloat16));
         });
  m.impl("block_ell_swiglu_fwd_ternary_prepared",
         [](const at::Tensor& xq, const at::Tensor&, const at::Tensor&, const at::Tensor&, const at::Tensor&,
            const at::Tensor&, const at::Tensor&, const at::Tensor&, const at::Tensor&, const at::Tensor&,
            const at::Tensor&, const at::Tensor&, const c10::optional<at::Tensor>&) {
           return at::empty(xq.sizes(), xq.options().dtype(at::kBFloat16));
         });
  m.impl("block_ell_swiglu_fwd_ternary_with_intermediate",
         [](const at::Tensor& xq, const at::Tensor&, const at::Tensor& pg, const at::Tensor&, const at::Tensor&,
            const at::Tensor&, const at::Tensor&, const at::Tensor&, const at::Tensor&, const at::Tensor&,
            const at::Tensor&, const c10::optional<at::Tensor>&) {
           const int64_t N = xq.size(0), d_ff = pg.size(0) * pg.size(2);
           return std::make_tuple(at::empty(xq.sizes(), xq.options().dtype(at::kBFloat16)),
                                  at::empty({N, d_ff}, xq.options().dtype(at::kBFloat16)),
                                  at::empty({N, d_ff}, xq.options().dtype(at::kChar)),
                                  at::empty({N}, xq.options().dtype(at::kFloat)));
         });
  m.impl("block_ell_swiglu_fwd_ternary_accumulators",
         [](const at::Tensor& xq, const at::Tensor&, const at::Tensor& pg, const at::Tensor&, const at::Tensor&,
            const at::Tensor&, const at::Tensor&, const at::Tensor&, const at::Tensor&, const at::Tensor&,
            const at::Tensor&, const c10::optional<at::Tensor>&) {
           const int64_t N = xq.size(0), d_ff = pg.size(0) * pg.size(2);
           auto o = xq.options();
           return std::make_tuple(at::empty(xq.sizes(), o.dtype(at::kBFloat16)), at::empty({N, d_ff}, o.dtype(at::kBFloat16)),
                                  at::empty({N, d_ff}, o.dtype(at::kChar)), at::empty({N}, o.dtype(at::kFloat)),
                                  at::empty({N, d_ff}, o.dtype(at::kInt)), at::empty({N, d_ff}, o.dtype(at::kInt)),
                                  at::empty(xq.sizes(), o.dtype(at::kInt)), at::empty({N, d_ff}, o.dtype(at::kFloat)),
                                  at::empty({N, d_ff}, o.dtype(at::kFloat)));
         });
  m.impl("check_columns", [](const at::Tensor& c, int64_t) { return at::empty({}, c.options()); });
}
