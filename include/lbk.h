/*
 * lbk.h — C ABI of the MI355X (gfx950) Block-ELL SwiGLU FFN library (liblbk.so).
 *
 * Everything here is plain C: pointers, sizes, status codes.  No torch types.
 * The library never allocates, frees or synchronises: callers own every buffer
 * (inputs, outputs, workspace) and pass the HIP stream the work is queued on.
 * Entry points are reentrant and keep no global state, with one exception:
 * lbk_swiglu_fwd_bf16_noalloc works in a fixed device array per GPU (below), so
 * its calls that overlap in time on one GPU race.  A workspace buffer may be
 * shared by calls only if those calls do not overlap in time.
 *
 * Block-ELL layout (reference looped_blockell/layers/block_ell.py:1-8, :53-66):
 *   values      [R, K, B, B]  bf16; tile values[r, k] is [B_in, B_out]
 *   col_idx     [R, K]        int32; input column block of each tile,
 *                             -1 = dead slot, skipped
 *                             (reference looped_blockell/opt/cms.py:229-230)
 *   B in {16, 32, 64}; the weight maps in = C*B features to out = R*B features.
 * Activations are row-major [N, features] bf16 with a row stride in elements.
 * bf16 values travel as uint16_t bit patterns.
 */
#ifndef LBK_H
#define LBK_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LBK_VERSION 1

/* Status codes (never exceptions across the ABI). */
enum {
    LBK_OK = 0,
    LBK_ERR_NULL = 1,          /* a required pointer is NULL */
    LBK_ERR_TILE = 2,          /* B not in {16, 32, 64} (or ternary B not a multiple of 16) */
    LBK_ERR_SHAPE = 3,         /* inconsistent R / K / features between operands */
    LBK_ERR_ALIGN = 4,         /* pointer or row stride not 16-byte aligned */
    LBK_ERR_WORKSPACE = 5,     /* workspace missing or smaller than required */
    LBK_ERR_LAUNCH = 6,        /* HIP reported an error launching a kernel */
    LBK_ERR_ARG = 7,           /* other invalid argument (N < 0, L < 0, eps < 0 ...) */
    LBK_ERR_COLUMN = 8,        /* reserved: column index >= C found by lbk_check_columns */
    LBK_ERR_TOO_LARGE = 9      /* the geometry needs more than the no-alloc entry point's fixed scratch */
};

/* Size of the fixed device scratch array behind lbk_swiglu_fwd_bf16_noalloc (per GPU). */
#define LBK_NOALLOC_SCRATCH_BYTES (4u << 20)

/* One Block-ELL weight with bf16 tiles. */
typedef struct lbk_bell {
    const uint16_t* values;    /* [R, K, B, B] bf16, tile [B_in, B_out], contiguous */
    const int32_t* col_idx;    /* [R, K] int32, -1 = dead slot */
    int32_t R, K, B;
} lbk_bell;

/* One ternary Block-ELL weight (format defined by this library):
 *   packed [R, K, B_out, B_in/16] uint32 — word (r,k,D,e) holds t[r,k,16e+i,D],
 *          i = 0..15, as a 2-bit code at bit 8*(i%4) + 2*(i/4);
 *          code 0b00 -> 0, 0b01 -> +1, 0b11 -> -1 (0b10 decodes to 0);
 *   scales [R, K] fp32 — one absmean scale per block. */
typedef struct lbk_bell_ternary {
    const uint32_t* packed;
    const float* scales;
    const int32_t* col_idx;
    int32_t R, K, B;
} lbk_bell_ternary;

/* Human-readable text of a status code (static storage). */
const char* lbk_status_string(int status);
int lbk_version(void);

/*
 * Validate that every column index lies in [-1, C).  Writes the number of
 * offending entries to *bad_count_dev (device int32, zeroed by this call).
 * Replaces nothing in the reference (the reference CUDA op does not check
 * columns, csrc/block_ell/swiglu_fwd.cu:236-256); used by the torch layer's
 * debug checks.
 */
int lbk_check_columns(const int32_t* col_idx, int64_t count, int32_t C, int32_t* bad_count_dev,
                      void* stream);

/*
 * y[N, R*B] = x[N, C*B] (Block-ELL) W   (+ bias[R*B] if bias != NULL)
 * Replaces block_ell_matmul (reference looped_blockell/layers/block_ell.py:149-182)
 * plus BlockELLLinear's bias (reference looped_blockell/layers/mlp.py:82).
 */
int lbk_block_ell_matmul_bf16(const uint16_t* x, int64_t N, int32_t in_features, int64_t ldx,
                              const lbk_bell* w, const float* bias, uint16_t* y, int64_t ldy,
                              void* stream);

/*
 * lbk_block_ell_matmul_bf16 for contiguous rows (ldx = in_features, ldy = R*B) with a workspace:
 * the tiles are packed into it (fragment-major) and the product runs on the SwiGLU kernels'
 * machinery -- the gate/up kernel's gate stream over an LDS panel of x when in_features is a
 * multiple of 128 up to 2048, the down kernel (x staged through LDS 512 columns at a time) for
 * wider inputs -- for B in {16, 32}; other shapes take the row-block kernel and need no
 * workspace (lbk_block_ell_matmul_workspace_bytes returns 0).  Same contract and result
 * (within float32 summation order) as lbk_block_ell_matmul_bf16.
 */
size_t lbk_block_ell_matmul_workspace_bytes(int64_t N, int32_t in_features, const lbk_bell* w);
int lbk_block_ell_matmul_ws_bf16(const uint16_t* x, int64_t N, int32_t in_features, const lbk_bell* w,
                                 const float* bias, uint16_t* y, void* workspace, size_t workspace_bytes,
                                 void* stream);

/*
 * The same product on tiles packed once (weights fixed across calls): lbk_block_ell_matmul_prepack_bf16
 * fills a buffer of lbk_block_ell_matmul_prepacked_bytes (0: the shape has no packed form, the
 * prepack is a no-op and the product takes the row-block kernel), reflecting values and col_idx
 * at the time of the call; lbk_block_ell_matmul_prepacked_bf16 then needs no workspace.  No
 * counterpart in the reference (its JAX product has no weight preparation).
 */
size_t lbk_block_ell_matmul_prepacked_bytes(int32_t in_features, const lbk_bell* w);
int lbk_block_ell_matmul_prepack_bf16(int32_t in_features, const lbk_bell* w, void* packed, size_t packed_bytes,
                                      void* stream);
int lbk_block_ell_matmul_prepacked_bf16(const uint16_t* x, int64_t N, int32_t in_features, const lbk_bell* w,
                                        const void* packed, size_t packed_bytes, const float* bias, uint16_t* y,
                                        void* stream);

/*
 * Workspace bytes needed by lbk_swiglu_fwd_bf16 for this geometry: packed
 * copies of the gate/up/down tiles (two-kernel path) plus the hidden state h
 * [N, d_ff] bf16 unless want_intermediates (then the caller passes h_out).
 */
size_t lbk_swiglu_workspace_bytes(int64_t N, int32_t d_model, const lbk_bell* gate,
                                  const lbk_bell* up, const lbk_bell* down, int want_intermediates);

/*
 * out[N, d_model] = W_down( silu(W_gate x) * (W_up x) )  (+ x if add_residual)
 * Optional outputs (NULL to skip; all [N, d_ff] bf16, row stride d_ff):
 *   h_out = silu(gate)*up, gate_pre_out = W_gate x, up_out = W_up x.
 * Replaces titan::block_ell_swiglu_fwd and ..._with_intermediate
 * (reference csrc/block_ell/block_ell_ops.cpp:51-76, csrc/block_ell/swiglu_fwd.cuh:75-141).
 * x and out are contiguous [N, d_model].
 */
int lbk_swiglu_fwd_bf16(const uint16_t* x, int64_t N, int32_t d_model,
                        const lbk_bell* gate, const lbk_bell* up, const lbk_bell* down,
                        int add_residual, uint16_t* out,
                        uint16_t* h_out, uint16_t* gate_pre_out, uint16_t* up_out,
                        void* workspace, size_t workspace_bytes, void* stream);

/*
 * Which kernels lbk_swiglu_fwd_bf16 (and its biased and prepacked forms) runs for a geometry:
 * LBK_PATH_DECODE (N <= 64 tokens: the decode pair), LBK_PATH_SPLIT (the two-kernel gate/up +
 * down path on packed tiles), LBK_PATH_ROWBLOCK (the general row-block kernels), or
 * LBK_PATH_NONE for N <= 0 or an invalid geometry.  want_intermediates as for
 * lbk_swiglu_workspace_bytes.  A query only (no launch); no counterpart in the reference, for
 * callers and tests that need to know which kernels serve a shape.
 */
enum lbk_path { LBK_PATH_NONE = 0, LBK_PATH_DECODE = 1, LBK_PATH_SPLIT = 2, LBK_PATH_ROWBLOCK = 3 };
int lbk_swiglu_forward_path(int64_t N, int32_t d_model, const lbk_bell* gate, const lbk_bell* up,
                            const lbk_bell* down, int want_intermediates);

/*
 * lbk_swiglu_fwd_bf16 (no optional outputs) for callers that cannot allocate: code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc.  No counterpart in the
 * reference.  Instead of a workspace it uses a fixed array of LBK_NOALLOC_SCRATCH_BYTES (4 MiB)
 * in device memory, one per GPU, held until the process ends; the call itself allocates and
 * frees nothing.  Geometries whose workspace (lbk_swiglu_workspace_bytes with
 * want_intermediates = 0) exceeds the array return LBK_ERR_TOO_LARGE without launching
 * anything: decode shapes fit (16 tokens at d_ff = 14336 need 459 KB).  All calls on one GPU
 * share its array: calls that overlap in time on one GPU race.  Same kernels, same results as
 * lbk_swiglu_fwd_bf16.
 *
 * lbk_noalloc_init looks up the device address of the current device's array (once per
 * device; later calls return at once).  The first lbk_swiglu_fwd_bf16_noalloc call on a device
 * does it too, but a caller about to capture a HIP graph calls lbk_noalloc_init (and makes one
 * eager call of each geometry, which sets the kernels' LDS limits) before the capture, so that
 * the captured call makes no runtime lookups.  The captured call records kernel launches only.
 */
size_t lbk_noalloc_scratch_bytes(void);
int lbk_noalloc_init(void);
int lbk_swiglu_fwd_bf16_noalloc(const uint16_t* x, int64_t N, int32_t d_model,
                                const lbk_bell* gate, const lbk_bell* up, const lbk_bell* down,
                                int add_residual, uint16_t* out, void* stream);

/*
 * lbk_swiglu_fwd_bf16 with the projections' biases (each fp32, optional):
 *   out = W_down(silu(W_gate x + b_gate) * (W_up x + b_up)) + b_down  (+ x if add_residual)
 * b_gate, b_up [d_ff], b_down [d_model]; gate_pre_out / up_out then hold W_gate x + b_gate and
 * W_up x + b_up.  The biases are added in fp32 in the kernels' epilogues.  Replaces the biased
 * BlockELLLinear projections of the reference's SwiGLU MLPBlock
 * (looped_blockell/layers/mlp.py:56-60, :82, :119-145).  Same workspace as lbk_swiglu_fwd_bf16.
 */
int lbk_swiglu_fwd_bias_bf16(const uint16_t* x, int64_t N, int32_t d_model,
                             const lbk_bell* gate, const lbk_bell* up, const lbk_bell* down,
                             const float* b_gate, const float* b_up, const float* b_down,
                             int add_residual, uint16_t* out,
                             uint16_t* h_out, uint16_t* gate_pre_out, uint16_t* up_out,
                             void* workspace, size_t workspace_bytes, void* stream);

/*
 * Weights packed once, forwards without the per-call pack.  The two-kernel path reads the
 * gate/up/down tiles in a fragment-major packed copy that lbk_swiglu_fwd_bf16 rebuilds on
 * every call; a caller whose weights do not change between forwards (inference, a decode
 * loop) builds it once with lbk_swiglu_prepack_bf16 into a buffer of
 * lbk_swiglu_prepacked_bytes and passes it to lbk_swiglu_fwd_prepacked_bf16.  The packed
 * copy reflects values and col_idx at the time of the prepack (dead and out-of-range slots
 * become zero tiles): pack again after either changes.  lbk_swiglu_prepacked_bytes returns 0
 * for geometries that read the tiles directly (no packed form); the prepack is then a no-op
 * and the forward ignores the buffer.  No counterpart in the reference, whose kernel reads
 * the tiles in place (csrc/block_ell/swiglu_fwd.cu:273-284); this layout's packing is the
 * part of titan::block_ell_swiglu_fwd (csrc/block_ell/block_ell_ops.cpp:51-63) that a caller
 * with fixed weights can hoist out of the loop.
 */
size_t lbk_swiglu_prepacked_bytes(int32_t d_model, const lbk_bell* gate, const lbk_bell* up,
                                  const lbk_bell* down);
int lbk_swiglu_prepack_bf16(int32_t d_model, const lbk_bell* gate, const lbk_bell* up,
                            const lbk_bell* down, void* packed, size_t packed_bytes, void* stream);

/*
 * lbk_swiglu_fwd_bias_bf16 from a prepacked copy (biases optional, as there).  gate/up/down
 * still describe the weights (col_idx, R, K, B; values are read on the decode and general
 * paths).  The workspace holds h [N, d_ff] bf16 unless h_out is given:
 * lbk_swiglu_prepacked_workspace_bytes.  Same kernels and results as lbk_swiglu_fwd_bias_bf16.
 */
size_t lbk_swiglu_prepacked_workspace_bytes(int64_t N, int32_t d_model, const lbk_bell* gate,
                                            const lbk_bell* up, const lbk_bell* down,
                                            int want_intermediates);
int lbk_swiglu_fwd_prepacked_bf16(const uint16_t* x, int64_t N, int32_t d_model,
                                  const lbk_bell* gate, const lbk_bell* up, const lbk_bell* down,
                                  const void* packed, size_t packed_bytes,
                                  const float* b_gate, const float* b_up, const float* b_down,
                                  int add_residual, uint16_t* out,
                                  uint16_t* h_out, uint16_t* gate_pre_out, uint16_t* up_out,
                                  void* workspace, size_t workspace_bytes, void* stream);

/*
 * Workspace bytes needed by lbk_swiglu_bwd_bf16 for this geometry: the transposed
 * column lists of the three weights, dg and du [N, d_ff] bf16, and fp32 partial
 * tile gradients (one set per 2048 tokens; per 1024 for a weight whose input rows are too
 * wide to stage and whose output rows are at most 1024 wide, e.g. the down weight, when
 * the token count fills the GPU).
 */
size_t lbk_swiglu_bwd_workspace_bytes(int64_t N, int32_t d_model, const lbk_bell* gate,
                                      const lbk_bell* up, const lbk_bell* down);

/*
 * Backward of out = W_down(silu(W_gate x) * (W_up x)) (+ x) for an output gradient
 * grad_out [N, d_model], from the forward's saved x, gate_pre_act = W_gate x,
 * up_output = W_up x and h (all bf16; the last three [N, d_ff], as
 * lbk_swiglu_fwd_bf16 returns them):
 *   dx             [N, d_model]  = dg W_gate + du W_up (+ grad_out if add_residual; the
 *                  reference operator always adds it)
 *   d_gate_values  [R_ff, K_g, B, B], d_up_values, d_down_values: tile gradients in the
 *                  values layout ([B_in, B_out] tiles); dead slots (col < 0 or >= C) get 0
 * with dh = grad_out W_down, dg = dh * up * silu'(gate), du = dh * silu(gate); fp32
 * accumulation, dg and du rounded to bf16 before the second products (as the
 * reference does).  No atomics: the results are deterministic.
 * Replaces titan::block_ell_swiglu_bwd (reference csrc/block_ell/block_ell_ops.cpp:78-97,
 * csrc/block_ell/swiglu_bwd.cu:608-834); B in {16, 32, 64}.
 */
int lbk_swiglu_bwd_bf16(const uint16_t* grad_out, const uint16_t* x, const uint16_t* gate_pre_act,
                        const uint16_t* up_output, const uint16_t* h, int64_t N, int32_t d_model,
                        const lbk_bell* gate, const lbk_bell* up, const lbk_bell* down, int add_residual,
                        uint16_t* dx, uint16_t* d_gate_values, uint16_t* d_up_values,
                        uint16_t* d_down_values, void* workspace, size_t workspace_bytes, void* stream);

/*
 * lbk_swiglu_bwd_bf16 plus the bias gradients of lbk_swiglu_fwd_bias_bf16 (each optional, fp32):
 * d_b_gate = column sums of dg, d_b_up = of du [d_ff], d_b_down = of grad_out [d_model],
 * summed per 64-row group and the groups in a fixed order (deterministic).  gate_pre_act and
 * up_output are the forward's biased pre-activations.  Its workspace
 * (lbk_swiglu_bwd_bias_workspace_bytes) adds the column-sum partials when a bias gradient is
 * asked for.
 */
size_t lbk_swiglu_bwd_bias_workspace_bytes(int64_t N, int32_t d_model, const lbk_bell* gate,
                                           const lbk_bell* up, const lbk_bell* down);
int lbk_swiglu_bwd_bias_bf16(const uint16_t* grad_out, const uint16_t* x, const uint16_t* gate_pre_act,
                             const uint16_t* up_output, const uint16_t* h, int64_t N, int32_t d_model,
                             const lbk_bell* gate, const lbk_bell* up, const lbk_bell* down,
                             int add_residual, uint16_t* dx, uint16_t* d_gate_values,
                             uint16_t* d_up_values, uint16_t* d_down_values, float* d_b_gate,
                             float* d_b_up, float* d_b_down, void* workspace, size_t workspace_bytes,
                             void* stream);

/*
 * out = x / sqrt(mean(x^2) + eps) * scale, rows of length d (bf16 in/out, fp32 math).
 * Replaces rmsnorm_cuda (reference csrc/loop/persistent_core.cuh:76-92) with the
 * layer-API semantics of looped_blockell/layers/norms.py:14-15.
 */
int lbk_rmsnorm_bf16(const uint16_t* x, int64_t N, int32_t d, const float* scale, float eps,
                     uint16_t* out, void* stream);

/*
 * Backward of lbk_rmsnorm_bf16 for an output gradient dy [N, d] (bf16):
 *   dx     [N, d] bf16 = rs * scale * dy - x * rs^3 * mean(scale * dy * x)
 *   dscale [d] fp32    = sum over rows of dy * x * rs,   rs = 1 / sqrt(mean(x^2) + eps)
 * fp32 arithmetic; dscale is summed per 64-row group into the workspace
 * (lbk_rmsnorm_bwd_workspace_bytes) and the groups in a fixed order: deterministic.
 * The reference differentiates its Flax RMSNorm with JAX autodiff
 * (looped_blockell/layers/norms.py:8-15).
 */
size_t lbk_rmsnorm_bwd_workspace_bytes(int64_t N, int32_t d);
int lbk_rmsnorm_bwd_bf16(const uint16_t* x, const uint16_t* dy, int64_t N, int32_t d, const float* scale,
                         float eps, uint16_t* dx, float* dscale, void* workspace, size_t workspace_bytes,
                         void* stream);

/*
 * h_out = h + e-injection: decay*h + dt*e with dt = softplus(log_dt),
 * decay = exp(-dt*exp(log_A)).  Replaces diagonal_injection_cuda
 * (reference csrc/loop/persistent_core.cuh:58-73, interop/pt_model.py:923-935).
 * h_out may alias h.
 */
int lbk_diagonal_injection_bf16(const uint16_t* h, const uint16_t* e, const float* log_A,
                                const float* log_dt, int64_t N, int32_t d, uint16_t* h_out,
                                void* stream);

/*
 * Backward of lbk_diagonal_injection_bf16 for an output gradient grad_out [N, d] (bf16):
 *   dh = decay * grad_out, de = dt * grad_out            (bf16, each optional)
 *   d_log_A[c]  = -sum_n grad_out * h * decay * dt * A    (fp32, optional; A = exp(log_A))
 *   d_log_dt[c] = sum_n grad_out * (e - h * decay * A) * sigmoid(log_dt)   (fp32, optional)
 * The sums run per 64 rows, then over those partials in a fixed order (deterministic); the
 * workspace (lbk_diagonal_injection_bwd_workspace_bytes) holds the partials.  The gradients of
 * the reference's PyTorch DiagonalInjection (interop/pt_model.py:923-935) under autograd; the
 * reference's CUDA operator has no backward.
 */
size_t lbk_diagonal_injection_bwd_workspace_bytes(int64_t N, int32_t d);
int lbk_diagonal_injection_bwd_bf16(const uint16_t* grad_out, const uint16_t* h, const uint16_t* e,
                                    const float* log_A, const float* log_dt, int64_t N, int32_t d,
                                    uint16_t* dh, uint16_t* de, float* d_log_A, float* d_log_dt,
                                    void* workspace, size_t workspace_bytes, void* stream);

/*
 * Looped pre-norm FFN block with shared weights, applied L times:
 *   h <- h + SwiGLU(RMSNorm(h; norm_scale, eps))
 * h_in, h_out: [N, d_model] bf16 (may alias).  On the two-kernel path the
 * carried state stays in fp32 in the workspace and h_out is rounded to bf16
 * once at the end; the row-block path rounds the state to bf16 per iteration.
 * Replaces the MLP loop of persistent_mlp_step (reference csrc/loop/persistent_core.cu:315-335,
 * schema csrc/loop/loop_ops.cpp:52-66) and the L-fold application of the
 * core block (reference looped_blockell/looping/looped_model.py:293-350).
 */
size_t lbk_looped_workspace_bytes(int64_t N, int32_t d_model, const lbk_bell* gate,
                                  const lbk_bell* up, const lbk_bell* down);
int lbk_looped_swiglu_bf16(const uint16_t* h_in, int64_t N, int32_t d_model,
                           const float* norm_scale, float eps, int32_t L,
                           const lbk_bell* gate, const lbk_bell* up, const lbk_bell* down,
                           uint16_t* h_out, void* workspace, size_t workspace_bytes,
                           void* stream);

/*
 * lbk_looped_swiglu_bf16 with the projections' biases (as lbk_swiglu_fwd_bias_bf16; each
 * optional): h <- h + (W_down(silu(W_gate n + b_gate) * (W_up n + b_up)) + b_down),
 * n = RMSNorm(h).  The looped block of the reference's MLPBlock with its biased projections
 * (looped_blockell/layers/mlp.py:56-60, looped_blockell/layers/transformer_block.py:83-84).
 */
int lbk_looped_swiglu_bias_bf16(const uint16_t* h_in, int64_t N, int32_t d_model,
                                const float* norm_scale, float eps, int32_t L,
                                const lbk_bell* gate, const lbk_bell* up, const lbk_bell* down,
                                const float* b_gate, const float* b_up, const float* b_down,
                                uint16_t* h_out, void* workspace, size_t workspace_bytes,
                                void* stream);

/*
 * lbk_looped_swiglu_bf16 as separate launches per iteration: the weight packing and an fp32
 * copy of h_in once, then a gate/up launch (RMSNorm of the state in its prologue) and a down
 * launch (state += product) per iteration, or, for shapes outside the two-kernel path, RMSNorm
 * and the row-block kernels per iteration with the state rounded to bf16 each time.  Same
 * workspace.  lbk_looped_swiglu_bf16 takes this path: it is faster than the persistent launch
 * (lbk_looped_swiglu_persistent_bf16) at every token count measured, by 6x at 64 tokens, where
 * the gate/up and down kernels split the weight rows over many workgroups and the persistent
 * launch has one workgroup per 64 tokens.
 */
int lbk_looped_swiglu_launches_bf16(const uint16_t* h_in, int64_t N, int32_t d_model,
                                    const float* norm_scale, float eps, int32_t L,
                                    const lbk_bell* gate, const lbk_bell* up, const lbk_bell* down,
                                    uint16_t* h_out, void* workspace, size_t workspace_bytes,
                                    void* stream);

/*
 * The looped block of lbk_looped_swiglu_bf16 in one persistent launch (after the weight
 * packing): workgroup b owns token block b (64 tokens) for all L iterations, so nothing is
 * exchanged between workgroups and no grid-wide barrier is needed.  Per iteration it runs
 * the gate/up tiles on an LDS panel of its RMS-normalised fp32 state rows (h of its tokens
 * to the workspace), then the down tiles with h staged back through LDS; the down phase adds
 * the result to the state and, when one workgroup covers every down row (d_model / B <= 32),
 * writes the next iteration's normalised panel itself, so the gate/up phase reads the state
 * only in the first iteration.  Same workspace (lbk_looped_workspace_bytes); the same tiles
 * in the same order as lbk_looped_swiglu_launches_bf16 (results agree to bf16 rounding: the
 * sums of squares of the norm are taken in another order).
 * Takes B in {16, 32}, d_model a multiple of 128 and at most 1024, gate and up with the same
 * K, K_down <= 63 and a 16-byte aligned norm_scale; LBK_ERR_SHAPE otherwise.
 * Replaces the persistent core loop of the reference's design notes
 * (Ai-notes/05-02-2026/CUDA-Kernel-Spec/spec.md:184-243: "persistent_core_loop", MLP path
 * only) over the host loop of persistent_mlp_step (csrc/loop/persistent_core.cu:315-335).
 */
int lbk_looped_swiglu_persistent_bf16(const uint16_t* h_in, int64_t N, int32_t d_model,
                                      const float* norm_scale, float eps, int32_t L,
                                      const lbk_bell* gate, const lbk_bell* up, const lbk_bell* down,
                                      uint16_t* h_out, void* workspace, size_t workspace_bytes,
                                      void* stream);

/*
 * The looped application of the FFN core (reference looped_blockell/looping/looped_model.py:293-340,
 * the scan body, and interop/pt_model.py:1441-1509, the PyTorch loop, on their FFN path;
 * csrc/loop/loop_ops.cpp:52-66 persistent_mlp_step is one iteration of it without the freeze).
 * For t = 0 .. L-1, per token row n:
 *   h_agg = h
 *   h_new = decay * h_agg + dt * e           (diagonal injection, per feature; skipped if e is NULL)
 *   for each core block c in order:          h_new = h_new + SwiGLU_c(RMSNorm_c(h_new))
 *   h = (t < depth(n)) ? h_new : h_agg        (depth(n) = depths[n / seq_len]; all L if depths is NULL)
 * with dt = softplus(log_dt), decay = exp(-dt * exp(log_A)) (as lbk_diagonal_injection_bf16),
 * RMSNorm_c with blocks[c].norm_scale and eps, SwiGLU_c as lbk_swiglu_fwd_bias_bf16 with the
 * block's weights and optional biases.  The state is carried in fp32 between blocks and
 * iterations; h_out = bf16(h).  h_in, e, h_out are [N, d_model] bf16 (h_out may alias h_in);
 * log_A, log_dt [d_model] fp32 (required with e); depths int32, one entry per run of seq_len
 * consecutive rows (the reference's per-sequence depths over [batch, seq]).  1 <= n_core <=
 * LBK_MAX_CORE_BLOCKS; every block maps d_model -> d_ff -> d_model.
 * The two-kernel path (every block within its shapes) runs a gate/up launch (RMSNorm of the
 * state in its prologue; token blocks whose rows are all past their depth are skipped) and a
 * down launch (state update with the depth mask; the last block also applies the next
 * iteration's injection) per block and iteration; other shapes run the decode or row-block
 * kernels and an elementwise state update.  Workspace: lbk_looped_core_workspace_bytes.
 */
#define LBK_MAX_CORE_BLOCKS 8
typedef struct lbk_core_block {
    const float* norm_scale;     /* [d_model] RMSNorm scale (16-byte aligned) */
    lbk_bell gate, up, down;     /* gate, up [d_ff / B, K, B, B]; down [d_model / B, K_d, B, B] */
    const float* b_gate;         /* [d_ff] or NULL */
    const float* b_up;           /* [d_ff] or NULL */
    const float* b_down;         /* [d_model] or NULL */
} lbk_core_block;
size_t lbk_looped_core_workspace_bytes(int64_t N, int32_t d_model, int32_t n_core, const lbk_core_block* blocks);
int lbk_looped_core_bf16(const uint16_t* h_in, const uint16_t* e, const float* log_A, const float* log_dt,
                         int64_t N, int32_t d_model, int32_t n_core, const lbk_core_block* blocks, float eps,
                         int32_t L, const int32_t* depths, int64_t seq_len, uint16_t* h_out,
                         void* workspace, size_t workspace_bytes, void* stream);

/*
 * lbk_looped_core_bf16 in one persistent launch (the reference design's K5 persistent_core_loop,
 * Ai-notes/05-02-2026/CUDA-Kernel-Spec/spec.md:184-243, MLP path: injection, n_core blocks, the
 * active-mask where, all L iterations): each workgroup owns 64 tokens for the whole loop, runs
 * only as many iterations as its deepest row and keeps the state of rows past their depth.
 * Same results as lbk_looped_core_bf16 up to the rounding of the fused normalisation.  Takes the
 * shapes of lbk_looped_swiglu_persistent_bf16 for every block, all blocks with the same tile size
 * and either all or none sharing the gate/up column buffer; LBK_ERR_SHAPE otherwise.  Same
 * workspace.
 */
int lbk_looped_core_persistent_bf16(const uint16_t* h_in, const uint16_t* e, const float* log_A,
                                    const float* log_dt, int64_t N, int32_t d_model, int32_t n_core,
                                    const lbk_core_block* blocks, float eps, int32_t L, const int32_t* depths,
                                    int64_t seq_len, uint16_t* h_out, void* workspace, size_t workspace_bytes,
                                    void* stream);

/*
 * Per-token absmax int8 quantisation of bf16 activations:
 *   absmax = max(max|x|, 1e-8); q = clamp(rint(x * (128/absmax)), -128, 127);
 *   sx = absmax / 128 (the dequantisation multiplier).
 * Restates activation_quantize (reference bonsai-test/bitlinear.py:58-69) in
 * integer form.  x row stride ldx elements; xq contiguous [N, F].
 */
int lbk_quantize_act_int8(const uint16_t* x, int64_t N, int32_t F, int64_t ldx, int8_t* xq,
                          float* sx, void* stream);

/*
 * Pack ternary tiles t[R, K, B, B] int8 in {-1,0,+1} ([B_in, B_out]) into the
 * 2-bit format of lbk_bell_ternary.packed.  Device to device.
 */
int lbk_pack_ternary(const int8_t* t, int32_t R, int32_t K, int32_t B, uint32_t* packed,
                     void* stream);

/*
 * Per-block absmean ternary quantisation of latent weights values[R,K,B,B]
 * (bf16): s = max(mean|w|, 1e-8), t = clamp(rint(w/s), -1, 1), written packed.
 * Restates ternary_quantize (reference bonsai-test/bitlinear.py:34-55) with
 * the group = one B x B block.
 */
int lbk_ternary_quantize_weights_bf16(const uint16_t* values, int32_t R, int32_t K, int32_t B,
                                      uint32_t* packed, float* scales, void* stream);

/*
 * Ternary Block-ELL product: y[n, r*B+j] ~= sx[n] * sum_k s[r,k] * P[n,r,k,j],
 * P = int32 block partial of xq against the ternary tile.  y bf16 [N, R*B].
 * The block scales are applied in per-row fixed point: m[r,k] = rint(s[r,k] * 2^e_r)
 * with e_r the largest exponent keeping |sum_k m * P| inside int32 for any int8
 * input (m at most 2^16 - 1), then y = f32(f32(sum_k m * P) * 2^-e_r) * sx
 * (within 2^-12 of exact fp32 scaling).
 * If partials != NULL the kernel also stores every P as int32 [N, R, K, B]
 * (dead slots store 0) — the exact integer accumulators before scaling.
 */
int lbk_ternary_matmul(const int8_t* xq, const float* sx, int64_t N, int32_t in_features,
                       const lbk_bell_ternary* w, uint16_t* y, int32_t* partials, void* stream);

/*
 * Ternary SwiGLU FFN on int8 activations (xq, sx from lbk_quantize_act_int8):
 *   g, u = ternary gate/up products; h = silu(g) * u (stored bf16);
 *   (hq, sh) = per-token int8 re-quantisation of h over d_ff;
 *   out = ternary down product of (hq, sh)  (+ x_resid if not NULL), bf16.
 * Optional outputs: h_out [N, d_ff] bf16, hq_out [N, d_ff] int8, sh_out [N] fp32.
 * Block scales use the fixed point of lbk_ternary_matmul.  The workspace
 * (lbk_ternary_swiglu_workspace_bytes, whose operands are those of the call)
 * holds the prepared weights for the B = 64 kernels, and h / hq / sh where the
 * optional outputs are not given; it may be NULL only when the size is 0.
 */
size_t lbk_ternary_swiglu_workspace_bytes(int64_t N, int32_t d_model, const lbk_bell_ternary* gate,
                                          const lbk_bell_ternary* up, const lbk_bell_ternary* down);
int lbk_swiglu_fwd_ternary(const int8_t* xq, const float* sx, int64_t N, int32_t d_model,
                           const lbk_bell_ternary* gate, const lbk_bell_ternary* up,
                           const lbk_bell_ternary* down, const uint16_t* x_resid,
                           uint16_t* out, uint16_t* h_out, int8_t* hq_out, float* sh_out,
                           void* workspace, size_t workspace_bytes, void* stream);

/* Optional exports of the ternary SwiGLU's accumulators before scaling (each pointer may be
 * NULL; all 16-byte aligned, row-major, row stride = the feature count):
 *   acc_gate, acc_up [N, d_ff] int32: sum_k m[r,k] * P[n,r,k,j] of the gate / up products
 *   acc_down         [N, d_model] int32: the same sum of the down product (over hq)
 *   gate_pre, up_pre [N, d_ff] fp32: f32(f32(acc) * 2^-e[r]) * sx[n], the pre-activations
 *                    that enter silu(g) * u
 * P is the exact int32 block partial of lbk_ternary_matmul and m, e its fixed point. */
typedef struct lbk_ternary_acc {
    int32_t* acc_gate;
    int32_t* acc_up;
    int32_t* acc_down;
    float* gate_pre;
    float* up_pre;
} lbk_ternary_acc;

/*
 * lbk_swiglu_fwd_ternary with the accumulator exports of *acc (acc may be NULL, which is
 * lbk_swiglu_fwd_ternary itself).  The same kernels run: the exports are extra stores in the
 * epilogues.  Replaces the int32 accumulate-then-scale contract of BitLinear (reference
 * bonsai-test/bitlinear.py:34-69, :132-138) with the group = one B x B block.
 */
int lbk_swiglu_fwd_ternary_acc(const int8_t* xq, const float* sx, int64_t N, int32_t d_model,
                               const lbk_bell_ternary* gate, const lbk_bell_ternary* up,
                               const lbk_bell_ternary* down, const uint16_t* x_resid,
                               uint16_t* out, uint16_t* h_out, int8_t* hq_out, float* sh_out,
                               const lbk_ternary_acc* acc, void* workspace, size_t workspace_bytes,
                               void* stream);

/*
 * Ternary weights prepared once.  The B = 64 two-kernel ternary path re-encodes the packed
 * tiles per call (fragment-major words in the t + 1 encoding, the per-row fixed-point scales);
 * a caller whose weights stay fixed builds them once with lbk_ternary_prepare into a buffer of
 * lbk_ternary_prepared_bytes and passes it to lbk_swiglu_fwd_ternary_prepared (same kernels,
 * same results as lbk_swiglu_fwd_ternary_acc; acc may be NULL; the workspace then holds only
 * the h maxima and h: lbk_ternary_prepared_workspace_bytes).  The buffer reflects packed,
 * scales and col_idx at the time of the call: prepare again after any of them changes.
 * lbk_ternary_prepared_bytes returns 0 for geometries without a prepared form (the prepare is a
 * no-op and the forward ignores the buffer).  No counterpart in the reference, which has no
 * ternary Block-ELL kernel (bonsai-test/bitlinear.py:132-138 dequantises and runs F.linear).
 */
size_t lbk_ternary_prepared_bytes(int32_t d_model, const lbk_bell_ternary* gate,
                                  const lbk_bell_ternary* up, const lbk_bell_ternary* down);
int lbk_ternary_prepare(int32_t d_model, const lbk_bell_ternary* gate, const lbk_bell_ternary* up,
                        const lbk_bell_ternary* down, void* prepared, size_t prepared_bytes,
                        void* stream);
size_t lbk_ternary_prepared_workspace_bytes(int64_t N, int32_t d_model, const lbk_bell_ternary* gate,
                                            const lbk_bell_ternary* up, const lbk_bell_ternary* down);
int lbk_swiglu_fwd_ternary_prepared(const int8_t* xq, const float* sx, int64_t N, int32_t d_model,
                                    const lbk_bell_ternary* gate, const lbk_bell_ternary* up,
                                    const lbk_bell_ternary* down, const void* prepared,
                                    size_t prepared_bytes, const uint16_t* x_resid, uint16_t* out,
                                    uint16_t* h_out, int8_t* hq_out, float* sh_out,
                                    const lbk_ternary_acc* acc, void* workspace,
                                    size_t workspace_bytes, void* stream);

/*
 * Backward of the Block-ELL product y = x W^T (bias excluded): dx = grad_out W (tile [B_in, B_out]
 * of slot (r, k) sends grad_out[:, r] back to column block col[r,k]) and, per tile,
 * d_values[r,k] = x[:, col]^T grad_out[:, r] (zero for dead slots).  grad_out [N, R*B],
 * x [N, in_features] (needed only for d_values), either output may be NULL.  Deterministic
 * (fixed summation order, no atomics).  The reference differentiates block_ell_matmul with JAX
 * autodiff (looped_blockell/layers/block_ell.py:149-182, tests/test_block_ell.py:57-72).
 */
size_t lbk_block_ell_matmul_bwd_workspace_bytes(int64_t N, int32_t in_features, const lbk_bell* w);
int lbk_block_ell_matmul_bwd_bf16(const uint16_t* grad_out, const uint16_t* x, int64_t N, int32_t in_features,
                                  const lbk_bell* w, uint16_t* dx, uint16_t* d_values, void* workspace,
                                  size_t workspace_bytes, void* stream);

/* ---- prune-time topology transforms (integer and copy work; alive masks are one byte per slot,
 * nonzero = alive).  Replaces the JAX functions of looped_blockell/opt/compaction.py and
 * looped_blockell/opt/column_reorder.py on device. */

/*
 * counts[r] = alive slots of row r, max_count[0] = their maximum (device scalar).
 * The compacted K is max(1, max_count) (reference looped_blockell/opt/compaction.py:43-45).
 */
int lbk_topology_alive_counts(const uint8_t* alive, int32_t R, int32_t K, int32_t* counts,
                              int32_t* max_count, void* stream);

/*
 * Packs each row's alive slots to the front (alive first, both groups in slot order) and keeps
 * the first K_new (1 <= K_new <= K) slots: out_values [R, K_new, B, B], out_col_idx and
 * out_alive [R, K_new].  Outputs must not overlap the inputs.
 * Replaces compact_single_layer (reference looped_blockell/opt/compaction.py:31-60).
 */
int lbk_topology_compact_bf16(const uint16_t* values, const int32_t* col_idx, const uint8_t* alive,
                              int32_t R, int32_t K, int32_t B, int32_t K_new, uint16_t* out_values,
                              int32_t* out_col_idx, uint8_t* out_alive, void* stream);

/*
 * importance[c] (c < C_ff <= 16384) = alive fc1 slots whose column is c (negative columns
 * skipped, columns >= C_ff counted at C_ff - 1) + alive slots of fc2 row c.
 * Replaces compute_column_importance (reference looped_blockell/opt/column_reorder.py:33-98).
 */
int lbk_column_importance(const int32_t* fc1_col_idx, const uint8_t* fc1_alive, int32_t R1, int32_t K1,
                          const uint8_t* fc2_alive, int32_t R2, int32_t K2, int32_t C_ff,
                          float* importance, void* stream);

/*
 * perm = stable argsort(-importance) (ties in index order, NaN last), int32 [C_ff].
 * Replaces compute_permutation (reference looped_blockell/opt/column_reorder.py:103-114).
 */
int lbk_column_permutation(const float* importance, int32_t C_ff, int32_t* perm, void* stream);

/*
 * Applies a d_ff permutation (perm[new] = old): is_column_dim != 0 remaps column indices
 * through the inverse permutation (sentinels stay -1); tiles and flags are copied to
 * out_values / out_alive, or left in place when those are NULL (the reference returns them
 * unchanged).  Otherwise (R == C_ff) output row i is input row perm[i] of values, column
 * indices and flags.  Outputs must not overlap the inputs.
 * Replaces apply_permutation_to_block_ell (reference looped_blockell/opt/column_reorder.py:121-177).
 */
int lbk_apply_permutation_bf16(const uint16_t* values, const int32_t* col_idx, const uint8_t* alive,
                               int32_t R, int32_t K, int32_t B, const int32_t* perm, int32_t C_ff,
                               int32_t is_column_dim, uint16_t* out_values, int32_t* out_col_idx,
                               uint8_t* out_alive, void* stream);

/*
 * k_active[0] = ceil((largest alive column + 1) / tiles_per_macro), 0 if nothing is alive.
 * Replaces compute_k_active_macros (reference looped_blockell/opt/column_reorder.py:233-269).
 */
int lbk_k_active_macros(const int32_t* col_idx, const uint8_t* alive, int32_t R, int32_t K,
                        int32_t tiles_per_macro, int32_t* k_active, void* stream);

/*
 * dst row i = src row perm[i] for i < n_dst, rows of row_bytes bytes, any element type: the
 * d_ff row permutation of optimizer moments and other per-row state.
 * Replaces apply_permutation_to_optimizer's row gather (reference
 * looped_blockell/opt/column_reorder.py:179-236).
 */
int lbk_gather_rows(const void* src, int64_t n_src, int64_t row_bytes, const int32_t* perm, int64_t n_dst,
                    void* dst, void* stream);

/*
 * Transposed (CSC) index of a Block-ELL topology: for every column block c < C (<= 16384),
 * entries[col_ptr[c] .. col_ptr[c+1]) are the slots e = r*K + k with col_idx[e] == c in
 * ascending order; col_ptr has C + 1 entries, entries up to R*K.  Slots whose column is
 * outside [0, C) (the -1 sentinel) are left out.  The reference has no such function: it is
 * the column-major view a transposed product (the backward's dy W, x^T G) walks.
 */
int lbk_transposed_index(const int32_t* col_idx, int32_t R, int32_t K, int32_t C, int32_t* col_ptr,
                         int32_t* entries, void* stream);

/* ---- storage-format bridges (copies move bits: elem_bytes 2 = bf16, 4 = fp32) ---- */

/*
 * Dense [R*B, C*B] row-major (leading dimension ld >= C*B elements) -> Block-ELL values
 * [R, K, B_in, B_out]: values[r,k] = transpose of dense block (r, col_idx[r,k]); a zero tile
 * where the column is outside [0, C).  With col_idx[r,k] = k and K = C this is the density-1
 * checkpoint conversion.
 * Replaces _dense_to_block_ell (reference interop/convert_checkpoint.py:114-131) and the
 * gather of create_block_ell_from_dense (reference looped_blockell/layers/block_ell.py:108-111).
 */
int lbk_dense_to_block_ell(const void* dense, int64_t ld, int32_t elem_bytes, int32_t R, int32_t C,
                           int32_t B, const int32_t* col_idx, int32_t K, void* values, void* stream);

/*
 * Block-ELL -> dense [R*B, C*B] (leading dimension ld): every block (r, c) gets the transposed
 * tile of the last slot of row r whose column is c (later slots overwrite earlier ones), or
 * zeros; sentinel slots write nothing.
 * Replaces _block_ell_to_dense (reference interop/convert_checkpoint.py:134-148) and
 * block_ell_to_dense (reference looped_blockell/layers/block_ell.py:118-146).
 */
int lbk_block_ell_to_dense(const void* values, const int32_t* col_idx, int32_t R, int32_t K,
                           int32_t B, int32_t C, int32_t elem_bytes, void* dense, int64_t ld,
                           void* stream);

/*
 * Per block row, the K (1 <= K <= C <= 16384) columns whose dense blocks have the largest
 * Frobenius norm (fp32; ties to the smaller column), written in ascending order to
 * col_idx_out [R, K].  dense and its rows (ld * elem_bytes) must be 16-byte aligned.
 * Replaces the top-K selection of create_block_ell_from_dense (reference
 * looped_blockell/layers/block_ell.py:100-106).
 */
int lbk_block_ell_topk_columns(const void* dense, int64_t ld, int32_t elem_bytes, int32_t R, int32_t C,
                               int32_t B, int32_t K, int32_t* col_idx_out, void* stream);

/*
 * bad_count[0] = number of 2-bit fields holding the unused code 0b10 in n_words packed ternary
 * words (0 for a valid file).  The packed ternary format has no reference counterpart: it is
 * this library's storage format, checked when a file is loaded.
 */
int lbk_ternary_check_codes(const uint32_t* words, int64_t n_words, int32_t* bad_count, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* LBK_H */
