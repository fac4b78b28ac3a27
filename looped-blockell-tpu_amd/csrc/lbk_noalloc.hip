// lbk_noalloc.hip — the SwiGLU forward for callers that cannot allocate device memory.
//
// lbk_swiglu_fwd_bf16 takes a caller-owned workspace (the packed tiles of the two-kernel path
// and the hidden state h).  Callers inside HIP graph capture, tight serving loops or harnesses
// that forbid hipMalloc cannot provide one per call; lbk_swiglu_fwd_bf16_noalloc serves them
// from `scratch`, a fixed array in device memory (each GPU the library runs on holds its own
// copy until the process ends).  The entry point allocates nothing: it checks the size the
// geometry needs against the array and runs the same kernels as lbk_swiglu_fwd_bf16 on it.
//
// `scratch` named in host code is a host-side stand-in, not a device address: the device
// address of each GPU's copy is looked up once per device (hipGetSymbolAddress, with that
// device current) and only that address is ever handed to kernels.  Every call on one GPU
// shares that GPU's array: calls that overlap in time on one GPU (different streams, no
// ordering between them) race on it.  No part of the workspace has to start at zero: every
// byte a kernel reads from it was written earlier in the same call.
#include <atomic>
#include <mutex>

#include <hip/hip_runtime.h>

#include "lbk.h"

namespace {

static __device__ __align__(256) unsigned char scratch[LBK_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch[kMaxDevices];
std::mutex g_scratch_mu;

// device address of the current device's scratch array (looked up on its first use there)
int scratch_address(void** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return LBK_ERR_LAUNCH;
  void* p = g_scratch[dev].load(std::memory_order_acquire);
  if (!p) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch[dev].load(std::memory_order_relaxed);
    if (!p) {
      if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return LBK_ERR_LAUNCH;
      g_scratch[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return LBK_OK;
}

}  // namespace

extern "C" {

size_t lbk_noalloc_scratch_bytes(void) { return (size_t)LBK_NOALLOC_SCRATCH_BYTES; }

int lbk_noalloc_init(void) {
  void* ws = nullptr;
  return scratch_address(&ws);
}

int lbk_swiglu_fwd_bf16_noalloc(const uint16_t* x, int64_t N, int32_t d_model, const lbk_bell* gate,
                                const lbk_bell* up, const lbk_bell* down, int add_residual, uint16_t* out,
                                void* stream) {
  if (!gate || !up || !down) return LBK_ERR_NULL;
  if (N < 0) return LBK_ERR_ARG;
  if (N == 0) return lbk_swiglu_fwd_bf16(x, N, d_model, gate, up, down, add_residual, out, nullptr, nullptr,
                                         nullptr, nullptr, 0, stream);
  const size_t need = lbk_swiglu_workspace_bytes(N, d_model, gate, up, down, 0);
  if (need > (size_t)LBK_NOALLOC_SCRATCH_BYTES) return LBK_ERR_TOO_LARGE;
  void* ws = nullptr;
  int st = scratch_address(&ws);
  if (st) return st;
  return lbk_swiglu_fwd_bf16(x, N, d_model, gate, up, down, add_residual, out, nullptr, nullptr, nullptr, ws,
                             (size_t)LBK_NOALLOC_SCRATCH_BYTES, stream);
}

}  // extern "C"
