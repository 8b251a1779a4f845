// SwiGLU of the layers' MLP, forward and backward, one pass each.
//
// The reference's layers use tunalab's GLU with silu (model/modules/layer.py:
// 23-28; the package is absent, so the definition is the textbook one):
// h = silu(g) * u with [g | u] = x W_gate_up^T.  torch composes it from a
// chunk, a silu and a multiply forward and four elementwise kernels plus a
// concatenation backward, each a pass over [N, H] bf16 rows; here the
// forward reads [g | u] once and writes h, and the backward reads [g | u]
// and dh once and writes [dg | du] into one buffer (the gate / up product's
// gradient, so no concatenation), all in fp32 arithmetic with one rounding:
//   s = sigmoid(g),  h = g s u,
//   dg = dh u s (1 + g (1 - s)),  du = dh g s.
// One thread per 8 consecutive columns (16-byte loads and stores).
#include "attn_kernels.h"

namespace t2t {

namespace {

constexpr int kGluThreads = 256;

__device__ __forceinline__ float sigmoid(float x) { return 1.f / (1.f + __expf(-x)); }

__global__ __launch_bounds__(kGluThreads) void swiglu_fwd_kernel(const __bf16* gu, int64_t gs,
                                                                  __bf16* h, int64_t hs,
                                                                  int64_t n_vec, int nv, int H) {
  const int64_t i = (int64_t)blockIdx.x * kGluThreads + threadIdx.x;
  if (i >= n_vec) return;
  const int64_t row = i / nv;
  const int c = (int)(i - row * nv) * 8;
  const bf16x8 g = *reinterpret_cast<const bf16x8*>(gu + row * gs + c);
  const bf16x8 u = *reinterpret_cast<const bf16x8*>(gu + row * gs + H + c);
  bf16x8 o;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float gf = (float)g[e];
    o[e] = (__bf16)(gf * sigmoid(gf) * (float)u[e]);
  }
  *reinterpret_cast<bf16x8*>(h + row * hs + c) = o;
}

__global__ __launch_bounds__(kGluThreads) void swiglu_bwd_kernel(const __bf16* gu, int64_t gs,
                                                                  const __bf16* dh, int64_t dhs,
                                                                  __bf16* dgu, int64_t dgs,
                                                                  int64_t n_vec, int nv, int H) {
  const int64_t i = (int64_t)blockIdx.x * kGluThreads + threadIdx.x;
  if (i >= n_vec) return;
  const int64_t row = i / nv;
  const int c = (int)(i - row * nv) * 8;
  const bf16x8 g = *reinterpret_cast<const bf16x8*>(gu + row * gs + c);
  const bf16x8 u = *reinterpret_cast<const bf16x8*>(gu + row * gs + H + c);
  const bf16x8 d = *reinterpret_cast<const bf16x8*>(dh + row * dhs + c);
  bf16x8 dg, du;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float gf = (float)g[e], uf = (float)u[e], df = (float)d[e];
    const float s = sigmoid(gf);
    dg[e] = (__bf16)(df * uf * s * (1.f + gf * (1.f - s)));
    du[e] = (__bf16)(df * gf * s);
  }
  *reinterpret_cast<bf16x8*>(dgu + row * dgs + c) = dg;
  *reinterpret_cast<bf16x8*>(dgu + row * dgs + H + c) = du;
}

}  // namespace

hipError_t launch_swiglu_fwd(const __bf16* gu, int64_t gs, __bf16* h, int64_t hs, int N, int H,
                             hipStream_t stream) {
  const int nv = H / 8;
  const int64_t n_vec = (int64_t)N * nv;
  if (n_vec == 0) return hipSuccess;
  hipLaunchKernelGGL(swiglu_fwd_kernel, dim3((unsigned)((n_vec + kGluThreads - 1) / kGluThreads)),
                     dim3(kGluThreads), 0, stream, gu, gs, h, hs, n_vec, nv, H);
  return hipGetLastError();
}

hipError_t launch_swiglu_bwd(const __bf16* gu, int64_t gs, const __bf16* dh, int64_t dhs,
                             __bf16* dgu, int64_t dgs, int N, int H, hipStream_t stream) {
  const int nv = H / 8;
  const int64_t n_vec = (int64_t)N * nv;
  if (n_vec == 0) return hipSuccess;
  hipLaunchKernelGGL(swiglu_bwd_kernel, dim3((unsigned)((n_vec + kGluThreads - 1) / kGluThreads)),
                     dim3(kGluThreads), 0, stream, gu, gs, dh, dhs, dgu, dgs, n_vec, nv, H);
  return hipGetLastError();
}

}  // namespace t2t
