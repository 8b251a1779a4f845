// RMS normalisation of token rows, forward and backward, one pass each.
//
// The reference's layers normalise twice per layer and once at the head
// (RMSNorm at model/modules/layer.py:14,19 and training_module.py:122-123,
// from the absent tunalab package):  y = x / sqrt(mean(x^2) + eps) * w,
// computed in fp32 and rounded once to the row dtype.  torch composes it from
// eight elementwise / reduction kernels with fp32 temporaries; here the
// forward is one read of x and one write of y (plus 4 bytes of 1/rms per row
// kept for the backward), and the backward one read of dy and x and one write
// of dx, with the weight gradient summed per work-group and reduced across
// work-groups in a second, deterministic launch (no atomics).
//
// Backward, with r = 1/rms, xh = x r, g = dy w:
//   dx = r (g - xh mean(g xh)),   dw = sum over rows of dy xh.
//
// Layout: rows of C elements (C % 8 == 0, C <= 4096) with a row stride; one
// wave per row, each lane holding VPL 16-byte vectors of the row.
#include "attn_kernels.h"

namespace t2t {

namespace {

constexpr int kNormThreads = 256;
constexpr int kNormWaves = kNormThreads / 64;
// Rows per wave in the backward (all loaded at once): fewer for long rows.
__host__ __device__ constexpr int bwd_rows_per_wave(int vpl) { return vpl <= 2 ? 4 : (vpl == 4 ? 2 : 1); }

__device__ __forceinline__ void load_w(const void* w, bool w_f32, int v, float (&out)[8]) {
  if (w_f32) {
    const float4 a = reinterpret_cast<const float4*>(w)[2 * v];
    const float4 b = reinterpret_cast<const float4*>(w)[2 * v + 1];
    out[0] = a.x; out[1] = a.y; out[2] = a.z; out[3] = a.w;
    out[4] = b.x; out[5] = b.y; out[6] = b.z; out[7] = b.w;
  } else {
    const bf16x8 x = reinterpret_cast<const bf16x8*>(w)[v];
#pragma unroll
    for (int e = 0; e < 8; ++e) out[e] = (float)x[e];
  }
}

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) x += __shfl_xor(x, off, 64);
  return x;
}

template <int VPL>
__global__ __launch_bounds__(kNormThreads) void rmsnorm_fwd_kernel(
    const __bf16* x, int64_t xs, const void* w, bool w_f32, __bf16* y, int64_t ys, float* rstd,
    int N, int C, float eps) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * kNormWaves + (threadIdx.x >> 6);
  if (row >= N) return;
  const int nv = C / 8;
  const __bf16* xr = x + (int64_t)row * xs;
  bf16x8 xv[VPL];
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < VPL; ++k) {
    const int v = lane + 64 * k;
    xv[k] = v < nv ? reinterpret_cast<const bf16x8*>(xr)[v] : bf16x8{};
#pragma unroll
    for (int e = 0; e < 8; ++e) ss = fmaf((float)xv[k][e], (float)xv[k][e], ss);
  }
  ss = wave_sum(ss);
  const float r = rsqrtf(ss / (float)C + eps);
  __bf16* yr = y + (int64_t)row * ys;
#pragma unroll
  for (int k = 0; k < VPL; ++k) {
    const int v = lane + 64 * k;
    if (v < nv) {
      float wv[8];
      load_w(w, w_f32, v, wv);
      bf16x8 o;
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = (__bf16)((float)xv[k][e] * r * wv[e]);
      reinterpret_cast<bf16x8*>(yr)[v] = o;
    }
  }
  if (lane == 0) rstd[row] = r;
}

// dx per row; the work-group's dw partial (sum over its rows of dy xh) goes to
// part[blockIdx.x][C].  A wave takes bwd_rows_per_wave(VPL) rows and issues all their
// loads before the first use, so a row costs a fraction of a memory latency.
template <int VPL>
__global__ __launch_bounds__(kNormThreads) void rmsnorm_bwd_kernel(
    const __bf16* dy, int64_t dys, const __bf16* x, int64_t xs, const void* w, bool w_f32,
    const float* rstd, __bf16* dx, int64_t dxs, float* part, int N, int C) {
  constexpr int RW = bwd_rows_per_wave(VPL);
  __shared__ float red[kNormWaves][VPL * 64 * 8];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nv = C / 8;
  float wv[VPL][8], dwp[VPL][8];
#pragma unroll
  for (int k = 0; k < VPL; ++k) {
    const int v = lane + 64 * k;
    if (v < nv) {
      load_w(w, w_f32, v, wv[k]);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) wv[k][e] = 0.f;
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) dwp[k][e] = 0.f;
  }
  const int row0 = (blockIdx.x * kNormWaves + wave) * RW;
  bf16x8 xv[RW][VPL], gv[RW][VPL];
  float r[RW];
#pragma unroll
  for (int i = 0; i < RW; ++i) {
    const int row = row0 + i;
    const bool ok = row < N;
    r[i] = ok ? rstd[row] : 0.f;
#pragma unroll
    for (int k = 0; k < VPL; ++k) {
      const int v = lane + 64 * k;
      const bool in = ok && v < nv;
      xv[i][k] = in ? reinterpret_cast<const bf16x8*>(x + (int64_t)row * xs)[v] : bf16x8{};
      gv[i][k] = in ? reinterpret_cast<const bf16x8*>(dy + (int64_t)row * dys)[v] : bf16x8{};
    }
  }
#pragma unroll
  for (int i = 0; i < RW; ++i) {
    const int row = row0 + i;
    float dot = 0.f;
#pragma unroll
    for (int k = 0; k < VPL; ++k) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float xh = (float)xv[i][k][e] * r[i];
        const float g = (float)gv[i][k][e];
        dot = fmaf(g * wv[k][e], xh, dot);
        dwp[k][e] = fmaf(g, xh, dwp[k][e]);
      }
    }
    const float c = wave_sum(dot) / (float)C;
    if (row < N) {
#pragma unroll
      for (int k = 0; k < VPL; ++k) {
        const int v = lane + 64 * k;
        if (v < nv) {
          bf16x8 o;
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float xh = (float)xv[i][k][e] * r[i];
            o[e] = (__bf16)(r[i] * ((float)gv[i][k][e] * wv[k][e] - xh * c));
          }
          reinterpret_cast<bf16x8*>(dx + (int64_t)row * dxs)[v] = o;
        }
      }
    }
  }
#pragma unroll
  for (int k = 0; k < VPL; ++k)
#pragma unroll
    for (int e = 0; e < 8; ++e) red[wave][(lane + 64 * k) * 8 + e] = dwp[k][e];
  __syncthreads();
  for (int col = threadIdx.x; col < C; col += kNormThreads) {
    float sacc = 0.f;
#pragma unroll
    for (int wv2 = 0; wv2 < kNormWaves; ++wv2) sacc += red[wv2][col];
    part[(size_t)blockIdx.x * C + col] = sacc;
  }
}

// dw[c] = sum over work-groups of part[.][c] in a fixed order: 16 waves per
// 64 columns, wave s summing groups s, s + 16, ... (eight loads in flight per
// lane), then the 16 wave sums in order through LDS.
constexpr int kDwWaves = 16;
__global__ __launch_bounds__(64 * kDwWaves) void rmsnorm_dw_kernel(const float* part, int nwg,
                                                                   int C, void* dw, bool w_f32) {
  __shared__ float red[kDwWaves][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int col = blockIdx.x * 64 + lane;
  float sacc = 0.f;
  if (col < C) {
#pragma unroll 8
    for (int g = wave; g < nwg; g += kDwWaves) sacc += part[(size_t)g * C + col];
  }
  red[wave][lane] = sacc;
  __syncthreads();
  if (wave == 0 && col < C) {
    float tot = 0.f;
#pragma unroll
    for (int s2 = 0; s2 < kDwWaves; ++s2) tot += red[s2][lane];
    if (w_f32)
      static_cast<float*>(dw)[col] = tot;
    else
      static_cast<__bf16*>(dw)[col] = (__bf16)tot;
  }
}

}  // namespace

// Vectors per lane of a C-element row, rounded up to the kernels' 1, 2, 4, 8.
static int vpl_class(int C) {
  const int v = (C / 8 + 63) / 64;
  return v <= 1 ? 1 : v <= 2 ? 2 : v <= 4 ? 4 : 8;
}

int rmsnorm_bwd_groups(int N, int C) {
  const int rows = kNormWaves * bwd_rows_per_wave(vpl_class(C));
  return (N + rows - 1) / rows;
}

hipError_t launch_rmsnorm_fwd(const __bf16* x, int64_t xs, const void* w, bool w_f32, __bf16* y,
                              int64_t ys, float* rstd, int N, int C, float eps,
                              hipStream_t stream) {
  if (N == 0) return hipSuccess;
  const dim3 grid((unsigned)((N + kNormWaves - 1) / kNormWaves));
  const int vpl = vpl_class(C);
  if (vpl <= 1)
    hipLaunchKernelGGL(rmsnorm_fwd_kernel<1>, grid, dim3(kNormThreads), 0, stream, x, xs, w,
                       w_f32, y, ys, rstd, N, C, eps);
  else if (vpl <= 2)
    hipLaunchKernelGGL(rmsnorm_fwd_kernel<2>, grid, dim3(kNormThreads), 0, stream, x, xs, w,
                       w_f32, y, ys, rstd, N, C, eps);
  else if (vpl <= 4)
    hipLaunchKernelGGL(rmsnorm_fwd_kernel<4>, grid, dim3(kNormThreads), 0, stream, x, xs, w,
                       w_f32, y, ys, rstd, N, C, eps);
  else
    hipLaunchKernelGGL(rmsnorm_fwd_kernel<8>, grid, dim3(kNormThreads), 0, stream, x, xs, w,
                       w_f32, y, ys, rstd, N, C, eps);
  return hipGetLastError();
}

hipError_t launch_rmsnorm_bwd(const __bf16* dy, int64_t dys, const __bf16* x, int64_t xs,
                              const void* w, bool w_f32, const float* rstd, __bf16* dx,
                              int64_t dxs, void* dw, float* part, int N, int C,
                              hipStream_t stream) {
  if (N == 0) return hipSuccess;
  const int nwg = rmsnorm_bwd_groups(N, C);
  const int vpl = vpl_class(C);
  const dim3 grid((unsigned)nwg);
  if (vpl <= 1)
    hipLaunchKernelGGL(rmsnorm_bwd_kernel<1>, grid, dim3(kNormThreads), 0, stream, dy, dys, x,
                       xs, w, w_f32, rstd, dx, dxs, part, N, C);
  else if (vpl <= 2)
    hipLaunchKernelGGL(rmsnorm_bwd_kernel<2>, grid, dim3(kNormThreads), 0, stream, dy, dys, x,
                       xs, w, w_f32, rstd, dx, dxs, part, N, C);
  else if (vpl <= 4)
    hipLaunchKernelGGL(rmsnorm_bwd_kernel<4>, grid, dim3(kNormThreads), 0, stream, dy, dys, x,
                       xs, w, w_f32, rstd, dx, dxs, part, N, C);
  else
    hipLaunchKernelGGL(rmsnorm_bwd_kernel<8>, grid, dim3(kNormThreads), 0, stream, dy, dys, x,
                       xs, w, w_f32, rstd, dx, dxs, part, N, C);
  hipLaunchKernelGGL(rmsnorm_dw_kernel, dim3((unsigned)((C + 63) / 64)), dim3(64 * kDwWaves), 0,
                     stream, part, nwg, C, dw, w_f32);
  return hipGetLastError();
}

}  // namespace t2t
