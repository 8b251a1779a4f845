// Shader-clock probe for the roofline's peak.
//
// The published bf16 peak assumes the 2.4 GHz peak engine clock; under a
// sustained matrix-core load the clock settles lower, by an amount that
// differs from box to box.  This kernel fills every SIMD with two waves of
// back-to-back v_mfma_f32_32x32x16_bf16 chains (the attention kernels' MFMA)
// and has wave 0 of work-group 0 read the shader-cycle counter (s_memtime)
// and the constant-rate wall-clock counter (s_memrealtime) around its own
// loop; cycles / wall ticks x the wall-clock rate is the engine clock under
// that load.
#include "attn_kernels.h"

namespace t2t {

namespace {

constexpr int kProbeThreads = 256;

__global__ __launch_bounds__(kProbeThreads, 2) void clock_probe_kernel(uint64_t* out, int iters,
                                                                      float seed) {
  const int lane = threadIdx.x & 63;
  bf16x8 a, b;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    a[j] = (__bf16)(seed * (float)(lane + j));
    b[j] = (__bf16)(seed * (float)(lane - j));
  }
  f32x16 acc[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) acc[c] = f32x16{};
  // wave 0 of work-group 0 (a wave-uniform condition)
  const bool rec = blockIdx.x == 0 && threadIdx.x < 64;
  uint64_t t0 = 0, w0 = 0;
  if (rec) {
    t0 = __builtin_amdgcn_s_memtime();
    w0 = __builtin_amdgcn_s_memrealtime();
  }
  for (int i = 0; i < iters; ++i) {
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[c] = mfma32(a, b, acc[c]);
  }
  // The sum reads every chain's result, so the chains have retired before
  // the second reading; its store keeps them live (never taken: the
  // products of these inputs are far from 1e30).
  float s = 0.f;
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int i = 0; i < 16; ++i) s += acc[c][i];
  if (s == 1.0e30f) out[1] = 0;
  if (rec) {
    const uint64_t t1 = __builtin_amdgcn_s_memtime();
    const uint64_t w1 = __builtin_amdgcn_s_memrealtime();
    if (lane == 0) {
      out[0] = t1 - t0;
      out[1] = w1 - w0;
    }
  }
}

}  // namespace

hipError_t launch_clock_probe(uint64_t* out, int iters, hipStream_t stream) {
  int dev = 0, cus = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  if (e != hipSuccess) return e;
  // two 4-wave work-groups per CU: two waves per SIMD
  hipLaunchKernelGGL(clock_probe_kernel, dim3(2 * cus), dim3(kProbeThreads), 0, stream, out,
                     iters, 1.0e-3f);
  return hipGetLastError();
}

hipError_t wall_clock_khz(int* khz) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  return hipDeviceGetAttribute(khz, hipDeviceAttributeWallClockRate, dev);
}

}  // namespace t2t
