// Cross-entropy rows of a linear head, loss and gradient in one pass over the
// logits: for each row r of bf16 logits x (columns 0 .. V-1 of a row of ld),
//   loss[r] = logsumexp(x) - x[t]                        (t = target[r])
//   grad[r][j] = (softmax(x)[j] - [j == t]) * scale       (bf16, j < V)
//   grad[r][j] = 0                                        (V <= j < ld)
// with rows whose target equals ignore_index giving loss 0 and a zero
// gradient.  This is the per-chunk work of the reference's FusedLinearCELoss
// (tunalab, a Liger-style fused linear cross-entropy; constructed at
// model/modules/training_module.py:127-133 and called at :209): torch's
// F.cross_entropy(logits.float(), targets, ignore_index, reduction="sum") and
// its backward, with the gradient produced in the forward so the head's
// products for dX and dW follow without recomputing the logits.
//
// One 512-thread work-group per row.  Pass 1 reads the row in 16-byte pieces
// (8 logits per lane) and keeps a running (max, sum of exp2) pair per lane in
// log2 units; the pairs are combined across the wave by shuffles and across
// the 8 waves through LDS.  Pass 2 reads the row again (an L2 / last-level
// cache hit for the most part: a row is 100 KB at V = 50257) and writes the
// gradient, which may overwrite the logits in place: every read of a row
// happens before the barrier that precedes its writes.
#include "attn_kernels.h"

namespace t2t {

namespace {

constexpr int kCeThreads = 512;
constexpr int kCeWaves = kCeThreads / 64;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

__device__ __forceinline__ uint32_t pack_bf16(float a, float b) {
  const __bf16 lo = (__bf16)a, hi = (__bf16)b;
  return (uint32_t)__builtin_bit_cast(uint16_t, lo) |
         ((uint32_t)__builtin_bit_cast(uint16_t, hi) << 16);
}

// (max, sum) pairs in log2 units: sum of exp2(v - max) over the values seen.
__device__ __forceinline__ void lse_add(float& m, float& s, float v) {
  if (v > m) {
    s = s * exp2f(m - v) + 1.f;
    m = v;
  } else {
    s += exp2f(v - m);
  }
}

__device__ __forceinline__ void lse_merge(float& m, float& s, float m2, float s2) {
  const float mm = fmaxf(m, m2);
  if (mm == -INFINITY) return;  // both empty
  s = s * exp2f(m - mm) + s2 * exp2f(m2 - mm);
  m = mm;
}

__global__ __launch_bounds__(kCeThreads) void ce_rows_kernel(
    const uint16_t* logits, uint16_t* grad, int64_t ld, int V,
    const int64_t* __restrict__ target, int64_t ignore_index, const float* __restrict__ scale,
    float* __restrict__ row_loss) {
  __shared__ float red_m[kCeWaves], red_s[kCeWaves];
  __shared__ float x_t;
  const int64_t row = blockIdx.x;
  const uint4* x = reinterpret_cast<const uint4*>(logits + row * ld);
  const int nvec = (int)(ld / 8);
  const int64_t t = target[row];
  const bool ignored = t == ignore_index;
  const bool valid = !ignored && t >= 0 && t < V;
  if (threadIdx.x == 0) x_t = valid ? __uint_as_float((uint32_t)logits[row * ld + t] << 16) : 0.f;

  float m = -INFINITY, s = 0.f;
  for (int i = threadIdx.x; i < nvec; i += kCeThreads) {
    const uint4 q = x[i];
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
    const int j0 = 8 * i;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      if (j0 + 2 * e < V) lse_add(m, s, bf16_lo(w[e]) * kLog2e);
      if (j0 + 2 * e + 1 < V) lse_add(m, s, bf16_hi(w[e]) * kLog2e);
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float m2 = __shfl_xor(m, off, 64), s2 = __shfl_xor(s, off, 64);
    lse_merge(m, s, m2, s2);
  }
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    red_m[wave] = m;
    red_s[wave] = s;
  }
  __syncthreads();  // also orders every read of the row before the writes below
  m = red_m[0];
  s = red_s[0];
#pragma unroll
  for (int w = 1; w < kCeWaves; ++w) lse_merge(m, s, red_m[w], red_s[w]);
  const float lse2 = m + __log2f(s);  // log2-sum-exp2 of x * log2 e

  if (threadIdx.x == 0) {
    float loss = 0.f;
    if (valid) loss = lse2 * kLn2 - x_t;
    else if (!ignored) loss = __builtin_nanf("");  // target outside [0, V)
    row_loss[row] = loss;
  }

  const float sc = valid ? *scale : 0.f;
  uint4* g = reinterpret_cast<uint4*>(grad + row * ld);
  for (int i = threadIdx.x; i < nvec; i += kCeThreads) {
    const uint4 q = x[i];
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
    const int j0 = 8 * i;
    uint32_t o[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int ja = j0 + 2 * e, jb = ja + 1;
      float pa = ja < V ? exp2f(bf16_lo(w[e]) * kLog2e - lse2) : 0.f;
      float pb = jb < V ? exp2f(bf16_hi(w[e]) * kLog2e - lse2) : 0.f;
      if (ja == t) pa -= 1.f;
      if (jb == t) pb -= 1.f;
      o[e] = pack_bf16(pa * sc, pb * sc);
    }
    g[i] = make_uint4(o[0], o[1], o[2], o[3]);
  }
}

}  // namespace

hipError_t launch_ce_rows(const uint16_t* logits, uint16_t* grad, int64_t rows, int V, int64_t ld,
                          const int64_t* target, int64_t ignore_index, const float* scale,
                          float* row_loss, hipStream_t stream) {
  if (rows == 0) return hipSuccess;
  hipLaunchKernelGGL(ce_rows_kernel, dim3((unsigned)rows), dim3(kCeThreads), 0, stream, logits,
                     grad, ld, V, target, ignore_index, scale, row_loss);
  return hipGetLastError();
}

}  // namespace t2t
