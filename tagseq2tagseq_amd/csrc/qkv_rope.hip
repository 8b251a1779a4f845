// Attention-module prologue: the QKV projection output split into per-head
// q, k, v rows with the rotary embedding applied to q and k, and the
// transpose of that map for the backward.
//
// The reference's attention module (tunalab FlexSelfAttention, used at
// model/modules/layer.py:16-21,33; its source is not part of the reference)
// projects x [B, T, C] to qkv, splits heads and rotates q and k before
// flex_attention.  Here one pass reads each projected row once and writes the
// [B, H, T, D] operands the attention kernels stream; torch's composition of
// the same map is a view, a chunk, four products, two sums and a cat per
// operand, each a separate HBM round trip, and again for the gradient.
//
// Rotation (half-split pairs, position p = pos0 + t, table row p):
//   y[i]       = x[i] cos[p][i] + x[i + D/2] sin[p][i]
//   y[i + D/2] = x[i + D/2] cos[p][i] - x[i] sin[p][i]        i < D/2
// computed in fp32 from the fp32 tables and rounded once to bf16.  The
// backward applies the transposed rotation (an orthogonal map, so also its
// inverse):  dx[i] = dy[i] cos - dy[i + D/2] sin,
//            dx[i + D/2] = dy[i] sin + dy[i + D/2] cos.
//
// One thread per (b, t, h, 8-pair group): it reads the group's two 16-byte
// halves of q, k and v and 32 bytes each of cos and sin (shared by the heads
// of a token, so L2-resident), and writes the same 96 bytes out.  Threads are
// ordered (b, t, h, group), so a wave reads whole projected rows.
#include "attn_kernels.h"

namespace t2t {

namespace {

constexpr int kRopeThreads = 256;

__device__ __forceinline__ void load_cs(const float* row, float (&c)[8]) {
  const float4 a = *reinterpret_cast<const float4*>(row);
  const float4 b = *reinterpret_cast<const float4*>(row + 4);
  c[0] = a.x; c[1] = a.y; c[2] = a.z; c[3] = a.w;
  c[4] = b.x; c[5] = b.y; c[6] = b.z; c[7] = b.w;
}

// (y1, y2) = (x1 c + x2 s, x2 c - x1 s) for sign = +1; the transpose
// (x1 c - x2 s, x1 s + x2 c) for sign = -1.
__device__ __forceinline__ void rotate(const bf16x8& x1, const bf16x8& x2, const float (&c)[8],
                                       const float (&s)[8], float sign, bf16x8& y1, bf16x8& y2) {
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float a = (float)x1[e], b = (float)x2[e], ss = sign * s[e];
    y1[e] = (__bf16)fmaf(a, c[e], b * ss);
    y2[e] = (__bf16)fmaf(b, c[e], -(a * ss));
  }
}

struct RopeArgs {
  const __bf16* packed;    // forward: qkv source; backward: dqkv destination
  int64_t p_sb, p_st;      // packed strides (elements); a token row is [3][H][D]
  TensorView ops[3];       // q, k, v ([B, H, T, D] views)
  const float* cos;        // [rows][D / 2]
  const float* sin;
  int B, T, H, D, pos0;
};

__global__ __launch_bounds__(kRopeThreads) void qkv_rope_fwd_kernel(RopeArgs a) {
  const int L = a.D / 16;  // 8-pair groups per head row
  const int64_t idx = (int64_t)blockIdx.x * kRopeThreads + threadIdx.x;
  const int64_t total = (int64_t)a.B * a.T * a.H * L;
  if (idx >= total) return;
  const int j = (int)(idx % L);
  int64_t r = idx / L;
  const int h = (int)(r % a.H);
  r /= a.H;
  const int t = (int)(r % a.T);
  const int b = (int)(r / a.T);
  const int half = a.D / 2;
  float c[8], s[8];
  load_cs(a.cos + (int64_t)(a.pos0 + t) * half + 8 * j, c);
  load_cs(a.sin + (int64_t)(a.pos0 + t) * half + 8 * j, s);
  const __bf16* row = a.packed + b * a.p_sb + (int64_t)t * a.p_st + (int64_t)h * a.D + 8 * j;
  const int64_t which_stride = (int64_t)a.H * a.D;
#pragma unroll
  for (int w = 0; w < 3; ++w) {
    const __bf16* src = row + w * which_stride;
    const bf16x8 x1 = *reinterpret_cast<const bf16x8*>(src);
    const bf16x8 x2 = *reinterpret_cast<const bf16x8*>(src + half);
    bf16x8 y1 = x1, y2 = x2;
    if (w < 2) rotate(x1, x2, c, s, 1.f, y1, y2);
    const TensorView& o = a.ops[w];
    __bf16* dst = static_cast<__bf16*>(o.data) + b * o.sb + h * o.sh + (int64_t)t * o.st + 8 * j;
    *reinterpret_cast<bf16x8*>(dst) = y1;
    *reinterpret_cast<bf16x8*>(dst + half) = y2;
  }
}

__global__ __launch_bounds__(kRopeThreads) void qkv_rope_bwd_kernel(RopeArgs a) {
  const int L = a.D / 16;
  const int64_t idx = (int64_t)blockIdx.x * kRopeThreads + threadIdx.x;
  const int64_t total = (int64_t)a.B * a.T * a.H * L;
  if (idx >= total) return;
  const int j = (int)(idx % L);
  int64_t r = idx / L;
  const int h = (int)(r % a.H);
  r /= a.H;
  const int t = (int)(r % a.T);
  const int b = (int)(r / a.T);
  const int half = a.D / 2;
  float c[8], s[8];
  load_cs(a.cos + (int64_t)(a.pos0 + t) * half + 8 * j, c);
  load_cs(a.sin + (int64_t)(a.pos0 + t) * half + 8 * j, s);
  __bf16* row = const_cast<__bf16*>(a.packed) + b * a.p_sb + (int64_t)t * a.p_st +
                (int64_t)h * a.D + 8 * j;
  const int64_t which_stride = (int64_t)a.H * a.D;
#pragma unroll
  for (int w = 0; w < 3; ++w) {
    const TensorView& g = a.ops[w];
    const __bf16* src =
        static_cast<const __bf16*>(g.data) + b * g.sb + h * g.sh + (int64_t)t * g.st + 8 * j;
    const bf16x8 d1 = *reinterpret_cast<const bf16x8*>(src);
    const bf16x8 d2 = *reinterpret_cast<const bf16x8*>(src + half);
    bf16x8 y1 = d1, y2 = d2;
    if (w < 2) rotate(d1, d2, c, s, -1.f, y1, y2);
    __bf16* dst = row + w * which_stride;
    *reinterpret_cast<bf16x8*>(dst) = y1;
    *reinterpret_cast<bf16x8*>(dst + half) = y2;
  }
}

hipError_t launch_rope(bool backward, const RopeArgs& a, hipStream_t stream) {
  const int64_t total = (int64_t)a.B * a.T * a.H * (a.D / 16);
  if (total == 0) return hipSuccess;
  const dim3 grid((unsigned)((total + kRopeThreads - 1) / kRopeThreads));
  if (backward)
    hipLaunchKernelGGL(qkv_rope_bwd_kernel, grid, dim3(kRopeThreads), 0, stream, a);
  else
    hipLaunchKernelGGL(qkv_rope_fwd_kernel, grid, dim3(kRopeThreads), 0, stream, a);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_qkv_rope(const __bf16* qkv, int64_t sb, int64_t st, const TensorView& q,
                           const TensorView& k, const TensorView& v, const float* cos,
                           const float* sin, int B, int T, int H, int D, int pos0,
                           hipStream_t stream) {
  RopeArgs a{qkv, sb, st, {q, k, v}, cos, sin, B, T, H, D, pos0};
  return launch_rope(false, a, stream);
}

hipError_t launch_qkv_rope_bwd(const TensorView& dq, const TensorView& dk, const TensorView& dv,
                               const float* cos, const float* sin, int B, int T, int H, int D,
                               int pos0, __bf16* dqkv, int64_t sb, int64_t st,
                               hipStream_t stream) {
  RopeArgs a{dqkv, sb, st, {dq, dk, dv}, cos, sin, B, T, H, D, pos0};
  return launch_rope(true, a, stream);
}

}  // namespace t2t
