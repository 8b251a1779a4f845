// First position at which two copies of a sequence's per-token inputs (token
// ids, doc ids, q / kv grant words) differ: the check of a generation
// key/value cache against the inputs of a new call.
//
// The cached forward for generation reuses every position whose token id and
// mask inputs are unchanged since the previous call; the reference itself
// recomputes the whole sequence per token (model/generation_loop.py:90-92 ->
// model/model.py:214-237), so this check has no counterpart there.  As torch
// ops it is a compare and a reduction per input array and a nonzero, about a
// dozen launches per token; here it is one launch: each thread checks four
// positions with every load issued before any compare, each work-group
// reduces its minimum differing position and lowers the caller's result
// (set to n beforehand) with one atomic min.
#include "attn_kernels.h"

namespace t2t {

namespace {

constexpr int kDiffThreads = 256;
constexpr int kDiffUnroll = 4;  // positions per thread, all loads issued first

__global__ __launch_bounds__(kDiffThreads) void first_diff_kernel(
    const int64_t* ta, const int64_t* tb, const int32_t* da, const int32_t* db,
    const uint64_t* qa, const uint64_t* qb, const uint64_t* ka, const uint64_t* kb, int64_t sa,
    int64_t sb, int words, int n, int32_t* out) {
  __shared__ int wave_min[kDiffThreads / 64];
  const int base = blockIdx.x * kDiffThreads * kDiffUnroll + threadIdx.x;
  bool diff[kDiffUnroll];
#pragma unroll
  for (int u = 0; u < kDiffUnroll; ++u) {
    const int i = base + u * kDiffThreads;
    diff[u] = i < n && (ta[i] != tb[i] || da[i] != db[i]);
  }
  for (int w = 0; w < words; ++w) {
#pragma unroll
    for (int u = 0; u < kDiffUnroll; ++u) {
      const int i = base + u * kDiffThreads;
      if (i < n)
        diff[u] = diff[u] || qa[w * sa + i] != qb[w * sb + i] || ka[w * sa + i] != kb[w * sb + i];
    }
  }
  int first = n;
#pragma unroll
  for (int u = kDiffUnroll - 1; u >= 0; --u)
    if (diff[u]) first = base + u * kDiffThreads;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) first = min(first, __shfl_xor(first, off, 64));
  if ((threadIdx.x & 63) == 0) wave_min[threadIdx.x >> 6] = first;
  __syncthreads();
  if (threadIdx.x == 0) {
    int v = n;
#pragma unroll
    for (int w = 0; w < kDiffThreads / 64; ++w) v = min(v, wave_min[w]);
    if (v < n) atomicMin(out, v);  // a vector atomic on the caller's int32
  }
}

}  // namespace

hipError_t launch_first_input_diff(const int64_t* ta, const int64_t* tb, const int32_t* da,
                                   const int32_t* db, const uint64_t* qa, const uint64_t* qb,
                                   const uint64_t* ka, const uint64_t* kb, int64_t sa, int64_t sb,
                                   int words, int n, int32_t* out, hipStream_t stream) {
  if (n == 0) return hipSuccess;
  const int per_wg = kDiffThreads * kDiffUnroll;
  hipLaunchKernelGGL(first_diff_kernel, dim3((unsigned)((n + per_wg - 1) / per_wg)),
                     dim3(kDiffThreads), 0, stream, ta, tb, da, db, qa, qb, ka, kb, sa, sb,
                     words, n, out);
  return hipGetLastError();
}

}  // namespace t2t
