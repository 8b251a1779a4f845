// Weight gradient of a linear map over many rows: C[m][n] = sum_k A[k][m] B[k][n]
// (dW = dY^T X for y = x W^T, with dY [K][M] and X [K][N] row-major bf16).
//
// At the configs[4] shapes (K = 16384 rows, M x N = 768 x 768 ... 4096 x 768)
// the output has only 36-192 tiles of 128 x 128, too few for 256 CUs, and the
// library products run at 0.2-0.7 PFLOP/s.  Here K is split: work-group
// (tile, s) contracts rows [s K / S, (s + 1) K / S) of one 128 x 128 output
// tile into an fp32 partial, S chosen so that about four work-groups per CU
// run, and a second launch sums the S partials of each element in a fixed
// order (deterministic, no atomics) and rounds once.
//
// Contraction: both operands are "column" operands of v_mfma_f32_32x32x16_bf16
// (the contraction runs over the rows of both tiles), read from row-major LDS
// tiles [32 rows][128 + 8] with ds_read_b64_tr_b16 pairs (lds_col8); A and B
// use the same row order within each 16-row step, so the products pair up.
// 4 waves, each a 64 x 64 quarter of the tile (2 x 2 MFMA blocks, 64 fp32
// accumulators per lane); rows arrive two steps of 32 ahead through two
// register stages and two LDS buffers, one barrier per step.
#include "attn_kernels.h"

namespace t2t {

namespace {

constexpr int kWgTile = 128;          // output tile edge
constexpr int kWgRows = 32;           // rows (K) per step
constexpr int kWgPitch = kWgTile + 8; // LDS row pitch (elements)
constexpr int kWgThreads = 256;

struct WgradArgs {
  const __bf16* a;  // [K][lda]
  const __bf16* b;  // [K][ldb]
  float* part;      // [S][M][N]
  int64_t lda, ldb;
  int M, N, K, S, kchunk;
};

__global__ __launch_bounds__(kWgThreads) void wgrad_kernel(WgradArgs p) {
  __shared__ __attribute__((aligned(16))) __bf16 sa[2][kWgRows * kWgPitch];
  __shared__ __attribute__((aligned(16))) __bf16 sb[2][kWgRows * kWgPitch];
  const int tiles_n = p.N / kWgTile;
  const int tiles = (p.M / kWgTile) * tiles_n;
  // The hardware hands work-groups to the 8 XCDs round-robin; give each XCD
  // a contiguous range of (split, tile) ids instead, so that the work-groups
  // sharing a row range of A and B (one split, neighbouring tiles) share an
  // L2.
  const int G = tiles * p.S;
  const int b = blockIdx.x;
  const int id = (G % 8 == 0) ? (b % 8) * (G / 8) + b / 8 : b;
  const int tile = id % tiles, s = id / tiles;
  const int m0 = (tile / tiles_n) * kWgTile, n0 = (tile % tiles_n) * kWgTile;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;  // this wave's quarter
  const int k_begin = s * p.kchunk;
  const int steps = p.kchunk / kWgRows;

  // thread tid moves 16 elements of row tid / 8 of each tile per step
  const int lr = tid >> 3, lc = (tid & 7) * 16;
  const __bf16* ga = p.a + (int64_t)(k_begin + lr) * p.lda + m0 + lc;
  const __bf16* gb = p.b + (int64_t)(k_begin + lr) * p.ldb + n0 + lc;
  const int64_t step_a = (int64_t)kWgRows * p.lda, step_b = (int64_t)kWgRows * p.ldb;

  // two register stages: the rows of step st + 1 are in flight while step st
  // is contracted, those of step st + 2 are requested before it
  uint4 xa0, xa1, xa2, xa3, xb0, xb1, xb2, xb3;
#define WG_LOAD(r0, r1, r2, r3, st)                                          \
  do {                                                                       \
    const uint4* qa = reinterpret_cast<const uint4*>(ga + (st) * step_a);    \
    const uint4* qb = reinterpret_cast<const uint4*>(gb + (st) * step_b);    \
    r0 = qa[0];                                                              \
    r1 = qa[1];                                                              \
    r2 = qb[0];                                                              \
    r3 = qb[1];                                                              \
  } while (0)
#define WG_STORE(r0, r1, r2, r3, buf)                                        \
  do {                                                                       \
    uint4* da = reinterpret_cast<uint4*>(&sa[buf][lr * kWgPitch + lc]);      \
    uint4* db = reinterpret_cast<uint4*>(&sb[buf][lr * kWgPitch + lc]);      \
    da[0] = r0;                                                              \
    da[1] = r1;                                                              \
    db[0] = r2;                                                              \
    db[1] = r3;                                                              \
  } while (0)
#define WG_CONTRACT(buf)                                                     \
  _Pragma("unroll") for (int h = 0; h < 2; ++h) {                            \
    const bf16x8 a0 = lds_col8<kWgTile>(sa[buf], 16 * h, wm, lane);          \
    const bf16x8 a1 = lds_col8<kWgTile>(sa[buf], 16 * h, wm + 32, lane);     \
    const bf16x8 b0 = lds_col8<kWgTile>(sb[buf], 16 * h, wn, lane);          \
    const bf16x8 b1 = lds_col8<kWgTile>(sb[buf], 16 * h, wn + 32, lane);     \
    c00 = mfma32(a0, b0, c00);                                               \
    c01 = mfma32(a0, b1, c01);                                               \
    c10 = mfma32(a1, b0, c10);                                               \
    c11 = mfma32(a1, b1, c11);                                               \
  }

  f32x16 c00 = {}, c01 = {}, c10 = {}, c11 = {};
  WG_LOAD(xa0, xa1, xa2, xa3, 0);
  WG_LOAD(xb0, xb1, xb2, xb3, 1);
  WG_STORE(xa0, xa1, xa2, xa3, 0);
  __syncthreads();
  // steps is even: step st from LDS buffer 0 (step st + 1 waiting in xb),
  // then step st + 1 from buffer 1 (step st + 2 waiting in xa)
  for (int st = 0; st < steps; st += 2) {
    if (st + 2 < steps) WG_LOAD(xa0, xa1, xa2, xa3, st + 2);
    WG_CONTRACT(0)
    WG_STORE(xb0, xb1, xb2, xb3, 1);
    __syncthreads();
    if (st + 3 < steps) WG_LOAD(xb0, xb1, xb2, xb3, st + 3);
    WG_CONTRACT(1)
    if (st + 2 < steps) WG_STORE(xa0, xa1, xa2, xa3, 0);
    __syncthreads();
  }
#undef WG_LOAD
#undef WG_STORE
#undef WG_CONTRACT
  const f32x16 acc[2][2] = {{c00, c01}, {c10, c11}};

  // C layout: lane l, entry i -> row acc_row(i, l / 32), column l % 32
  float* out = p.part + (int64_t)s * p.M * p.N;
  const int g = lane >> 5, c = lane & 31;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int m = m0 + wm + 32 * i + acc_row(e, g);
        const int n = n0 + wn + 32 * j + c;
        out[(int64_t)m * p.N + n] = acc[i][j][e];
      }
}

// out[m][n] = sum over s (in order) of part[s][m][n]; 4 elements per thread.
__global__ __launch_bounds__(kWgThreads) void wgrad_sum_kernel(const float* part, int S,
                                                               int64_t mn, void* out,
                                                               bool out_f32) {
  const int64_t i4 = ((int64_t)blockIdx.x * kWgThreads + threadIdx.x) * 4;
  if (i4 >= mn) return;
  float4 acc = *reinterpret_cast<const float4*>(part + i4);
  for (int s = 1; s < S; ++s) {
    const float4 v = *reinterpret_cast<const float4*>(part + (int64_t)s * mn + i4);
    acc.x += v.x;
    acc.y += v.y;
    acc.z += v.z;
    acc.w += v.w;
  }
  if (out_f32) {
    *reinterpret_cast<float4*>(static_cast<float*>(out) + i4) = acc;
  } else {
    bf16x4 o;
    o[0] = (__bf16)acc.x;
    o[1] = (__bf16)acc.y;
    o[2] = (__bf16)acc.z;
    o[3] = (__bf16)acc.w;
    *reinterpret_cast<bf16x4*>(static_cast<__bf16*>(out) + i4) = o;
  }
}

}  // namespace

int wgrad_splits(int M, int N, int K) {
  const int tiles = (M / kWgTile) * (N / kWgTile);
  int S = (1024 + tiles - 1) / tiles;  // about four work-groups per CU
  const int max_s = K / (8 * kWgRows);  // at least 8 steps per work-group
  if (S > max_s) S = max_s;
  if (S < 1) S = 1;
  // whole pairs of steps per work-group (K is a multiple of 2 kWgRows)
  while (S > 1 && K % (S * 2 * kWgRows) != 0) --S;
  return S;
}

hipError_t launch_wgrad(const __bf16* a, int64_t lda, const __bf16* b, int64_t ldb, float* part,
                        void* out, bool out_f32, int M, int N, int K, hipStream_t stream) {
  const int S = wgrad_splits(M, N, K);
  WgradArgs p{a, b, part, lda, ldb, M, N, K, S, K / S};
  const int tiles = (M / kWgTile) * (N / kWgTile);
  hipLaunchKernelGGL(wgrad_kernel, dim3(tiles * S), dim3(kWgThreads), 0, stream, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int64_t mn = (int64_t)M * N;
  const int64_t blocks = (mn / 4 + kWgThreads - 1) / kWgThreads;
  hipLaunchKernelGGL(wgrad_sum_kernel, dim3((unsigned)blocks), dim3(kWgThreads), 0, stream, part,
                     S, mn, out, out_f32);
  return hipGetLastError();
}

}  // namespace t2t
