// Linear maps of a few token rows with the neighbouring element-wise work
// fused in: the per-layer matrix-vector products of a generation step.
//
// Each layer of the reference (model/modules/layer.py:32-35) applies four
// nn.Linear weights to its rows: the attention module's qkv projection and
// out-projection, and the GLU's gate_up and down (tunalab FlexSelfAttention
// and GLU, which the reference imports).  When a generation step feeds one
// to eight new rows, each product is one read of the weight matrix (2 N K
// bytes for N K weights), so the step is HBM- and latency-bound; a GEMM
// library launch at these shapes takes several times the weight traffic,
// and the RMSNorm before it and the residual add or SwiGLU after it are
// further launches with their own round trips.  Here one launch does
//
//   [RMSNorm of the input rows] -> W x -> store | residual add | SwiGLU
//                                        | rotary embedding + q / cache rows
//
// with the rounding points of the unfused sequence: the normalised rows
// rounded to bf16 as t2t_rms_norm writes them (x r w), every product rounded
// to bf16 before the residual add, the activation or the rotation, silu(g)
// = g / (1 + e^-g) rounded before its product with u, the rotation computed
// in fp32 from the fp32 tables as t2t_qkv_rope does.  Sums over K are fp32
// in an order of this kernel's own, so products agree with a library GEMM's
// to bf16 rounding, not bit for bit.
//
// The residual add can take a second, weighted residual: the backbone's skip
// connection (model/modules/backbone.py:93-104) that the next layer adds to
// its input, x + w skip, folded into this layer's last product.
//
// Layout: W [rows][K] bf16, row-major (nn.Linear's weight); x [M][K],
// y [M][N], res [M][N] bf16 with row strides; K <= 4096, M <= 8.  Rows are
// read in 16-byte vectors when K, the x row stride and the pointers allow it,
// else element by element (e.g. the GLU hidden width int(8/3 C) = 1365 for
// C = 512), with the chunk past K read as zero.
// A work-group is four waves.  Each wave takes R output units (an output
// column; for SwiGLU the (gate, up) row pair; for the qkv mode the rotation
// pair (i, i + D/2) of one head's q, k or v rows) and issues every 16-byte
// load of its weight rows before anything else (lane l holds the 8-element
// chunks l, l + 64, ...); the work-group then writes its (normalised) input
// rows to LDS as bf16 (M K 2 bytes), and each wave multiplies, sums over
// lanes with xor shuffles, and lane m writes row m's outputs.
#include "attn_kernels.h"

namespace t2t {

namespace {

constexpr int kLinThreads = 256;
constexpr int kLinWaves = kLinThreads / 64;

struct RowsArgs {
  const __bf16* x;
  int64_t xs;
  const __bf16* w;
  const void* norm_w;  // RMSNorm weight of the input rows, or NULL
  int norm_f32;
  float eps;
  const __bf16* res;   // residual rows (kRowsAdd)
  int64_t rs;
  const __bf16* skip;  // kRowsAdd: second residual rows, or NULL for the sum itself
  int64_t ss;
  const void* skip_w;  // kRowsAdd: scalar weight of the second residual, or NULL for none
  int skip_w_f32;
  __bf16* y;           // output rows (all modes but kRowsQkvRope)
  int64_t ys;
  int M, K, N;         // N: output columns; SwiGLU: hidden width; qkv: H D
  int aligned;         // K, the row strides and pointers allow 16-byte row loads
  // kRowsQkvRope: q rows [H][M][D] (the views' t axis), k / v cache rows at
  // the rows' positions, cos / sin tables [table_rows][D / 2].
  const float* cos;
  const float* sin;
  const int64_t* pos;  // per-row positions, or NULL for pos0 + m
  int pos0, H, D, max_pos;
  TensorView q, k, v;
};

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) x += __shfl_xor(x, off, 64);
  return x;
}

// Elements 8c .. 8c + 7 of a row of K, zero past K: one 16-byte load when the
// rows are 16-byte aligned, else element loads.
__device__ __forceinline__ bf16x8 load8(const __bf16* row, int c, int K, int aligned) {
  if (aligned) return reinterpret_cast<const bf16x8*>(row)[c];
  bf16x8 v;
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = 8 * c + e < K ? row[8 * c + e] : (__bf16)0.f;
  return v;
}

__device__ __forceinline__ void norm_weight8(const void* w, int f32, int v, float (&out)[8],
                                             int K, int aligned) {
  if (!aligned) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int i = 8 * v + e;
      out[e] = i >= K ? 0.f
                      : (f32 ? static_cast<const float*>(w)[i]
                             : (float)static_cast<const __bf16*>(w)[i]);
    }
    return;
  }
  if (f32) {
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

__device__ __forceinline__ float bf(float x) { return (float)(__bf16)x; }

// Weight rows per unit and units per wave: about four 16-byte loads per lane
// in flight before the first use.
template <int MODE>
__host__ __device__ constexpr int rows_per_unit() { return MODE >= kRowsSwiglu ? 2 : 1; }
template <int KV, int MODE>
__host__ __device__ constexpr int units_per_wave() {
  return rows_per_unit<MODE>() * KV >= 4 ? 1 : 4 / (rows_per_unit<MODE>() * KV);
}

__host__ __device__ inline int unit_count(int mode, int N) {
  return mode == kRowsQkvRope ? 3 * N / 2 : N;
}

template <int MODE>
__device__ __forceinline__ int weight_row(const RowsArgs& a, int u, int s) {
  if (MODE == kRowsSwiglu) return u + s * a.N;
  if (MODE == kRowsQkvRope) {
    const int half = a.D >> 1;
    return (u / half) * a.D + u % half + s * half;
  }
  return u;
}

template <int KV, int MT, int MODE>
__global__ __launch_bounds__(kLinThreads) void rows_linear_kernel(RowsArgs a) {
  constexpr int P = rows_per_unit<MODE>();
  constexpr int R = units_per_wave<KV, MODE>();
  constexpr int NW = P * R;
  extern __shared__ bf16x8 xl[];  // [MT][K / 8]
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nv = (a.K + 7) >> 3;
  const int nunits = unit_count(MODE, a.N);
  const int u0 = (blockIdx.x * kLinWaves + wave) * R;

  // 1. The wave's weight rows, every load issued before any other work.
  bf16x8 wv[NW][KV];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int s = 0; s < P; ++s) {
      const bool ok = u0 + r < nunits;
      const __bf16* wr = a.w + (int64_t)(ok ? weight_row<MODE>(a, u0 + r, s) : 0) * a.K;
#pragma unroll
      for (int k = 0; k < KV; ++k) {
        const int c = lane + 64 * k;
        wv[r * P + s][k] = (ok && c < nv) ? load8(wr, c, a.K, a.aligned) : bf16x8{};
      }
    }

  // 2. Input rows to LDS, RMS-normalised when a norm weight is given; rows
  //    M .. MT - 1 are zero.
  for (int m = wave; m < MT; m += kLinWaves) {
    bf16x8* dst = xl + m * nv;
    if (m >= a.M) {
#pragma unroll
      for (int k = 0; k < KV; ++k)
        if (lane + 64 * k < nv) dst[lane + 64 * k] = bf16x8{};
      continue;
    }
    const __bf16* xr = a.x + (int64_t)m * a.xs;
    bf16x8 xv[KV];
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < KV; ++k) {
      const int c = lane + 64 * k;
      xv[k] = c < nv ? load8(xr, c, a.K, a.aligned) : bf16x8{};
#pragma unroll
      for (int e = 0; e < 8; ++e) ss = fmaf((float)xv[k][e], (float)xv[k][e], ss);
    }
    if (a.norm_w) {
      const float rr = rsqrtf(wave_sum(ss) / (float)a.K + a.eps);
#pragma unroll
      for (int k = 0; k < KV; ++k) {
        const int c = lane + 64 * k;
        if (c < nv) {
          float nw[8];
          norm_weight8(a.norm_w, a.norm_f32, c, nw, a.K, a.aligned);
          bf16x8 o;
#pragma unroll
          for (int e = 0; e < 8; ++e) o[e] = (__bf16)((float)xv[k][e] * rr * nw[e]);
          dst[c] = o;
        }
      }
    } else {
#pragma unroll
      for (int k = 0; k < KV; ++k)
        if (lane + 64 * k < nv) dst[lane + 64 * k] = xv[k];
    }
  }
  __syncthreads();
  if (u0 >= nunits) return;

  // 3. Partial dot products per lane, then sums over the wave.
  float acc[NW][MT];
#pragma unroll
  for (int j = 0; j < NW; ++j)
#pragma unroll
    for (int m = 0; m < MT; ++m) acc[j][m] = 0.f;
#pragma unroll
  for (int k = 0; k < KV; ++k) {
    const int c = lane + 64 * k;
    if (c < nv) {
      bf16x8 xm[MT];
#pragma unroll
      for (int m = 0; m < MT; ++m) xm[m] = xl[m * nv + c];
#pragma unroll
      for (int e = 0; e < 8; ++e)
#pragma unroll
        for (int j = 0; j < NW; ++j) {
          const float wf = (float)wv[j][k][e];
#pragma unroll
          for (int m = 0; m < MT; ++m) acc[j][m] = fmaf(wf, (float)xm[m][e], acc[j][m]);
        }
    }
  }
#pragma unroll
  for (int j = 0; j < NW; ++j)
#pragma unroll
    for (int m = 0; m < MT; ++m) acc[j][m] = wave_sum(acc[j][m]);

  // 4. Epilogue: lane m writes row m.
  const int m = lane;
  if (m >= a.M) return;
  float sel[NW];
#pragma unroll
  for (int j = 0; j < NW; ++j) {
    sel[j] = acc[j][0];
#pragma unroll
    for (int i = 1; i < MT; ++i)
      if (m == i) sel[j] = acc[j][i];
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int u = u0 + r;
    if (u >= nunits) break;
    if (MODE == kRowsStore) {
      a.y[(int64_t)m * a.ys + u] = (__bf16)sel[r];
    } else if (MODE == kRowsAdd) {
      float t = bf((float)a.res[(int64_t)m * a.rs + u] + bf(sel[r]));
      if (a.skip_w) {
        const float sw = a.skip_w_f32 ? *static_cast<const float*>(a.skip_w)
                                      : (float)*static_cast<const __bf16*>(a.skip_w);
        const float sk = a.skip ? (float)a.skip[(int64_t)m * a.ss + u] : t;
        t = bf(t + bf(sw * sk));
      }
      a.y[(int64_t)m * a.ys + u] = (__bf16)t;
    } else if (MODE == kRowsSwiglu) {
      const float g = bf(sel[2 * r]), up = bf(sel[2 * r + 1]);
      const float act = bf(g / (1.0f + expf(-g)));
      a.y[(int64_t)m * a.ys + u] = (__bf16)(act * up);
    } else {
      const int half = a.D >> 1;
      const int slot = u / half, i = u % half;
      const int which = slot / a.H, h = slot % a.H;
      const int p = a.pos ? (int)a.pos[m] : a.pos0 + m;
      if (p < 0 || p >= a.max_pos) continue;  // outside the tables / cache: not written
      float y1 = bf(sel[2 * r]), y2 = bf(sel[2 * r + 1]);
      if (which < 2) {
        const float c = a.cos[(int64_t)p * half + i], s = a.sin[(int64_t)p * half + i];
        const float x1 = y1, x2 = y2;
        y1 = fmaf(x1, c, x2 * s);
        y2 = fmaf(x2, c, -(x1 * s));
      }
      const TensorView& t = which == 0 ? a.q : (which == 1 ? a.k : a.v);
      __bf16* dst = static_cast<__bf16*>(t.data) + (int64_t)h * t.sh +
                    (int64_t)(which == 0 ? m : p) * t.st + i;
      dst[0] = (__bf16)y1;
      dst[half] = (__bf16)y2;
    }
  }
}

template <int KV, int MT, int MODE>
hipError_t launch_kmm(const RowsArgs& a, hipStream_t stream) {
  constexpr int per_wg = kLinWaves * units_per_wave<KV, MODE>();
  const int units = unit_count(MODE, a.N);
  const dim3 grid((unsigned)((units + per_wg - 1) / per_wg));
  const size_t lds = (size_t)MT * ((a.K + 7) / 8) * sizeof(bf16x8);
  hipLaunchKernelGGL((rows_linear_kernel<KV, MT, MODE>), grid, dim3(kLinThreads), lds, stream,
                     a);
  return hipGetLastError();
}

template <int KV, int MT>
hipError_t launch_km(int mode, const RowsArgs& a, hipStream_t stream) {
  switch (mode) {
    case kRowsStore: return launch_kmm<KV, MT, kRowsStore>(a, stream);
    case kRowsAdd: return launch_kmm<KV, MT, kRowsAdd>(a, stream);
    case kRowsSwiglu: return launch_kmm<KV, MT, kRowsSwiglu>(a, stream);
    default: return launch_kmm<KV, MT, kRowsQkvRope>(a, stream);
  }
}

template <int KV>
hipError_t launch_k(int mode, const RowsArgs& a, hipStream_t stream) {
  if (a.M <= 1) return launch_km<KV, 1>(mode, a, stream);
  if (a.M <= 2) return launch_km<KV, 2>(mode, a, stream);
  if (a.M <= 4) return launch_km<KV, 4>(mode, a, stream);
  return launch_km<KV, 8>(mode, a, stream);
}

hipError_t launch_rows(int mode, RowsArgs a, hipStream_t stream) {
  const int nv = (a.K + 7) / 8;
  const uintptr_t ptrs = reinterpret_cast<uintptr_t>(a.x) | reinterpret_cast<uintptr_t>(a.w) |
                         reinterpret_cast<uintptr_t>(a.norm_w);
  a.aligned = a.K % 8 == 0 && a.xs % 8 == 0 && ptrs % 16 == 0;
  if (nv <= 64) return launch_k<1>(mode, a, stream);
  if (nv <= 128) return launch_k<2>(mode, a, stream);
  if (nv <= 256) return launch_k<4>(mode, a, stream);
  return launch_k<8>(mode, a, stream);
}

}  // namespace

hipError_t launch_rows_linear(int mode, const __bf16* x, int64_t xs, int M, int K,
                              const __bf16* w, int N, const void* norm_w, bool norm_f32,
                              float eps, const __bf16* res, int64_t rs, const __bf16* skip,
                              int64_t ss, const void* skip_w, bool skip_w_f32, __bf16* y,
                              int64_t ys, hipStream_t stream) {
  RowsArgs a{};
  a.x = x; a.xs = xs; a.w = w; a.norm_w = norm_w; a.norm_f32 = norm_f32; a.eps = eps;
  a.res = res; a.rs = rs; a.skip = skip; a.ss = ss; a.skip_w = skip_w; a.skip_w_f32 = skip_w_f32;
  a.y = y; a.ys = ys; a.M = M; a.K = K; a.N = N;
  return launch_rows(mode, a, stream);
}

hipError_t launch_rows_qkv_rope(const __bf16* x, int64_t xs, int M, int K, const __bf16* w,
                                const void* norm_w, bool norm_f32, float eps, int H, int D,
                                const float* cos, const float* sin, const int64_t* pos, int pos0,
                                int max_pos, const TensorView& q, const TensorView& k,
                                const TensorView& v, hipStream_t stream) {
  RowsArgs a{};
  a.x = x; a.xs = xs; a.w = w; a.norm_w = norm_w; a.norm_f32 = norm_f32; a.eps = eps;
  a.M = M; a.K = K; a.N = H * D;
  a.cos = cos; a.sin = sin; a.pos = pos; a.pos0 = pos0; a.H = H; a.D = D; a.max_pos = max_pos;
  a.q = q; a.k = k; a.v = v;
  return launch_rows(kRowsQkvRope, a, stream);
}

}  // namespace t2t
