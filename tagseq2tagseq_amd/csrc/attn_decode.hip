// Masked attention of a few new query rows against a key/value cache: the
// decode step of generation.
//
// The reference regenerates every token by rebuilding the mask and running
// the full forward over the whole packed sequence
// (model/generation_loop.py:90-92 -> TS2TSModel.forward_inference,
// model/model.py:214-237) and keeps only the last position's logits.  With
// the keys and values of the unchanged prefix cached, one step needs the
// attention of the new rows only, against every cached key -- an HBM-bound
// gather: each allowed key costs its K and V rows (4 D bytes), each masked
// key only its mask inputs (4 + 8 W bytes), because the mask is evaluated per
// key before any K/V load:
//   allowed(q, j) = j <= pos(q) && (doc[j] == doc(q) ||
//                   OR_w (q_bits[w](q) & kv_bits[w][j]) != 0)
// (the doc_causal / cross_doc_link mask_mod, cross_doc_mask.py:348-357,
// block_mask_creator.py:121-129).
//
// Split-KV.  attn_decode_partial: one work-group per (256-key chunk, kv head,
// batch row) handles all R = G * Tq query rows of the kv head (G query heads
// of the GQA group x Tq new tokens, R <= 8).  A key is read by D/8 adjacent
// lanes, 16 bytes each, so a K or V row is one coalesced run; the lanes of a
// key hold the query rows' matching 8 elements in registers, and the partial
// dot products are summed across them with DPP butterflies.  Pass 1 writes the
// chunk's scores to LDS, pass 2 takes the chunk's row max, weights the V rows
// by exp2(s - max) and sums them across the key groups (DPP, then LDS across
// waves).  The kernel has two dependent memory stages: the keys' mask
// inputs with the query rows, then the K and V rows of the allowed keys.
// Each (row, chunk) leaves (max, sum, unnormalised o[D]) in the
// workspace; attn_decode_combine merges the chunks of a row into o (bf16)
// and the log2-domain LSE.  Fully masked rows give o = 0 and LSE = -inf.
#include "attn_kernels.h"

namespace t2t {

namespace {

constexpr int kDecThreads = 256;
constexpr int kDecChunk = 256;  // keys per work-group

struct DecodeArgs {
  TensorView q, k, v;  // q [B][Hq][Tq][D]; k, v [B][Hkv][cap][D]
  const int32_t* key_doc;
  const uint64_t* key_bits;  // [Bm][W][key_stride]
  int64_t key_stride;
  const int32_t* q_pos;      // [Bm][Tq]
  const int32_t* q_doc;
  const uint64_t* q_bits;    // [Bm][W][Tq]
  int Bm, W, B, Hq, Hkv, Tq, Tkv, nch;
  float c;                   // scale * log2(e)
  float* part;               // [B][Hq][Tq][nch][D + 2]
};

// Sum over the GL = D/8 lanes of a key group (8 or 16 adjacent, aligned
// lanes): DPP quad_perm [1,0,3,2] and [2,3,0,1] sum each quad, row_half_mirror
// adds the other quad of the 8-lane half row, row_mirror the other half of the
// 16-lane row.  Every lane of the group ends with the group's sum.
template <int GL>
__device__ __forceinline__ float group_sum(float x) {
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0xB1, 0xF, 0xF, false));
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x4E, 0xF, 0xF, false));
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x141, 0xF, 0xF, false));
  if constexpr (GL == 16)
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x140, 0xF, 0xF, false));
  return x;
}

// RMAX: compile-time bound on the R query rows (1, 2, 4 or 8), so the common
// single-row step holds 8 + 8 accumulators per lane rather than 64 + 64.
template <int D, int RMAX>
__global__ __launch_bounds__(kDecThreads) void attn_decode_partial(DecodeArgs a) {
  constexpr int GL = D / 8;                    // lanes per key
  constexpr int NKG = kDecThreads / GL;        // key groups per work-group
  constexpr int KPG = kDecChunk / NKG;         // keys per group
  __shared__ float sc[RMAX][kDecChunk];        // scores (log2 units)
  __shared__ float red[kDecThreads / 64][RMAX][D];
  __shared__ float rmax[RMAX];
  __shared__ int32_t qpos_s[RMAX], qdoc_s[RMAX];
  __shared__ uint64_t qbits_s[kMaxWords][RMAX];

  const int chunk = blockIdx.x, hk = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int dg = tid % GL, kg = tid / GL;
  const int G = a.Hq / a.Hkv;
  const int R = G * a.Tq;
  const int mb = a.Bm > 1 ? b : 0;
  const int j0 = chunk * kDecChunk;

  const __bf16* kbase = static_cast<const __bf16*>(a.k.data) + b * a.k.sb + hk * a.k.sh + 8 * dg;
  const __bf16* vbase = static_cast<const __bf16*>(a.v.data) + b * a.v.sb + hk * a.v.sh + 8 * dg;
  const int32_t* kdoc = a.key_doc + (size_t)mb * a.key_stride;
  const uint64_t* kbits = a.key_bits + (size_t)mb * a.W * a.key_stride;

  // The keys' doc ids and first grant word depend on nothing else: their
  // loads go out first, with the query rows' and the new rows' mask inputs.
  int dj[KPG];
  uint64_t kw0[KPG];
#pragma unroll
  for (int i = 0; i < KPG; ++i) {
    const int j = j0 + kg + NKG * i;
    dj[i] = j < a.Tkv ? kdoc[j] : 0;
    kw0[i] = (a.W > 0 && j < a.Tkv) ? kbits[j] : 0ull;
  }

  if (tid < a.Tq) {
    qpos_s[tid] = a.q_pos[(size_t)mb * a.Tq + tid];
    qdoc_s[tid] = a.q_doc[(size_t)mb * a.Tq + tid];
    for (int w = 0; w < a.W; ++w)
      qbits_s[w][tid] = a.q_bits[((size_t)mb * a.W + w) * a.Tq + tid];
  }

  // Query rows r = g * Tq + tq (query head hk * G + g), elements 8 dg .. 8 dg + 7.
  float qf[RMAX][8];
#pragma unroll
  for (int r = 0; r < RMAX; ++r) {
    if (r < R) {
      const int g = r / a.Tq, tq = r - g * a.Tq;
      const __bf16* qp = static_cast<const __bf16*>(a.q.data) + b * a.q.sb +
                         (int64_t)(hk * G + g) * a.q.sh + (int64_t)tq * a.q.st + 8 * dg;
      const bf16x8 x = *reinterpret_cast<const bf16x8*>(qp);
#pragma unroll
      for (int e = 0; e < 8; ++e) qf[r][e] = (float)x[e] * a.c;
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) qf[r][e] = 0.f;
    }
  }
  __syncthreads();

  // Mask of the group's keys j0 + kg + NKG i: bit tq of allow[i] = allowed for
  // new row tq.  Every load of a stage is issued before any is consumed, so a
  // stage costs one memory latency, not one per key.
  uint32_t allow[KPG];
  {
#pragma unroll
    for (int i = 0; i < KPG; ++i) allow[i] = 0;
    for (int tq = 0; tq < a.Tq; ++tq) {
      const int qd = qdoc_s[tq];
#pragma unroll
      for (int i = 0; i < KPG; ++i) allow[i] |= (dj[i] == qd ? 1u : 0u) << tq;
    }
    for (int w = 0; w < a.W; ++w) {
      uint64_t kw[KPG];
#pragma unroll
      for (int i = 0; i < KPG; ++i) {
        const int j = j0 + kg + NKG * i;
        kw[i] = w == 0 ? kw0[i] : (j < a.Tkv ? kbits[(size_t)w * a.key_stride + j] : 0ull);
      }
      for (int tq = 0; tq < a.Tq; ++tq) {
        const uint64_t qw = qbits_s[w][tq];
#pragma unroll
        for (int i = 0; i < KPG; ++i) allow[i] |= ((qw & kw[i]) != 0ull ? 1u : 0u) << tq;
      }
    }
#pragma unroll
    for (int i = 0; i < KPG; ++i) {
      const int j = j0 + kg + NKG * i;
      uint32_t causal = 0;
      for (int tq = 0; tq < a.Tq; ++tq) causal |= (j <= qpos_s[tq] ? 1u : 0u) << tq;
      allow[i] = j < a.Tkv ? (allow[i] & causal) : 0u;
    }
  }

  // Pass 1: K and V rows of the allowed keys (both issued here: V depends
  // only on the mask), scores to LDS (-inf where masked).
  bf16x8 vx[KPG];
  {
    bf16x8 kx[KPG];
#pragma unroll
    for (int i = 0; i < KPG; ++i) {
      kx[i] = bf16x8{};
      vx[i] = bf16x8{};
      if (allow[i]) {
        kx[i] = *reinterpret_cast<const bf16x8*>(kbase + (int64_t)(j0 + kg + NKG * i) * a.k.st);
        vx[i] = *reinterpret_cast<const bf16x8*>(vbase + (int64_t)(j0 + kg + NKG * i) * a.v.st);
      }
    }
#pragma unroll
    for (int i = 0; i < KPG; ++i) {
      const int jl = kg + NKG * i;
#pragma unroll
      for (int r = 0; r < RMAX; ++r) {
        if (r < R) {
          float acc = 0.f;
#pragma unroll
          for (int e = 0; e < 8; ++e) acc = fmaf(qf[r][e], (float)kx[i][e], acc);
          // The lanes of a key group hold the same allow[i]; the sum runs on all.
          const float tot = group_sum<GL>(acc);
          if (dg == 0) sc[r][jl] = ((allow[i] >> (r % a.Tq)) & 1u) ? tot : -INFINITY;
        }
      }
    }
  }
  __syncthreads();

  // Chunk row max: wave w reduces rows w, w + 4.
  for (int r = wave; r < R; r += kDecThreads / 64) {
    float m = -INFINITY;
    for (int x = lane; x < kDecChunk; x += 64) m = fmaxf(m, sc[r][x]);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
    if (lane == 0) rmax[r] = m;
  }
  __syncthreads();

  // Pass 2: o[r] = sum_j exp2(s - max) V[j], l[r] = sum_j exp2(s - max).
  float o[RMAX][8], l[RMAX];
#pragma unroll
  for (int r = 0; r < RMAX; ++r) {
    l[r] = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[r][e] = 0.f;
  }
  {
#pragma unroll
    for (int i = 0; i < KPG; ++i) {
      const int jl = kg + NKG * i;
#pragma unroll
      for (int r = 0; r < RMAX; ++r) {
        if (r < R) {
          const float sv = sc[r][jl];
          const float pr = sv == -INFINITY ? 0.f : fast_exp2(sv - rmax[r]);
          l[r] += pr;
#pragma unroll
          for (int e = 0; e < 8; ++e) o[r][e] = fmaf(pr, (float)vx[i][e], o[r][e]);
        }
      }
    }
  }
  // Sum over the key groups of a wave (lanes GL apart), then across waves.
#pragma unroll
  for (int r = 0; r < RMAX; ++r) {
    if (r < R) {
#pragma unroll
      for (int off = GL; off < 64; off <<= 1) {
        l[r] += __shfl_xor(l[r], off, 64);
#pragma unroll
        for (int e = 0; e < 8; ++e) o[r][e] += __shfl_xor(o[r][e], off, 64);
      }
      if (lane < GL) {
#pragma unroll
        for (int e = 0; e < 8; ++e) red[wave][r][8 * dg + e] = o[r][e];
      }
    }
  }
  __shared__ float lsum[kDecThreads / 64][RMAX];
  if (lane == 0) {
#pragma unroll
    for (int r = 0; r < RMAX; ++r) lsum[wave][r] = l[r];
  }
  __syncthreads();
  for (int x = tid; x < R * (D + 2); x += kDecThreads) {
    const int r = x / (D + 2), col = x - r * (D + 2);
    const int g = r / a.Tq, tq = r - g * a.Tq;
    float val;
    if (col == 0) {
      val = rmax[r];
    } else if (col == 1) {
      val = 0.f;
      for (int w = 0; w < kDecThreads / 64; ++w) val += lsum[w][r];
    } else {
      val = 0.f;
      for (int w = 0; w < kDecThreads / 64; ++w) val += red[w][r][col - 2];
    }
    const size_t row = ((size_t)b * a.Hq + hk * G + g) * a.Tq + tq;
    a.part[(row * a.nch + chunk) * (D + 2) + col] = val;
  }
}

// One wave per (new token, query head, batch row).  The chunk maxima load one
// chunk per lane; the weighted sum over chunks then issues its loads
// independently (eight in flight per lane), so the merge costs a few memory
// latencies whatever the chunk count.
template <int D>
__global__ __launch_bounds__(64) void attn_decode_combine(DecodeArgs a, TensorView o,
                                                          float* lse2) {
  constexpr int PER = D / 64;
  constexpr int S = D + 2;
  __shared__ float wsh[64];
  const int tq = blockIdx.x, h = blockIdx.y, b = blockIdx.z, lane = threadIdx.x;
  const size_t row = ((size_t)b * a.Hq + h) * a.Tq + tq;
  const float* pr = a.part + row * a.nch * S;
  float M = -INFINITY;
  for (int c = lane; c < a.nch; c += 64) M = fmaxf(M, pr[(size_t)c * S]);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) M = fmaxf(M, __shfl_xor(M, off, 64));
  float L = 0.f, acc[PER];
#pragma unroll
  for (int e = 0; e < PER; ++e) acc[e] = 0.f;
  if (M != -INFINITY) {
    for (int base = 0; base < a.nch; base += 64) {
      const int c = base + lane;
      float w = 0.f;
      if (c < a.nch) {
        const float m = pr[(size_t)c * S];
        w = m == -INFINITY ? 0.f : fast_exp2(m - M);
        L += w * pr[(size_t)c * S + 1];
      }
      wsh[lane] = w;
      __syncthreads();
      const int n = min(64, a.nch - base);
#pragma unroll 8
      for (int k = 0; k < n; ++k) {
        const float wk = wsh[k];
#pragma unroll
        for (int e = 0; e < PER; ++e)
          acc[e] = fmaf(wk, pr[(size_t)(base + k) * S + 2 + lane + 64 * e], acc[e]);
      }
      __syncthreads();
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) L += __shfl_xor(L, off, 64);
  }
  const float inv = L > 0.f ? 1.f / L : 0.f;
  __bf16* op = static_cast<__bf16*>(o.data) + b * o.sb + h * o.sh + (int64_t)tq * o.st;
#pragma unroll
  for (int e = 0; e < PER; ++e) op[lane + 64 * e] = (__bf16)(acc[e] * inv);
  if (lane == 0) lse2[row] = L > 0.f ? M + log2f(L) : -INFINITY;
}

template <int D>
void launch_partial(int R, dim3 grid, const DecodeArgs& a, hipStream_t stream) {
  if (R <= 1)
    hipLaunchKernelGGL((attn_decode_partial<D, 1>), grid, dim3(kDecThreads), 0, stream, a);
  else if (R <= 2)
    hipLaunchKernelGGL((attn_decode_partial<D, 2>), grid, dim3(kDecThreads), 0, stream, a);
  else if (R <= 4)
    hipLaunchKernelGGL((attn_decode_partial<D, 4>), grid, dim3(kDecThreads), 0, stream, a);
  else
    hipLaunchKernelGGL((attn_decode_partial<D, 8>), grid, dim3(kDecThreads), 0, stream, a);
}

}  // namespace

int64_t decode_workspace_floats(int B, int Hq, int Tq, int Tkv, int D) {
  const int64_t nch = (Tkv + kDecChunk - 1) / kDecChunk;
  return (int64_t)B * Hq * Tq * (nch > 0 ? nch : 1) * (D + 2);
}

hipError_t launch_attn_decode(const TensorView& q, const TensorView& k, const TensorView& v,
                              const TensorView& o, float* lse2, const int32_t* key_doc,
                              const uint64_t* key_bits, int64_t key_stride, const int32_t* q_pos,
                              const int32_t* q_doc, const uint64_t* q_bits, int Bm, int W,
                              int B, int Hq, int Hkv, int Tq, int Tkv, int D, float scale,
                              float* workspace, hipStream_t stream) {
  DecodeArgs a{q,     k,      v,    key_doc, key_bits, key_stride, q_pos, q_doc,
               q_bits, Bm,    W,    B,       Hq,       Hkv,        Tq,    Tkv,
               (Tkv + kDecChunk - 1) / kDecChunk, scale * kLog2e, workspace};
  if (a.nch == 0) a.nch = 1;  // no keys: one chunk that finds nothing
  const dim3 pgrid((unsigned)a.nch, (unsigned)Hkv, (unsigned)B);
  const dim3 cgrid((unsigned)Tq, (unsigned)Hq, (unsigned)B);
  const int R = (Hq / Hkv) * Tq;
  if (D == 64) {
    launch_partial<64>(R, pgrid, a, stream);
    hipLaunchKernelGGL(attn_decode_combine<64>, cgrid, dim3(64), 0, stream, a, o, lse2);
  } else {
    launch_partial<128>(R, pgrid, a, stream);
    hipLaunchKernelGGL(attn_decode_combine<128>, cgrid, dim3(64), 0, stream, a, o, lse2);
  }
  return hipGetLastError();
}

}  // namespace t2t
