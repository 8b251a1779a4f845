// Masked flash-attention forward, bf16 in / fp32 accumulate, gfx950 MFMA.
//
// Computes, per (batch b, query head h, 128-query tile), the output of
// torch's math_attention (torch/_higher_order_ops/flex_attention.py:202-267):
//   O = softmax_masked(Q K^T * scale) V,   LSE = logsumexp of the masked row,
// with fully masked rows giving O = 0 and LSE = -inf.  The reference's Triton
// template iterates the row's partial KV tiles with the mask and its full
// tiles without it; this kernel consumes the same BlockMask lists
// (kv_num_blocks / kv_indices, full_kv_num_blocks / full_kv_indices).
//
// Formulation (per wave, 32 queries):  S^T = K Q^T  so that every lane owns a
// single query column (row max / row sum need one cross-half exchange), then
// O^T += V^T P^T with P^T fed straight from the S^T accumulators and V^T read
// from the row-major LDS tile by transpose loads.  The softmax runs in the
// log2 domain (scores pre-multiplied by scale * log2 e); LSE is written in
// that domain, and the host multiplies by ln 2 for the natural-log value.
#include "attn_kernels.h"

namespace t2t {

namespace {

template <int D>
struct FwdSmem {
  static constexpr int kPitch = D + 8;  // +16 B per row: spreads row reads over banks
  __bf16 k[kTile * kPitch];
  __bf16 v[kTile * kPitch];
  int32_t kdoc[kTile];
  uint64_t kbits[kMaxWords][kTile];
};

struct FwdParams {
  const __bf16* q; int64_t q_sb, q_sh, q_st;
  const __bf16* k; int64_t k_sb, k_sh, k_st;
  const __bf16* v; int64_t v_sb, v_sh, v_st;
  __bf16* o; int64_t o_sb, o_sh, o_st;
  float* lse2;
  int B, Hq, Hkv, T, nt;
  float scale_log2;
  MaskTables m;
};

// Copy token rows [t0, t0 + 128) of a [T, D] slice into a row-major LDS tile
// (rows past T are zero-filled).
template <int D, int PITCH>
__device__ __forceinline__ void load_tile(__bf16* dst, const __bf16* src, int64_t st, int t0,
                                          int T, int tid) {
  constexpr int kChunks = D / 8;  // 16-byte chunks per row
  constexpr int kIters = kTile * kChunks / kThreads;
  uint4 buf[kIters];
#pragma unroll
  for (int it = 0; it < kIters; ++it) {
    const int c = tid + it * kThreads;
    const int r = c / kChunks, col = (c % kChunks) * 8;
    const int t = t0 + r;
    buf[it] = (t < T) ? *reinterpret_cast<const uint4*>(src + (int64_t)t * st + col)
                      : make_uint4(0, 0, 0, 0);
  }
#pragma unroll
  for (int it = 0; it < kIters; ++it) {
    const int c = tid + it * kThreads;
    const int r = c / kChunks, col = (c % kChunks) * 8;
    *reinterpret_cast<uint4*>(dst + r * PITCH + col) = buf[it];
  }
}

}  // namespace

template <int D>
__global__ __launch_bounds__(kThreads, 1) void attn_fwd_bf16_kernel(FwdParams p) {
  constexpr int PITCH = FwdSmem<D>::kPitch;
  constexpr int KS = D / 16;  // MFMA k-steps over the head dim
  constexpr int DT = D / 32;  // 32-wide output column tiles
  __shared__ FwdSmem<D> sm;

  const int qt = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int g = lane >> 5, n = lane & 31;
  const int hk = h / (p.Hq / p.Hkv);
  const int mb = p.m.Bm > 1 ? b : 0;
  const int T = p.T, nt = p.nt, words = p.m.words;
  const int q0 = qt * kTile;
  const int qrow = q0 + 32 * wave + n;
  const bool qvalid = qrow < T;

  // Q^T operand: lane (g, n) holds Q[qrow][16 s + 8 g + j].
  bf16x8 qf[KS];
  {
    const __bf16* qp = p.q + b * p.q_sb + h * p.q_sh + (int64_t)(qvalid ? qrow : 0) * p.q_st;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      bf16x8 x = *reinterpret_cast<const bf16x8*>(qp + 16 * s + 8 * g);
      qf[s] = qvalid ? x : bf16x8{};
    }
  }
  const int32_t* mdoc = p.m.doc + (size_t)mb * T;
  const uint64_t* mqb = p.m.qbits + (size_t)mb * words * T;
  const uint64_t* mkb = p.m.kvbits + (size_t)mb * words * T;
  int32_t qdoc = qvalid ? mdoc[qrow] : 0;
  uint64_t qbits[kMaxWords];
#pragma unroll
  for (int w = 0; w < kMaxWords; ++w) qbits[w] = (w < words && qvalid) ? mqb[(size_t)w * T + qrow] : 0ull;

  const __bf16* kbase = p.k + b * p.k_sb + hk * p.k_sh;
  const __bf16* vbase = p.v + b * p.v_sb + hk * p.v_sh;
  const size_t row = (size_t)mb * nt + qt;
  const int npart = p.m.kv_num[row];
  const int nfull = p.m.full_kv_num[row];
  const int32_t* pidx = p.m.kv_idx + row * nt;
  const int32_t* fidx = p.m.full_kv_idx + row * nt;

  f32x16 oacc[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) oacc[dt] = f32x16{};
  float m_run = -INFINITY, l_run = 0.f;

  for (int it = 0; it < npart + nfull; ++it) {
    const bool partial = it < npart;
    const int kt = partial ? pidx[it] : fidx[it - npart];
    const int k0 = kt * kTile;
    __syncthreads();
    load_tile<D, PITCH>(sm.k, kbase, p.k_st, k0, T, tid);
    load_tile<D, PITCH>(sm.v, vbase, p.v_st, k0, T, tid);
    if (partial && tid < kTile) {
      const int t = k0 + tid;
      sm.kdoc[tid] = t < T ? mdoc[t] : 0;
      for (int w = 0; w < words; ++w) sm.kbits[w][tid] = t < T ? mkb[(size_t)w * T + t] : 0ull;
    }
    __syncthreads();

    // S^T (4 blocks of 32 keys) = K Q^T.
    f32x16 st[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      st[j] = f32x16{};
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        const bf16x8 kf = lds_row8(&sm.k[(32 * j + n) * PITCH + 16 * s + 8 * g]);
        st[j] = mfma32(kf, qf[s], st[j]);
      }
    }

    // Scale into the log2 domain, mask partial tiles, running max.
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        float x = st[j][i] * p.scale_log2;
        if (partial) {
          const int kk = 32 * j + acc_row(i, g);
          const int key = k0 + kk;
          bool ok = qvalid && key < T && key <= qrow;
          if (ok && qdoc != sm.kdoc[kk]) {
            bool hit = false;
            for (int w = 0; w < words; ++w) hit |= (qbits[w] & sm.kbits[w][kk]) != 0ull;
            ok = hit;
          }
          if (!ok) x = -INFINITY;
        }
        st[j][i] = x;
        mx = fmaxf(mx, x);
      }
    }
    mx = fmaxf(mx, swap_halves(mx));
    const float m_new = fmaxf(m_run, mx);
    const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
    const float alpha = fast_exp2(m_run - m_use);
    float rs = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const float e = fast_exp2(st[j][i] - m_use);
        st[j][i] = e;
        rs += e;
      }
    }
    rs += swap_halves(rs);
    l_run = l_run * alpha + rs;
    m_run = m_new;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) oacc[dt] *= alpha;

    // O^T += V^T P^T, 16 keys per k-step.
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const int j = s >> 1, hh = s & 1;
      const bf16x8 pf = pack_half(st[j], hh);
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const bf16x8 vf = lds_col8(sm.v, PITCH, 32 * j + 16 * hh, 8, 32 * dt, lane);
        oacc[dt] = mfma32(vf, pf, oacc[dt]);
      }
    }
  }

  if (qvalid) {
    const float inv_l = l_run > 0.f ? 1.f / l_run : 0.f;
    __bf16* op = p.o + b * p.o_sb + h * p.o_sh + (int64_t)qrow * p.o_st;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
#pragma unroll
      for (int i = 0; i < 16; i += 4) {
        bf16x4 w4;
#pragma unroll
        for (int e = 0; e < 4; ++e) w4[e] = (__bf16)(oacc[dt][i + e] * inv_l);
        *reinterpret_cast<bf16x4*>(op + 32 * dt + acc_row(i, g)) = w4;
      }
    }
    if (g == 0)
      p.lse2[((size_t)b * p.Hq + h) * T + qrow] = l_run > 0.f ? m_run + __log2f(l_run) : -INFINITY;
  }
}

hipError_t launch_attn_fwd_bf16(const TensorView& q, const TensorView& k, const TensorView& v,
                                const TensorView& o, float* lse2, const AttnDims& dims,
                                const MaskTables& mask, hipStream_t stream) {
  FwdParams p;
  p.q = static_cast<const __bf16*>(q.data); p.q_sb = q.sb; p.q_sh = q.sh; p.q_st = q.st;
  p.k = static_cast<const __bf16*>(k.data); p.k_sb = k.sb; p.k_sh = k.sh; p.k_st = k.st;
  p.v = static_cast<const __bf16*>(v.data); p.v_sb = v.sb; p.v_sh = v.sh; p.v_st = v.st;
  p.o = static_cast<__bf16*>(o.data); p.o_sb = o.sb; p.o_sh = o.sh; p.o_st = o.st;
  p.lse2 = lse2;
  p.B = dims.B; p.Hq = dims.Hq; p.Hkv = dims.Hkv; p.T = dims.T;
  p.nt = (dims.T + kTile - 1) / kTile;
  p.scale_log2 = dims.scale * 1.4426950408889634f;
  p.m = mask;
  if (p.nt == 0 || dims.B == 0 || dims.Hq == 0) return hipSuccess;
  dim3 grid(p.nt, dims.Hq, dims.B);
  if (dims.D == 64)
    hipLaunchKernelGGL(attn_fwd_bf16_kernel<64>, grid, dim3(kThreads), 0, stream, p);
  else
    hipLaunchKernelGGL(attn_fwd_bf16_kernel<128>, grid, dim3(kThreads), 0, stream, p);
  return hipGetLastError();
}

}  // namespace t2t
