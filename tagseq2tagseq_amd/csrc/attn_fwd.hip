// Masked flash-attention forward, bf16 in / fp32 accumulate, gfx950 MFMA.
//
// Computes, per (batch b, query head h, 128-query tile), the output of
// torch's math_attention (torch/_higher_order_ops/flex_attention.py:202-267):
//   O = softmax_masked(Q K^T * scale) V,   LSE = logsumexp of the masked row,
// with fully masked rows giving O = 0 and LSE = -inf.  The reference's Triton
// template iterates the row's partial KV tiles with the mask and its full
// tiles without it; this kernel consumes the same BlockMask lists
// (kv_num_blocks / kv_indices, full_kv_num_blocks / full_kv_indices) and, for
// partial tiles, the precomputed allowed-pair bitmap of the tile.
//
// Formulation (per wave, 32 queries):  S^T = K Q^T  so that every lane owns a
// single query column (row max / row sum need one cross-half exchange), then
// O^T += V^T P^T with P^T fed straight from the S^T accumulators (keys in
// tok_perm order) and V^T read from the row-major LDS tile by transpose loads
// in the same key order.  The softmax runs in the
// log2 domain (scores times scale * log2 e); LSE is written in that domain,
// and the host multiplies by ln 2 for the natural-log value.
//
// Work-groups are dispatched longest row first (row_order) with the head as
// the fastest grid dimension, so the heads sharing an XCD (blockIdx.x mod 8)
// stream the same K/V through that XCD's L2.
#include "attn_kernels.h"

namespace t2t {

namespace {

template <int D>
struct FwdSmem {
  __bf16 k[kTile * pitch<D>()];  // padded rows
  __bf16 v[kTile * pitch<D>()];
};

struct FwdParams {
  const __bf16* q; int64_t q_sb, q_sh, q_st;
  const __bf16* k; int64_t k_sb, k_sh, k_st;
  const __bf16* v; int64_t v_sb, v_sh, v_st;
  __bf16* o; int64_t o_sb, o_sh, o_st;
  float* lse2;
  int B, Hq, Hkv, T;
  float scale_log2;
  MaskTables m;
};

}  // namespace

template <int D>
__global__ __launch_bounds__(kThreads, 2) void attn_fwd_bf16_kernel(FwdParams p) {
  constexpr int KS = D / 16;  // MFMA k-steps over the head dim
  constexpr int DT = D / 32;  // 32-wide output column tiles
  __shared__ FwdSmem<D> sm;

  const int h = blockIdx.x, b = blockIdx.z;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int g = lane >> 5, n = lane & 31;
  const int hk = h / (p.Hq / p.Hkv);
  const int mb = p.m.Bm > 1 ? b : 0;
  const int T = p.T, nt = p.m.nt;
  const int qt = uniform(p.m.row_order[(size_t)mb * nt + blockIdx.y]);
  const int q0 = qt * kTile;
  const int qloc = 32 * wave + n;  // query row within the tile
  const int qrow = q0 + qloc;
  const bool qvalid = qrow < T;
  const float c = p.scale_log2;

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

  const auto krs = slice_rsrc(p.k + b * p.k_sb + hk * p.k_sh, p.k_st, T, D);
  const auto vrs = slice_rsrc(p.v + b * p.v_sb + hk * p.v_sh, p.v_st, T, D);
  const size_t row = (size_t)mb * nt + qt;
  const int npart = uniform(p.m.kv_num[row]);
  const int nfull = uniform(p.m.full_kv_num[row]);
  const int32_t* pidx = p.m.kv_idx + row * nt;
  const int32_t* fidx = p.m.full_kv_idx + row * nt;
  const uint32_t* bits_base = p.m.tile_bits + (size_t)p.m.kv_bits_off[row] * kTileBitsWords + qloc * 4;

  f32x16 oacc[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) oacc[dt] = f32x16{};
  float m_run = -INFINITY, l_run = 0.f;  // running max of raw scores, running sum

  for (int it = 0; it < npart + nfull; ++it) {
    const bool partial = it < npart;
    const int kt = uniform(partial ? pidx[it] : fidx[it - npart]);
    const int k0 = kt * kTile;
    uint4 mbits = make_uint4(~0u, ~0u, ~0u, ~0u);
    if (partial) mbits = *reinterpret_cast<const uint4*>(bits_base + (size_t)it * kTileBitsWords);
    __syncthreads();
    load_tile_lds<D>(sm.k, krs, p.k_st, k0, tid);
    load_tile_lds<D>(sm.v, vrs, p.v_st, k0, tid);
    __syncthreads();

    // 32-key blocks of this wave: empty (no allowed pair: skipped), full (no
    // masking) or mixed (masked through the accumulator seed).  Wave-uniform.
    const uint32_t w4[4] = {mbits.x, mbits.y, mbits.z, mbits.w};
    bool act[4], mixed[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {  // full tiles carry all-ones words
      act[j] = __ballot(w4[j] != 0u) != 0ull;
      mixed[j] = __ballot(w4[j] != ~0u) != 0ull;
    }

    // The tile is processed as two 64-key halves, each a complete online
    // softmax step; this bounds the live score registers to 32 per lane.
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      const int j0 = 2 * half;
      if (!act[j0] && !act[j0 + 1]) continue;
      // S^T (2 blocks of 32 keys) = K Q^T (+ mask bias).
      f32x16 st[2];
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        const int j = j0 + jj;
        if (!act[j]) continue;
        const bf16x8 kf0 = lds_row8<D>(sm.k, 32 * j + tok_perm(n), 8 * g);
        if (mixed[j]) st[jj] = mfma32(kf0, qf[0], mask_bias(w4[j] >> g));
        else st[jj] = mfma32(kf0, qf[0], f32x16{});
#pragma unroll
        for (int s = 1; s < KS; ++s) {
          const bf16x8 kf = lds_row8<D>(sm.k, 32 * j + tok_perm(n), 16 * s + 8 * g);
          st[jj] = mfma32(kf, qf[s], st[jj]);
        }
      }

      float mx = -INFINITY;
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        if (!act[j0 + jj]) continue;
#pragma unroll
        for (int i = 0; i < 16; ++i) mx = fmaxf(mx, st[jj][i]);
      }
      mx = halves_max(mx);
      const float m_new = fmaxf(m_run, mx);
      const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
      const float neg = -m_use * c;
      float rs = 0.f;
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        if (!act[j0 + jj]) continue;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const float e = fast_exp2(fmaf(st[jj][i], c, neg));
          st[jj][i] = e;
          rs += e;
        }
      }
      rs = halves_sum(rs);
      // Rescale O only when some lane's running max moved (alpha == 1 otherwise).
      if (__ballot(m_new != m_run) != 0ull) {
        const float alpha = fast_exp2((m_run - m_use) * c);
        l_run *= alpha;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) oacc[dt] *= alpha;
      }
      l_run += rs;
      m_run = m_new;

      // O^T += V^T P^T, 16 keys per k-step.
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int jj = s >> 1, hh = s & 1;
        const int j = j0 + jj;
        if (!act[j]) continue;
        const bf16x8 pf = pack_half(st[jj], hh);
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
          const bf16x8 vf = lds_col8<D>(sm.v, 32 * j + 16 * hh, 32 * dt, lane);
          oacc[dt] = mfma32(vf, pf, oacc[dt]);
        }
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
      p.lse2[((size_t)b * p.Hq + h) * T + qrow] =
          l_run > 0.f ? m_run * c + __log2f(l_run) : -INFINITY;
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
  p.scale_log2 = dims.scale * kLog2e;
  p.m = mask;
  if (mask.nt == 0 || dims.B == 0 || dims.Hq == 0) return hipSuccess;
  dim3 grid(dims.Hq, mask.nt, dims.B);
  if (dims.D == 64)
    hipLaunchKernelGGL(attn_fwd_bf16_kernel<64>, grid, dim3(kThreads), 0, stream, p);
  else
    hipLaunchKernelGGL(attn_fwd_bf16_kernel<128>, grid, dim3(kThreads), 0, stream, p);
  return hipGetLastError();
}

}  // namespace t2t
