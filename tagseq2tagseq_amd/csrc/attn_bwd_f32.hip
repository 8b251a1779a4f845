// Masked flash-attention backward for float32 inputs, gfx950 fp32 MFMA.
//
// The float32 form of sdpa_dense_backward
// (torch/_higher_order_ops/flex_attention.py:825-994): P = exp(S - LSE),
// Delta = rowsum(O * dO), dS = P (dP - Delta) * scale, dQ = dS K,
// dK = dS^T Q (summed over each GQA group), dV = P^T dO; masked pairs and
// fully masked rows contribute nothing.  Every product and sum is float32
// (v_mfma_f32_32x32x2_f32); no atomics, so the result is deterministic.
//
// Two launches: dQ (which also computes each of its rows' Delta and writes it
// out), then dK/dV.  Both read their operands straight from global memory
// (the L2 serves the re-reads) rather than staging them through LDS: a
// float32 row is twice a bf16 row, and a register-resident operand per lane
// keeps the kernels short.  The operand mapping is the float32 forward's:
// k-step s of a contraction over the head dim pairs d = s and d = s + D/2
// (lane group g takes g D/2 + s), and a contraction over tokens takes, at
// k-step ks, the token of accumulator entry ks (acc_row(ks, g)), so a P or dS
// accumulator entry is directly the B operand; output row m of tile dt is head
// dim DT m + dt.
#include "attn_kernels.h"

namespace t2t {

namespace {

struct BwdF32Params {
  const float* q; int64_t q_sb, q_sh, q_st;
  const float* k; int64_t k_sb, k_sh, k_st;
  const float* v; int64_t v_sb, v_sh, v_st;
  const float* o; int64_t o_sb, o_sh, o_st;
  const float* dout; int64_t do_sb, do_sh, do_st;
  float* dq; int64_t dq_sb, dq_sh, dq_st;
  float* dk; int64_t dk_sb, dk_sh, dk_st;
  float* dv; int64_t dv_sb, dv_sh, dv_st;
  const float* lse2;  // [B][Hq][T], log2 domain of scaled scores
  float* delta;       // [B][Hq][T]
  int B, Hq, Hkv, T;
  float scale, scale_log2;
  MaskTables m;
};

__device__ __forceinline__ f32x16 mfma32_f32(float a, float b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// Mixed-block seed, tokens in natural order: 0 allowed, -inf masked; nw =
// ~w >> (4 g), entry i of lane group g = token acc_row(i, g) of the block.
template <int I = 0>
__device__ __forceinline__ void seed_fill(f32x16& c, uint32_t nw) {
  if constexpr (I < 16) {
    c[I] = __int_as_float(sbfe1_c<8 * (I >> 2) + (I & 3)>(nw) & (int)0xff800000);
    seed_fill<I + 1>(c, nw);
  }
}

// Stores a 32 x 32 accumulator block of the transposed gradient (row m of
// tile dt = head dim DT m + dt, column = the lane's token) into out_row.
template <int DT>
__device__ __forceinline__ void store_rows(float* out_row, const f32x16* acc, int g, float mul) {
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    float* dst = out_row + DT * acc_row(i, g);
    if constexpr (DT == 4) {
      f32x4 w;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) w[dt] = acc[dt][i] * mul;
      *reinterpret_cast<f32x4*>(dst) = w;
    } else {
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) dst[dt] = acc[dt][i] * mul;
    }
  }
}

// The DT consecutive floats [DT n, DT n + DT) of a row.
template <int DT>
__device__ __forceinline__ f32x4 row_piece(const float* row, int n) {
  if constexpr (DT == 4) {
    return *reinterpret_cast<const f32x4*>(row + DT * n);
  } else {
    const float2 x = *reinterpret_cast<const float2*>(row + DT * n);
    return f32x4{x.x, x.y, 0.f, 0.f};
  }
}

}  // namespace

// dQ (and Delta) for one (b, query head, 128-query tile); wave w takes
// queries 32 w .. 32 w + 31, one per lane (S^T = K Q^T, keys in the
// accumulator rows), and walks the row's KV tiles 32 keys at a time.
template <int D>
__global__ __launch_bounds__(kThreads, 1) void bwd_dq_f32_kernel(BwdF32Params p) {
  constexpr int KS = D / 2;
  constexpr int DT = D / 32;
  const int h = blockIdx.x, b = blockIdx.z;
  const int tid = threadIdx.x, wave = uniform(tid >> 6), lane = tid & 63;
  const int g = lane >> 5, n = lane & 31;
  const int hk = h / (p.Hq / p.Hkv);
  const int mb = p.m.Bm > 1 ? b : 0;
  const int T = p.T, nt = p.m.nt;
  const int qt = uniform(p.m.row_order[(size_t)mb * nt + blockIdx.y]);
  const int qloc = 32 * wave + n;
  const int qrow = qt * kTile + qloc;
  const bool qvalid = qrow < T;
  const int qr = qvalid ? qrow : T - 1;  // rows past T only reach their own, unstored dQ
  const size_t rowstat = ((size_t)b * p.Hq + h) * T + qr;
  const float c = p.scale_log2;

  float qf[KS], dof[KS];
  float delta = 0.f;
  {
    const float* qp = p.q + b * p.q_sb + h * p.q_sh + (int64_t)qr * p.q_st + g * KS;
    const float* dp = p.dout + b * p.do_sb + h * p.do_sh + (int64_t)qr * p.do_st + g * KS;
    const float* op = p.o + b * p.o_sb + h * p.o_sh + (int64_t)qr * p.o_st + g * KS;
#pragma unroll
    for (int s = 0; s < KS; s += 4) {
      const f32x4 a = *reinterpret_cast<const f32x4*>(qp + s);
      const f32x4 d = *reinterpret_cast<const f32x4*>(dp + s);
      const f32x4 o = *reinterpret_cast<const f32x4*>(op + s);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        qf[s + e] = a[e];
        dof[s + e] = d[e];
        delta = fmaf(o[e], d[e], delta);
      }
    }
  }
  delta = halves_sum(delta);  // Delta = rowsum(O * dO) (both lane halves)
  if (qvalid && g == 0) p.delta[rowstat] = delta;
  const float lrow = p.lse2[rowstat];
  const float neg_lse = (!qvalid || lrow == -INFINITY) ? -INFINITY : -lrow;

  const size_t row = (size_t)mb * nt + qt;
  const int npart = uniform(p.m.kv_num[row]);
  const int ntiles = npart + uniform(p.m.full_kv_num[row]);
  const int32_t* pidx = p.m.kv_idx + row * nt;
  const int32_t* fidx = p.m.full_kv_idx + row * nt;
  const uint32_t* bits_row = p.m.tile_bits + (size_t)p.m.kv_bits_off[row] * kTileBitsWords;
  const float* kbase = p.k + b * p.k_sb + hk * p.k_sh;
  const float* vbase = p.v + b * p.v_sb + hk * p.v_sh;

  f32x16 dqacc[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) dqacc[dt] = f32x16{};

  for (int it = 0; it < ntiles; ++it) {
    const bool partial = it < npart;
    const int kt = uniform(partial ? pidx[it] : fidx[it - npart]);
    uint4 wq = make_uint4(~0u, ~0u, ~0u, ~0u);
    if (partial)
      wq = *reinterpret_cast<const uint4*>(bits_row + (size_t)kt * kTileBitsWords + qloc * 4);
#pragma unroll 1
    for (int j = 0; j < 4; ++j) {
      const uint32_t w = j == 0 ? wq.x : j == 1 ? wq.y : j == 2 ? wq.z : wq.w;
      if (partial && __ballot(w != 0u) == 0ull) continue;
      const int kb = kt * kTile + 32 * j;
      f32x16 sacc = f32x16{}, dpacc = f32x16{};
      if (partial && __ballot(w != ~0u) != 0ull) seed_fill(sacc, ~w >> (4 * g));
      // S^T = K Q^T, dP^T = V dO^T: lane (g, n) supplies key kb + n.  Keys
      // past T (masked by the padded tile bitmap) read row T - 1.
      const int krow = min(kb + n, T - 1);
      const float* kp = kbase + (int64_t)krow * p.k_st + g * KS;
      const float* vp = vbase + (int64_t)krow * p.v_st + g * KS;
#pragma unroll
      for (int s = 0; s < KS; s += 4) {
        const f32x4 ka = *reinterpret_cast<const f32x4*>(kp + s);
        const f32x4 va = *reinterpret_cast<const f32x4*>(vp + s);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          sacc = mfma32_f32(ka[e], qf[s + e], sacc);
          dpacc = mfma32_f32(va[e], dof[s + e], dpacc);
        }
      }
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const float pv = fast_exp2(fmaf(sacc[i], c, neg_lse));
        dpacc[i] = pv * (dpacc[i] - delta);  // dS^T
      }
      // dQ^T += K^T dS^T over the block's 32 keys.
#pragma unroll
      for (int ks = 0; ks < 16; ++ks) {
        const f32x4 kc = row_piece<DT>(kbase + (int64_t)min(kb + acc_row(ks, g), T - 1) * p.k_st, n);
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) dqacc[dt] = mfma32_f32(kc[dt], dpacc[ks], dqacc[dt]);
      }
    }
  }
  if (qvalid)
    store_rows<DT>(p.dq + b * p.dq_sb + h * p.dq_sh + (int64_t)qrow * p.dq_st, dqacc, g, p.scale);
}

// dK, dV for one (b, kv head, 128-key tile); wave w owns keys 32 w .. 32 w +
// 31, one per lane, with their K and V rows in registers (S = Q K^T, queries
// in the accumulator rows), and walks the column's (query head, query tile)
// items 32 queries at a time.
template <int D>
__global__ __launch_bounds__(kThreads, 1) void bwd_dkdv_f32_kernel(BwdF32Params p) {
  constexpr int KS = D / 2;
  constexpr int DT = D / 32;
  const int hk = blockIdx.x, b = blockIdx.z;
  const int tid = threadIdx.x, wave = uniform(tid >> 6), lane = tid & 63;
  const int g = lane >> 5, n = lane & 31;
  const int G = p.Hq / p.Hkv;
  const int mb = p.m.Bm > 1 ? b : 0;
  const int T = p.T, nt = p.m.nt;
  const int kt = uniform(p.m.col_order[(size_t)mb * nt + blockIdx.y]);
  const int kloc = 32 * wave + n;
  const int key = kt * kTile + kloc;
  const bool kvalid = key < T;
  const int kr = kvalid ? key : T - 1;
  const float c = p.scale_log2;

  float kf[KS], vf[KS];
  {
    const float* kp = p.k + b * p.k_sb + hk * p.k_sh + (int64_t)kr * p.k_st + g * KS;
    const float* vp = p.v + b * p.v_sb + hk * p.v_sh + (int64_t)kr * p.v_st + g * KS;
#pragma unroll
    for (int s = 0; s < KS; s += 4) {
      const f32x4 a = *reinterpret_cast<const f32x4*>(kp + s);
      const f32x4 d = *reinterpret_cast<const f32x4*>(vp + s);
#pragma unroll
      for (int e = 0; e < 4; ++e) { kf[s + e] = a[e]; vf[s + e] = d[e]; }
    }
  }

  const size_t col = (size_t)mb * nt + kt;
  const int npart = uniform(p.m.q_num[col]);
  const int nq = npart + uniform(p.m.full_q_num[col]);
  const int32_t* pidx = p.m.q_idx + col * nt;
  const int32_t* fidx = p.m.full_q_idx + col * nt;
  const int32_t* pslot = p.m.q_bits_slot + col * nt;
  const uint32_t* bits_col = p.m.tile_bits + kTile * 4 + kloc * 4;

  f32x16 dkacc[DT], dvacc[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) { dkacc[dt] = f32x16{}; dvacc[dt] = f32x16{}; }

  for (int hh = 0; hh < G; ++hh) {
    const int h = hk * G + hh;
    const float* qbase = p.q + b * p.q_sb + h * p.q_sh;
    const float* dbase = p.dout + b * p.do_sb + h * p.do_sh;
    const float* lbase = p.lse2 + ((size_t)b * p.Hq + h) * T;
    const float* dlbase = p.delta + ((size_t)b * p.Hq + h) * T;
    for (int it = 0; it < nq; ++it) {
      const bool partial = it < npart;
      const int qt = uniform(partial ? pidx[it] : fidx[it - npart]);
      uint4 wk = make_uint4(~0u, ~0u, ~0u, ~0u);
      if (partial)
        wk = *reinterpret_cast<const uint4*>(bits_col + (size_t)pslot[it] * kTileBitsWords);
#pragma unroll 1
      for (int j = 0; j < 4; ++j) {
        const uint32_t w = j == 0 ? wk.x : j == 1 ? wk.y : j == 2 ? wk.z : wk.w;
        if (partial && __ballot(w != 0u) == 0ull) continue;
        const int qb = qt * kTile + 32 * j;
        f32x16 sacc = f32x16{}, dpacc = f32x16{};
        if (partial && __ballot(w != ~0u) != 0ull) seed_fill(sacc, ~w >> (4 * g));
        // S = Q K^T, dP = dO V^T: lane (g, n) supplies query qb + n.
        // Queries past T (masked by the padded tile bitmap) read row T - 1.
        const int qrow = min(qb + n, T - 1);
        const float* qp = qbase + (int64_t)qrow * p.q_st + g * KS;
        const float* dp = dbase + (int64_t)qrow * p.do_st + g * KS;
#pragma unroll
        for (int s = 0; s < KS; s += 4) {
          const f32x4 qa = *reinterpret_cast<const f32x4*>(qp + s);
          const f32x4 da = *reinterpret_cast<const f32x4*>(dp + s);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            sacc = mfma32_f32(qa[e], kf[s + e], sacc);
            dpacc = mfma32_f32(da[e], vf[s + e], dpacc);
          }
        }
        // P and dS; entry i is query qb + acc_row(i, g).  A fully masked row
        // (LSE = -inf) has only -inf scores; clamping its LSE keeps P at 0.
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int qi = min(qb + acc_row(i, g), T - 1);
          const float lse = fmaxf(lbase[qi], -3.402823466e38f);
          const float pv = fast_exp2(fmaf(sacc[i], c, -lse));
          sacc[i] = pv;
          dpacc[i] = pv * (dpacc[i] - dlbase[qi]);
        }
        // dV^T += dO^T P, dK^T += Q^T dS over the block's 32 queries.
#pragma unroll
        for (int ks = 0; ks < 16; ++ks) {
          const int qi = min(qb + acc_row(ks, g), T - 1);
          const f32x4 dc = row_piece<DT>(dbase + (int64_t)qi * p.do_st, n);
          const f32x4 qc = row_piece<DT>(qbase + (int64_t)qi * p.q_st, n);
#pragma unroll
          for (int dt = 0; dt < DT; ++dt) {
            dvacc[dt] = mfma32_f32(dc[dt], sacc[ks], dvacc[dt]);
            dkacc[dt] = mfma32_f32(qc[dt], dpacc[ks], dkacc[dt]);
          }
        }
      }
    }
  }
  if (kvalid) {
    store_rows<DT>(p.dk + b * p.dk_sb + hk * p.dk_sh + (int64_t)key * p.dk_st, dkacc, g, p.scale);
    store_rows<DT>(p.dv + b * p.dv_sb + hk * p.dv_sh + (int64_t)key * p.dv_st, dvacc, g, 1.f);
  }
}

hipError_t launch_attn_bwd_f32(const TensorView& q, const TensorView& k, const TensorView& v,
                               const TensorView& o, const TensorView& dout, const float* lse2,
                               float* delta, const TensorView& dq, const TensorView& dk,
                               const TensorView& dv, const AttnDims& dims, const MaskTables& mask,
                               hipStream_t stream) {
  BwdF32Params p;
  p.q = static_cast<const float*>(q.data); p.q_sb = q.sb; p.q_sh = q.sh; p.q_st = q.st;
  p.k = static_cast<const float*>(k.data); p.k_sb = k.sb; p.k_sh = k.sh; p.k_st = k.st;
  p.v = static_cast<const float*>(v.data); p.v_sb = v.sb; p.v_sh = v.sh; p.v_st = v.st;
  p.o = static_cast<const float*>(o.data); p.o_sb = o.sb; p.o_sh = o.sh; p.o_st = o.st;
  p.dout = static_cast<const float*>(dout.data);
  p.do_sb = dout.sb; p.do_sh = dout.sh; p.do_st = dout.st;
  p.dq = static_cast<float*>(dq.data); p.dq_sb = dq.sb; p.dq_sh = dq.sh; p.dq_st = dq.st;
  p.dk = static_cast<float*>(dk.data); p.dk_sb = dk.sb; p.dk_sh = dk.sh; p.dk_st = dk.st;
  p.dv = static_cast<float*>(dv.data); p.dv_sb = dv.sb; p.dv_sh = dv.sh; p.dv_st = dv.st;
  p.lse2 = lse2;
  p.delta = delta;
  p.B = dims.B; p.Hq = dims.Hq; p.Hkv = dims.Hkv; p.T = dims.T;
  p.scale = dims.scale;
  p.scale_log2 = dims.scale * kLog2e;
  p.m = mask;
  if (mask.nt == 0 || dims.B == 0 || dims.Hq == 0) return hipSuccess;
  const bool d64 = dims.D == 64;
  const dim3 gq(dims.Hq, mask.nt, dims.B), gk(dims.Hkv, mask.nt, dims.B);
  if (d64) hipLaunchKernelGGL(bwd_dq_f32_kernel<64>, gq, dim3(kThreads), 0, stream, p);
  else hipLaunchKernelGGL(bwd_dq_f32_kernel<128>, gq, dim3(kThreads), 0, stream, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  if (d64) hipLaunchKernelGGL(bwd_dkdv_f32_kernel<64>, gk, dim3(kThreads), 0, stream, p);
  else hipLaunchKernelGGL(bwd_dkdv_f32_kernel<128>, gk, dim3(kThreads), 0, stream, p);
  return hipGetLastError();
}

}  // namespace t2t
