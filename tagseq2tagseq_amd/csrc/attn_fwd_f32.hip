// Masked flash-attention forward for float32 inputs, gfx950 fp32 MFMA.
//
// The float32 form of the reference's math_attention
// (torch/_higher_order_ops/flex_attention.py:202-267): S = Q K^T * scale,
// P = softmax of the masked row, O = P V with P kept in float32 (the
// reference's P.to(dtype) is a no-op for float32), fully masked rows giving
// O = 0 and LSE = -inf.  Every product and sum is float32
// (v_mfma_f32_32x32x2_f32).
//
// It walks the same BlockMask lists and tile bitmaps as the bf16 kernel, with
// the same per-(b, query head, 128-query tile) work-groups, 64-key halves
// (the bf16 kernel's step at D = 64; its D = 128 form uses 32-key steps)
// double-buffered in LDS by direct global->LDS copies (a float32 row of D
// values is copied as a bf16 row of 2 D, so the copy units and row padding
// are the bf16 ones: pitch D + 4 floats) and lazy-rescaled online softmax in
// the log2 domain.  What differs is the operand mapping of the 2-deep fp32
// contraction, chosen so that every operand is a plain row-major LDS read:
//   S^T = K Q^T, k-step s pairs head dims s and s + D/2 (lane group g takes
//     d = g D/2 + s), so a lane's K and Q pieces are contiguous; keys in
//     natural order in the accumulator rows, queries in the lanes.
//   O^T += V^T P^T, k-step ks of a 32-key block takes the keys of
//     accumulator entry ks (key acc_row(ks, g) for lane group g), so P^T is
//     the S^T accumulator entry itself; output row m of tile dt is head dim
//     DT m + dt, so a lane's V piece for all DT tiles is one contiguous read.
#include "attn_kernels.h"

namespace t2t {

namespace {

struct FwdF32Params {
  const float* q; int64_t q_sb, q_sh, q_st;
  const float* k; int64_t k_sb, k_sh, k_st;
  const float* v; int64_t v_sb, v_sh, v_st;
  float* o; int64_t o_sb, o_sh, o_st;
  float* lse2;
  int B, Hq, Hkv, T;
  float scale_log2;
  MaskTables m;
};

typedef float f32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ f32x16 mfma32_f32(float a, float b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// Seed of a mixed 32-key block for keys in natural order: 0 where the pair
// is allowed, -inf where it is masked.  nw = ~w >> (4 g): entry i of lane
// group g is key acc_row(i, g) = 8 (i / 4) + 4 g + i % 4.
template <int I = 0>
__device__ __forceinline__ void mask_seed_fill(f32x16& c, uint32_t nw) {
  if constexpr (I < 16) {
    c[I] = __int_as_float(sbfe1_c<8 * (I >> 2) + (I & 3)>(nw) & (int)0xff800000);
    mask_seed_fill<I + 1>(c, nw);
  }
}

}  // namespace

template <int D>
__global__ __launch_bounds__(kThreads, 1) void attn_fwd_f32_kernel(FwdF32Params p) {
  constexpr int KS = D / 2;   // MFMA k-steps over the head dim
  constexpr int DT = D / 32;  // 32-row output tiles
  constexpr int P = D + 4;    // LDS row pitch (floats)
  using U = UnitDma<2 * D>;   // a float row of D = a bf16 row of 2 D
  constexpr int kUnit = U::kRows * P;
  static_assert(U::kRows * pitch<2 * D>() == 2 * kUnit, "fp32 unit = bf16 unit of 2 D");
  __shared__ __attribute__((aligned(16))) float k_lo[kUnit], k_hi[kUnit], v_lo[kUnit], v_hi[kUnit];
  __shared__ __attribute__((aligned(16))) uint32_t bits_lds[2][kTile * 4];

  const int h = blockIdx.x, b = blockIdx.z;
  const int tid = threadIdx.x, wave = uniform(tid >> 6), lane = tid & 63;
  const int g = lane >> 5, n = lane & 31;
  const int hk = h / (p.Hq / p.Hkv);
  const int mb = p.m.Bm > 1 ? b : 0;
  const int T = p.T, nt = p.m.nt;
  const int qt = uniform(p.m.row_order[(size_t)mb * nt + blockIdx.y]);
  const int q0 = qt * kTile;
  const int qloc = 32 * wave + n;
  const int qrow = q0 + qloc;
  const bool qvalid = qrow < T;
  const float c = p.scale_log2;

  // Q^T operand: lane (g, n) holds Q[qrow][g D/2 + s], s = 0 .. D/2 - 1.
  float qf[KS];
  {
    const float* qp = p.q + b * p.q_sb + h * p.q_sh + (int64_t)(qvalid ? qrow : 0) * p.q_st + g * KS;
#pragma unroll
    for (int s = 0; s < KS; s += 4) {
      const f32x4 x = *reinterpret_cast<const f32x4*>(qp + s);
#pragma unroll
      for (int e = 0; e < 4; ++e) qf[s + e] = qvalid ? x[e] : 0.f;
    }
  }

  const float* kbase = p.k + b * p.k_sb + hk * p.k_sh;
  const float* vbase = p.v + b * p.v_sb + hk * p.v_sh;
  int koff[U::kPerWave + 1], voff[U::kPerWave + 1];
#pragma unroll
  for (int j = 0; j < U::kPerWave; ++j) {
    koff[j] = unit_dma_offset<2 * D>(wave + kWaves * j, 2 * p.k_st, lane);
    voff[j] = unit_dma_offset<2 * D>(wave + kWaves * j, 2 * p.v_st, lane);
  }
  koff[U::kPerWave] = unit_dma_offset<2 * D>(U::kInsts - 1, 2 * p.k_st, lane);
  voff[U::kPerWave] = unit_dma_offset<2 * D>(U::kInsts - 1, 2 * p.v_st, lane);

  const size_t row = (size_t)mb * nt + qt;
  const int npart = uniform(p.m.kv_num[row]);
  const int nfull = uniform(p.m.full_kv_num[row]);
  const int ntiles = npart + nfull;
  const int32_t* pidx = p.m.kv_idx + row * nt;
  const int32_t* fidx = p.m.full_kv_idx + row * nt;
  const uint32_t* bits_row = p.m.tile_bits + (size_t)p.m.kv_bits_off[row] * kTileBitsWords;

  auto load_chunk = [&](int chunk) {
    const int it = 64 * chunk + lane;
    return it < npart ? pidx[it] : (it < ntiles ? fidx[it - npart] : 0);
  };
  int tiles_v = load_chunk(0);
  auto tile_of = [&](int it) { return __builtin_amdgcn_readlane(tiles_v, it & 63); };
  const auto krs = slice_rsrc(reinterpret_cast<const __bf16*>(kbase), 2 * p.k_st, T, 2 * D);
  const auto vrs = slice_rsrc(reinterpret_cast<const __bf16*>(vbase), 2 * p.v_st, T, 2 * D);
  const int k_row4 = (int)p.k_st * 4, v_row4 = (int)p.v_st * 4;
  // K and V rows [t0, t0 + 64) into one half's units (rows past T read zero).
  auto load_half = [&](float* kd, float* vd, int t0) {
    unit_dma<2 * D>(reinterpret_cast<__bf16*>(kd), krs, koff, t0 * k_row4, wave, 0);
    unit_dma<2 * D>(reinterpret_cast<__bf16*>(vd), vrs, voff, t0 * v_row4, wave, 1);
  };
  // bitmap of iteration it: KV tile kt, slot kv_bits_off + kt
  auto load_bits = [&](int it, int kt) {
    const bool has = it < npart;
    const auto rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint32_t*>(bits_row + (has ? (size_t)kt * kTileBitsWords : 0)), 0,
        has ? kTile * 16 : 0, 0x00020000);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        rs, (__attribute__((address_space(3))) void*)(&bits_lds[it & 1][(wave & 1) * 256]), 16,
        (wave & 1) * 1024 + lane * 16, 0, 0, 0);
  };

  f32x16 oacc[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) oacc[dt] = f32x16{};
  float m_ref = -INFINITY, l_run = 0.f;

  // One 64-key half (two 32-key blocks j): S^T = K Q^T (+ mask seed),
  // lazy-rescaled online softmax, O^T += V^T P^T.
  auto half_step = [&](const float* kt_lds, const float* vt_lds, uint32_t w0, uint32_t w1,
                       bool partial) {
    if (partial && __ballot((w0 | w1) != 0u) == 0ull) return;
    f32x16 st[2];
    if (partial && __ballot((w0 & w1) != ~0u) != 0ull) {
      mask_seed_fill(st[0], ~w0 >> (4 * g));
      mask_seed_fill(st[1], ~w1 >> (4 * g));
    } else {
      st[0] = f32x16{};
      st[1] = f32x16{};
    }
#pragma unroll
    for (int s4 = 0; s4 < KS; s4 += 4) {
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const f32x4 kf = *reinterpret_cast<const f32x4*>(kt_lds + (32 * j + n) * P + g * KS + s4);
#pragma unroll
        for (int e = 0; e < 4; ++e) st[j] = mfma32_f32(kf[e], qf[s4 + e], st[j]);
      }
    }
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int i = 0; i < 16; ++i) mx = fmaxf(mx, st[j][i]);
    mx = halves_max(mx);
    const bool move = (mx - m_ref) * c > 8.f;
    if (__ballot(move) != 0ull) {
      const float alpha = move ? fast_exp2((m_ref - mx) * c) : 1.f;
      l_run *= alpha;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) oacc[dt] *= alpha;
      m_ref = move ? mx : m_ref;
    }
    const float neg = m_ref == -INFINITY ? 0.f : -m_ref * c;
    float rs = 0.f;
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        st[j][i] = fast_exp2(fmaf(st[j][i], c, neg));
        rs += st[j][i];
      }
    l_run += halves_sum(rs);
    // O^T += V^T P^T: k-step ks of block j takes key 32 j + acc_row(ks, g).
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int ks = 0; ks < 16; ++ks) {
        const float* vr = vt_lds + (32 * j + acc_row(ks, g)) * P + DT * n;
        if constexpr (DT == 4) {
          const f32x4 vf = *reinterpret_cast<const f32x4*>(vr);
#pragma unroll
          for (int dt = 0; dt < DT; ++dt) oacc[dt] = mfma32_f32(vf[dt], st[j][ks], oacc[dt]);
        } else {
          const f32x2 vf = *reinterpret_cast<const f32x2*>(vr);
#pragma unroll
          for (int dt = 0; dt < DT; ++dt) oacc[dt] = mfma32_f32(vf[dt], st[j][ks], oacc[dt]);
        }
      }
  };

  int k0_next = ntiles > 0 ? tile_of(0) * kTile : 0;
  if (ntiles > 0) {
    load_half(k_lo, v_lo, k0_next);
    if (npart > 0) load_bits(0, k0_next / kTile);
  }
  for (int it = 0; it < ntiles; ++it) {
    const bool partial = it < npart;
    const int k0 = k0_next;
    dma_barrier();
    uint4 mbits = make_uint4(~0u, ~0u, ~0u, ~0u);
    if (partial) mbits = *reinterpret_cast<const uint4*>(&bits_lds[it & 1][qloc * 4]);
    load_half(k_hi, v_hi, k0 + 64);
    half_step(k_lo, v_lo, mbits.x, mbits.y, partial);

    dma_barrier();
    const bool more = it + 1 < ntiles;
    if (more) {
      if (((it + 1) & 63) == 0) tiles_v = load_chunk((it + 1) >> 6);
      k0_next = tile_of(it + 1) * kTile;
      load_half(k_lo, v_lo, k0_next);
      load_bits(it + 1, k0_next / kTile);
    }
    half_step(k_hi, v_hi, mbits.z, mbits.w, partial);
  }

  if (qvalid) {
    const float inv_l = l_run > 0.f ? 1.f / l_run : 0.f;
    float* op = p.o + b * p.o_sb + h * p.o_sh + (int64_t)qrow * p.o_st;
    // Output row m of tile dt is head dim DT m + dt.
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int d0 = DT * acc_row(i, g);
      if constexpr (DT == 4) {
        f32x4 w;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) w[dt] = oacc[dt][i] * inv_l;
        *reinterpret_cast<f32x4*>(op + d0) = w;
      } else {
        f32x2 w;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) w[dt] = oacc[dt][i] * inv_l;
        *reinterpret_cast<f32x2*>(op + d0) = w;
      }
    }
    if (g == 0)
      p.lse2[((size_t)b * p.Hq + h) * T + qrow] =
          l_run > 0.f ? m_ref * c + __log2f(l_run) : -INFINITY;
  }
}

hipError_t launch_attn_fwd_f32(const TensorView& q, const TensorView& k, const TensorView& v,
                               const TensorView& o, float* lse2, const AttnDims& dims,
                               const MaskTables& mask, hipStream_t stream) {
  FwdF32Params p;
  p.q = static_cast<const float*>(q.data); p.q_sb = q.sb; p.q_sh = q.sh; p.q_st = q.st;
  p.k = static_cast<const float*>(k.data); p.k_sb = k.sb; p.k_sh = k.sh; p.k_st = k.st;
  p.v = static_cast<const float*>(v.data); p.v_sb = v.sb; p.v_sh = v.sh; p.v_st = v.st;
  p.o = static_cast<float*>(o.data); p.o_sb = o.sb; p.o_sh = o.sh; p.o_st = o.st;
  p.lse2 = lse2;
  p.B = dims.B; p.Hq = dims.Hq; p.Hkv = dims.Hkv; p.T = dims.T;
  p.scale_log2 = dims.scale * kLog2e;
  p.m = mask;
  if (mask.nt == 0 || dims.B == 0 || dims.Hq == 0) return hipSuccess;
  dim3 grid(dims.Hq, mask.nt, dims.B);
  if (dims.D == 64)
    hipLaunchKernelGGL(attn_fwd_f32_kernel<64>, grid, dim3(kThreads), 0, stream, p);
  else
    hipLaunchKernelGGL(attn_fwd_f32_kernel<128>, grid, dim3(kThreads), 0, stream, p);
  return hipGetLastError();
}

}  // namespace t2t
