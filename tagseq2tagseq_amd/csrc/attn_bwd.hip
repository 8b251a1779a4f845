// Masked flash-attention backward, bf16 in / fp32 accumulate, gfx950 MFMA.
//
// Arithmetic of torch's sdpa_dense_backward
// (torch/_higher_order_ops/flex_attention.py:825-994):
//   P  = exp(S - LSE) on allowed pairs (0 elsewhere)
//   dV = P^T dO                       Delta = rowsum(O * dO)
//   dP = dO V^T                       dS = P * (dP - Delta)
//   dQ = dS K * scale                 dK = dS^T Q * scale
// with dK / dV summed over the query heads that share a KV head (GQA).
//
// Launches, none of them atomic (t2t_attn_bwd runs 3 then 2, with 3
// computing Delta for its rows; the separate phases run 1, 2, 3):
//   1. bwd_delta:  Delta per query row.
//   2. bwd_dkdv:   one work-group per (b, kv head, 128-key tile); walks the
//                  column's partial and full query tiles (q_num_blocks /
//                  q_indices, full_q_*) for every query head of the group and
//                  accumulates dK, dV in registers -- deterministic.  D = 128:
//                  bwd_dkdv_kernel; D = 64: bwd_dkdv_pair_kernel (two
//                  work-groups per CU, the work of a key group split between
//                  two waves).
//   3. bwd_dq:     one work-group per (b, query head, 128-query tile); walks
//                  the row's KV tiles and accumulates dQ in registers.
#include "attn_kernels.h"

namespace t2t {

namespace {

struct BwdParams {
  const __bf16* q; int64_t q_sb, q_sh, q_st;
  const __bf16* k; int64_t k_sb, k_sh, k_st;
  const __bf16* v; int64_t v_sb, v_sh, v_st;
  const __bf16* o; int64_t o_sb, o_sh, o_st;
  const __bf16* dout; int64_t do_sb, do_sh, do_st;
  __bf16* dq; int64_t dq_sb, dq_sh, dq_st;
  __bf16* dk; int64_t dk_sb, dk_sh, dk_st;
  __bf16* dv; int64_t dv_sb, dv_sh, dv_st;
  const float* lse2;  // [B][Hq][T], log2 domain of scaled scores
  float* delta;       // [B][Hq][T]
  int B, Hq, Hkv, T;
  float scale, scale_log2;
  int fuse_delta;  // dQ computes and writes Delta itself (kBwdDqDelta)
  MaskTables m;
};

// Stores a transposed 32 x 32 f32 accumulator block (rows = d, cols = token)
// scaled by `mul` as bf16 into out[token][d0 + d].
__device__ __forceinline__ void store_acc_t(__bf16* out_row, const f32x16& acc, int d0, int g,
                                            float mul) {
#pragma unroll
  for (int i = 0; i < 16; i += 4) {
    bf16x4 w4;
#pragma unroll
    for (int e = 0; e < 4; ++e) w4[e] = (__bf16)(acc[i + e] * mul);
    *reinterpret_cast<bf16x4*>(out_row + d0 + acc_row(i, g)) = w4;
  }
}

}  // namespace

// Delta[b, h, t] = sum_d O * dO.  D/8 lanes per row, 8 d-values per lane.
template <int D>
__global__ __launch_bounds__(kThreads) void bwd_delta_kernel(BwdParams p) {
  constexpr int kLanesPerRow = D / 8;
  constexpr int kRowsPerBlock = kThreads / kLanesPerRow;
  const int tid = threadIdx.x;
  const int sub = tid % kLanesPerRow;
  const int64_t rowid = (int64_t)blockIdx.x * kRowsPerBlock + tid / kLanesPerRow;
  const int64_t nrows = (int64_t)p.B * p.Hq * p.T;
  float acc = 0.f;
  if (rowid < nrows) {
    const int t = (int)(rowid % p.T);
    const int h = (int)((rowid / p.T) % p.Hq);
    const int b = (int)(rowid / ((int64_t)p.T * p.Hq));
    const bf16x8 ov = *reinterpret_cast<const bf16x8*>(p.o + b * p.o_sb + h * p.o_sh + (int64_t)t * p.o_st + 8 * sub);
    const bf16x8 gv = *reinterpret_cast<const bf16x8*>(p.dout + b * p.do_sb + h * p.do_sh + (int64_t)t * p.do_st + 8 * sub);
#pragma unroll
    for (int j = 0; j < 8; ++j) acc += (float)ov[j] * (float)gv[j];
  }
#pragma unroll
  for (int off = kLanesPerRow / 2; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
  if (rowid < nrows && sub == 0) p.delta[rowid] = acc;
}

// P and dS of a mixed dK/dV block in place (sacc = S - LSE / c -> P,
// dpacc = dP - Delta -> dS) for a lane whose bitmap word, shifted right by
// its lane group, is wg: P of a masked pair is cleared with the pair's
// sign-extended mask bit.
template <int I = 0>
__device__ __forceinline__ void keep_masked(f32x16& sacc, uint32_t wg, f32x16& dpacc, float c) {
  if constexpr (I < 16) {
    const float e = fast_exp2(sacc[I] * c);
    const float pv = __int_as_float(__float_as_int(e) & sbfe1_c<acc_tok_bit(I)>(wg));
    sacc[I] = pv;
    dpacc[I] = pv * dpacc[I];
    keep_masked<I + 1>(sacc, wg, dpacc, c);
  }
}

// The 16 accumulator rows of lane group g (rows 8 a + 4 g + 0..3) of a
// 32-row slot array, as four 16-byte reads -- the same reads for mixed and
// unmasked blocks.
__device__ __forceinline__ f32x16 acc_rows(const float* base, int g) {
  f32x16 r;
#pragma unroll
  for (int a = 0; a < 4; ++a) {
    const float4 x = *reinterpret_cast<const float4*>(base + 8 * a + 4 * g);
    r[4 * a] = x.x; r[4 * a + 1] = x.y; r[4 * a + 2] = x.z; r[4 * a + 3] = x.w;
  }
  return r;
}

constexpr int kDkdvWaves = 8;  // 4 key groups x 2 query blocks
constexpr int kDkdvThreads = 64 * kDkdvWaves;

// dK, dV for one (b, kv head, 128-key tile).  8 waves: wave (kw, qh) owns
// keys 32 kw .. 32 kw + 31.  Each query tile is consumed as two 64-query
// halves; in the phase of a half, wave (kw, qh) takes its queries
// 32 qh .. 32 qh + 31, and the two query blocks of a key group are summed
// through LDS at the end.  S = Q K^T and dP = dO V^T put the key in the lane
// and the query in the accumulator rows, so P and dS feed dV^T += dO^T P and
// dK^T += Q^T dS directly as B operands.
//
// K and V stay in LDS for the whole column.  Q, dO, LSE and Delta stream
// through LDS per 64-query half: while the waves compute on one half, the
// other half's units are refilled by direct global->LDS copies issued right
// after the barrier that retired them (the next (head, tile) item's first
// half is fetched during the current item's second half), so each copy has
// one phase of compute to land in.
template <int D>
__global__ __launch_bounds__(kDkdvThreads, 1) void bwd_dkdv_kernel(BwdParams p) {
  constexpr int KS = D / 16;
  constexpr int DT = D / 32;
  using U = UnitDma<D, kDkdvWaves>;
  constexpr int kUnit = U::kRows * pitch<D>();
  // (16-byte aligned: the end of the kernel reuses them as float4 and row buffers)
  __shared__ __align__(16) __bf16 k_s[kTile * pitch<D>()], v_s[kTile * pitch<D>()];
  __shared__ __align__(16) __bf16 q_lo[kUnit], q_hi[kUnit], do_lo[kUnit], do_hi[kUnit];
  // LSE (log2 domain) and Delta of a half, slot 32 blk + m = query
  // 32 blk + tok_perm(m) (accumulator-row order).
  // (16-byte aligned: rows are read four at a time)
  __shared__ __align__(16) float lse_lo[64], lse_hi[64], dl_lo[64], dl_hi[64];

  const int hk = blockIdx.x, b = blockIdx.z;
  const int tid = threadIdx.x, wave = uniform(tid >> 6), lane = tid & 63;
  // Waves w and w + 4 share a SIMD; pairing key groups two apart there keeps
  // both busy on tiles whose upper key groups are masked for a whole half
  // (the causal diagonal), where the same key group would leave it idle.
  const int qh = wave >> 2, kw = (wave + 2 * qh) & 3;
  const int g = lane >> 5, n = lane & 31;
  const int G = p.Hq / p.Hkv;
  const int mb = p.m.Bm > 1 ? b : 0;
  const int T = p.T, nt = p.m.nt;
  const int kt = uniform(p.m.col_order[(size_t)mb * nt + blockIdx.y]);
  const int k0 = kt * kTile;
  const int kloc = 32 * kw + n;
  const float c = p.scale_log2;

  const size_t col = (size_t)mb * nt + kt;
  const int npart = uniform(p.m.q_num[col]);
  const int nfull = uniform(p.m.full_q_num[col]);
  const int nq = npart + nfull;
  const int nu = G * nq;  // (query head, query tile) items
  const int32_t* pidx = p.m.q_idx + col * nt;
  const int32_t* fidx = p.m.full_q_idx + col * nt;
  const int32_t* pslot = p.m.q_bits_slot + col * nt;
  const uint32_t* bits_col = p.m.tile_bits + kTile * 4 + kloc * 4;

  int qoff[U::kPerWave + 1], ooff[U::kPerWave + 1];
#pragma unroll
  for (int j = 0; j < U::kPerWave; ++j) {
    qoff[j] = unit_dma_offset<D>(wave + kDkdvWaves * j, p.q_st, lane);
    ooff[j] = unit_dma_offset<D>(wave + kDkdvWaves * j, p.do_st, lane);
  }
  qoff[U::kPerWave] = unit_dma_offset<D>(U::kInsts - 1, p.q_st, lane);
  ooff[U::kPerWave] = unit_dma_offset<D>(U::kInsts - 1, p.do_st, lane);
  const int lrow = 32 * (lane >> 5) + tok_perm(lane & 31);  // query of LSE / Delta slot `lane`

  // Query-tile list of the column, 64 entries per chunk (lane j: entry
  // 64 * chunk + j), read back with readlane; reloaded when a chunk changes.
  int chunk = 0;
  auto load_chunk = [&](int ch) {
    const int it = 64 * ch + lane;
    return make_int2(it < npart ? pidx[it] : (it < nq ? fidx[it - npart] : 0),
                     it < npart ? pslot[it] : 0);
  };
  int2 list_v = load_chunk(0);

  // K and V of the key tile stay in LDS; lane (g, n) reads row kloc as the B
  // operand (k = d, n = key) of S = Q K^T and dP = dO V^T.  They travel as
  // direct global->LDS copies (two 64-row units each) issued after the query
  // tile list and before the first Q / dO half, so the three are in flight
  // together; the first barrier of the loop publishes them.
  {
    int koff[U::kPerWave + 1], voff[U::kPerWave + 1];
#pragma unroll
    for (int j = 0; j < U::kPerWave; ++j) {
      koff[j] = unit_dma_offset<D>(wave + kDkdvWaves * j, p.k_st, lane);
      voff[j] = unit_dma_offset<D>(wave + kDkdvWaves * j, p.v_st, lane);
    }
    koff[U::kPerWave] = unit_dma_offset<D>(U::kInsts - 1, p.k_st, lane);
    voff[U::kPerWave] = unit_dma_offset<D>(U::kInsts - 1, p.v_st, lane);
    const auto krs = slice_rsrc(p.k + b * p.k_sb + hk * p.k_sh, p.k_st, T, D);
    const auto vrs = slice_rsrc(p.v + b * p.v_sb + hk * p.v_sh, p.v_st, T, D);
    const int kr2 = (int)p.k_st * 2, vr2 = (int)p.v_st * 2;
    unit_dma<D, kDkdvWaves>(k_s, krs, koff, k0 * kr2, wave, 4);
    unit_dma<D, kDkdvWaves>(k_s + kUnit, krs, koff, (k0 + 64) * kr2, wave, 5);
    unit_dma<D, kDkdvWaves>(v_s, vrs, voff, k0 * vr2, wave, 6);
    unit_dma<D, kDkdvWaves>(v_s + kUnit, vrs, voff, (k0 + 64) * vr2, wave, 7);
  }
  auto entry = [&](int it) {
    if ((it >> 6) != chunk) {
      chunk = it >> 6;
      list_v = load_chunk(chunk);
    }
    return make_int2(__builtin_amdgcn_readlane(list_v.x, it & 63),
                     __builtin_amdgcn_readlane(list_v.y, it & 63));
  };

  // Copies of query rows [r0, r0 + 64) of head h into one half's units
  // (Q + LSE, dO + Delta).  LSE and Delta go one dword per lane, gathered
  // into accumulator-row order; rows at or past T read zero.  Both are
  // staged as the starting values of the score and dP chains, -LSE / c and
  // -Delta: waves 2 and 3 load them into a register and store the seeds
  // into the half's slots just before the barrier that publishes the half
  // (publish_rows), by which time the loads have long landed.
  uint32_t row_pend = 0u;     // wave 2: LSE, wave 3: Delta bits of the half in flight
  float* row_dst = nullptr;   // and its slot array (null: nothing pending)
  const float inv_c = 1.f / c;
  auto load_q_part = [&](__bf16* qd, float* ld, int h, int r0) {
    const auto qrs = slice_rsrc(p.q + b * p.q_sb + h * p.q_sh, p.q_st, T, D);
    unit_dma<D, kDkdvWaves>(qd, qrs, qoff, r0 * (int)p.q_st * 2, wave, 0);
    const auto lrs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(p.lse2 + ((size_t)b * p.Hq + h) * T), 0, T * 4, 0x00020000);
    if (wave == 2) {
      row_pend = __builtin_amdgcn_raw_buffer_load_b32(lrs, (r0 + lrow) * 4, 0, 0);
      row_dst = ld;
    }
  };
  auto load_do_part = [&](__bf16* dd, float* dld, int h, int r0) {
    const auto drs = slice_rsrc(p.dout + b * p.do_sb + h * p.do_sh, p.do_st, T, D);
    unit_dma<D, kDkdvWaves>(dd, drs, ooff, r0 * (int)p.do_st * 2, wave, 1);
    const auto drs2 = __builtin_amdgcn_make_buffer_rsrc(p.delta + ((size_t)b * p.Hq + h) * T, 0,
                                                        T * 4, 0x00020000);
    if (wave == 3) {
      row_pend = __builtin_amdgcn_raw_buffer_load_b32(drs2, (r0 + lrow) * 4, 0, 0);
      row_dst = dld;
    }
  };
  auto publish_rows = [&]() {
    if (row_dst != nullptr) {  // waves 2 and 3 only
      const float x = __uint_as_float(row_pend);
      row_dst[lane] = wave == 2 ? -x * inv_c : -x;
      row_dst = nullptr;
    }
  };
  // The lane's bitmap words (its key, queries 32 w .. 32 w + 31, w = 0..3)
  // of a partial tile; full tiles carry all ones.
  auto tile_words = [&](int2 e, bool partial) {
    uint4 w = make_uint4(~0u, ~0u, ~0u, ~0u);
    if (partial) w = *reinterpret_cast<const uint4*>(bits_col + (size_t)e.y * kTileBitsWords);
    return w;
  };

  f32x16 dkacc[DT], dvacc[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) { dkacc[dt] = f32x16{}; dvacc[dt] = f32x16{}; }

  // One 32-query x 32-key block: rows 32 qh .. 32 qh + 31 of a half's units.
  auto block = [&](const __bf16* qu, const __bf16* du, const float* lu, const float* dlu,
                   uint32_t w, bool partial) {
    if (partial && __ballot(w != 0u) == 0ull) return;
    const bool mixed = partial && __ballot(w != ~0u) != 0ull;
    const int rb = 32 * qh;
    // Chains start from -LSE / c and -Delta and end at S - LSE / c, dP - Delta.
    f32x16 sacc = acc_rows(lu + rb, g);
    f32x16 dpacc = acc_rows(dlu + rb, g);
    __builtin_amdgcn_s_setprio(1);  // MFMA runs at raised wave priority
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const bf16x8 qa = lds_row8<D>(qu, rb + tok_perm(n), 16 * s + 8 * g);
      const bf16x8 da = lds_row8<D>(du, rb + tok_perm(n), 16 * s + 8 * g);
      const bf16x8 kb = lds_row8<D>(k_s, kloc, 16 * s + 8 * g);
      const bf16x8 vb = lds_row8<D>(v_s, kloc, 16 * s + 8 * g);
      sacc = mfma32(qa, kb, sacc);
      dpacc = mfma32(da, vb, dpacc);
    }
    if constexpr (D == 64) {
      // The seeds and the operand reads of the first two MFMAs first, then
      // each MFMA followed by the reads of the one two ahead (3 % faster at
      // D = 64; at D = 128 the compiler's own order is faster).
      __builtin_amdgcn_sched_group_barrier(0x100, 12, 0);
#pragma unroll
      for (int i = 0; i < 2 * KS - 2; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
    }
    __builtin_amdgcn_s_setprio(0);
    // Masked pairs of a mixed block: P is cleared by and-ing its bits with
    // the pair's sign-extended mask bit, after the exponential.  Only a
    // mixed block can hold a fully masked row (LSE = -inf), whose
    // exp2(+inf) is cleared the same way; every other row has a finite LSE.
    if (mixed) {
      keep_masked(sacc, w >> g, dpacc, c);
    } else {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const float pv = fast_exp2(sacc[i] * c);
        sacc[i] = pv;                  // P
        dpacc[i] = pv * dpacc[i];      // dS
      }
    }
    // dV^T += dO^T P, dK^T += Q^T dS (contraction over the 32 queries).
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int h2 = 0; h2 < 2; ++h2) {
      const bf16x8 pb = pack_half(sacc, h2);
      const bf16x8 sb = pack_half(dpacc, h2);
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const bf16x8 doa = lds_col8<D>(du, rb + 16 * h2, 32 * dt, lane);
        const bf16x8 qa = lds_col8<D>(qu, rb + 16 * h2, 32 * dt, lane);
        dvacc[dt] = mfma32(doa, pb, dvacc[dt]);
        dkacc[dt] = mfma32(qa, sb, dkacc[dt]);
      }
    }
    if constexpr (D == 64) {
      // transpose reads one MFMA ahead
      __builtin_amdgcn_sched_group_barrier(0x100, 4, 1);
#pragma unroll
      for (int i = 0; i < 4 * DT - 2; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 1);
      }
      __builtin_amdgcn_sched_group_barrier(0x008, 2, 1);
    }
    __builtin_amdgcn_s_setprio(0);
  };

  int2 e_next = make_int2(0, 0);
  uint4 wb = make_uint4(~0u, ~0u, ~0u, ~0u);
  if (nu > 0) {
    e_next = entry(0);
    load_q_part(q_lo, lse_lo, hk * G, e_next.x * kTile);
    load_do_part(do_lo, dl_lo, hk * G, e_next.x * kTile);
    wb = tile_words(e_next, 0 < npart);
  }
  for (int u = 0, hh = 0, it = 0; u < nu; ++u) {
    const int h = hk * G + hh;
    const int q0 = e_next.x * kTile;
    const bool partial = it < npart;
    // Query rows [q0, q0 + 64): their units have landed; the other half's
    // units are free again.
    publish_rows();
    dma_barrier();
    load_q_part(q_hi, lse_hi, h, q0 + 64);
    load_do_part(do_hi, dl_hi, h, q0 + 64);
    block(q_lo, do_lo, lse_lo, dl_lo, qh ? wb.y : wb.x, partial);

    // Query rows [q0 + 64, q0 + 128); the first half's units are free again.
    publish_rows();
    dma_barrier();
    if (++it == nq) { it = 0; ++hh; }
    uint4 wn = wb;
    const bool more = u + 1 < nu;
    const int hn = hk * G + hh;
    if (more) {
      e_next = entry(it);
      load_q_part(q_lo, lse_lo, hn, e_next.x * kTile);
      load_do_part(do_lo, dl_lo, hn, e_next.x * kTile);
      wn = tile_words(e_next, it < npart);
    }
    block(q_hi, do_hi, lse_hi, dl_hi, qh ? wb.w : wb.z, partial);
    wb = wn;
  }

  // Sum the two query blocks of each key group and store the tile's dK and
  // dV.  The waves of a key group swap halves of their partials: (kw, 1)
  // hands over its dK partial and (kw, 0) its dV partial (16 KiB per wave,
  // one float4 per lane and step, in eight 16 KiB regions over the K / V
  // tiles and the Q / dO units, all free after the loop), so (kw, 0) sums
  // dK and (kw, 1) dV.  The sums go to LDS as bf16 rows of the tile (dK over
  // the K tile, dV over the V tile, padded pitch), and all eight waves then
  // store the 128 rows of each as whole rows, 16 bytes per lane -- instead
  // of every lane writing 16-byte pieces of its own key's row.
  {
    static_assert(DT * 16 * 64 * sizeof(float) <= kUnit * sizeof(__bf16), "a region fits a unit");
    static_assert(2 * DT * 16 * 64 * sizeof(float) <= kTile * pitch<D>() * sizeof(__bf16),
                  "two regions fit a tile");
    constexpr int kRegion = DT * 16 * 64;  // floats
    auto region = [&](int r) {            // r < 4: dK partial of key group r, else dV of r - 4
      float* base = r < 2 ? reinterpret_cast<float*>(k_s) + r * kRegion
                  : r < 4 ? reinterpret_cast<float*>(v_s) + (r - 2) * kRegion
                  : reinterpret_cast<float*>(r == 4 ? q_lo : r == 5 ? q_hi : r == 6 ? do_lo : do_hi);
      return reinterpret_cast<float4*>(base);
    };
    dma_barrier();
    {
      float4* out = region(qh == 1 ? kw : 4 + kw);
      const f32x16* give = qh == 1 ? dkacc : dvacc;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int a = 0; a < 4; ++a)
          out[(dt * 4 + a) * 64 + lane] = make_float4(give[dt][4 * a], give[dt][4 * a + 1],
                                                      give[dt][4 * a + 2], give[dt][4 * a + 3]);
    }
    __syncthreads();
    f32x16* mine = qh == 0 ? dkacc : dvacc;
    {
      const float4* in = region(qh == 0 ? kw : 4 + kw);
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int a = 0; a < 4; ++a) {
          const float4 x = in[(dt * 4 + a) * 64 + lane];
          mine[dt][4 * a] += x.x; mine[dt][4 * a + 1] += x.y;
          mine[dt][4 * a + 2] += x.z; mine[dt][4 * a + 3] += x.w;
        }
    }
    __syncthreads();
    {
      __bf16* rows = qh == 0 ? k_s : v_s;  // bf16 row kloc of dK (qh 0) or dV (qh 1)
      const float mul = qh == 0 ? p.scale : 1.f;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int a = 0; a < 4; ++a) {
          bf16x4 w4;
#pragma unroll
          for (int e = 0; e < 4; ++e) w4[e] = (__bf16)(mine[dt][4 * a + e] * mul);
          *reinterpret_cast<bf16x4*>(rows + kloc * pitch<D>() + 32 * dt + acc_row(4 * a, g)) = w4;
        }
    }
    __syncthreads();
    constexpr int kChunks = D / 8;  // 16-byte pieces per row
    __bf16* dkp = p.dk + b * p.dk_sb + hk * p.dk_sh;
    __bf16* dvp = p.dv + b * p.dv_sb + hk * p.dv_sh;
#pragma unroll
    for (int j = 0; j < kTile * kChunks / kDkdvThreads; ++j) {
      const int c = tid + kDkdvThreads * j;
      const int r = c / kChunks, ch = c % kChunks;
      if (k0 + r < T) {
        const int64_t row = k0 + r;
        *reinterpret_cast<uint4*>(dkp + row * p.dk_st + 8 * ch) =
            *reinterpret_cast<const uint4*>(k_s + r * pitch<D>() + 8 * ch);
        *reinterpret_cast<uint4*>(dvp + row * p.dv_st + 8 * ch) =
            *reinterpret_cast<const uint4*>(v_s + r * pitch<D>() + 8 * ch);
      }
    }
  }
}

// P of a mixed block in place: P of a masked pair cleared with the pair's
// sign-extended mask bit (wg: the lane's bitmap word shifted right by its
// lane group).
template <int I = 0>
__device__ __forceinline__ void masked_clear(f32x16& pacc, uint32_t wg) {
  if constexpr (I < 16) {
    pacc[I] = __int_as_float(__float_as_int(pacc[I]) & sbfe1_c<acc_tok_bit(I)>(wg));
    masked_clear<I + 1>(pacc, wg);
  }
}

constexpr int kPairWaves = 8;  // 4 key groups x (P / dV wave, dS / dK wave)

// dK, dV at D = 64 for one (b, kv head, 128-key tile), two work-groups per
// CU, with the work of a key group split between two waves:
//   P wave:  S = Q K^T, P = exp(S - LSE) (masked pairs cleared), dV^T += dO^T P
//   dS wave: dP = dO V^T, dS = P (dP - Delta),                dK^T += Q^T dS
// Each wave holds its key group's K row (P wave) or V row (dS wave) in
// registers for the whole column and its own accumulator (dV or dK, 32
// registers), so a key group's dK and dV are complete in one wave each, the
// end of the kernel has no reduction, and the kernel fits 128 registers and
// 77.5 KiB of LDS -- two work-groups per CU, whose phases hide each other's
// copies and barriers (the single-work-group form at D = 64, and this
// kernel's D = 128 form, which holds one work-group per CU, measure slower
// than bwd_dkdv_kernel).  Each query tile is consumed as two 64-query
// halves, both 32-query blocks of a half by each wave; a half is one phase:
//   P waves:  S, P -> LDS  | dV, then the copies of the half two ahead
//   dS waves: dP           | P <- LDS, dS, dK
// with a barrier at the bar (P written to LDS as the bf16 MFMA operand it
// already is) and one at the end.  The halves of a phase overlap across the
// two waves of a SIMD (the P wave's exponentials with the dS wave's dP
// chain, the dS wave's dS with the P wave's dV).  Q, dO, LSE and Delta (in
// accumulator-row order) and the column bitmap words travel by direct
// global->LDS copies into three buffers, issued two phases ahead into the
// buffer freed at the start of the phase, so every copy has a whole phase
// to land in; the end barrier waits only for the copies older than the
// phase's own.
template <int D>
__global__ __launch_bounds__(kPairWaves * 64) __attribute__((amdgpu_waves_per_eu(4, 4)))
void bwd_dkdv_pair_kernel(BwdParams p) {
  static_assert(D == 64, "two work-groups per CU fit at D = 64 only");
  constexpr int KS = D / 16;
  constexpr int DT = D / 32;
  using UC = UnitDma<D, 4>;  // unit copies split over the four P waves
  constexpr int KP = UC::kPerWave;
  constexpr int kUnit = UC::kRows * pitch<D>();
  // Three buffers of each kind: the phase's half, the next one landing, the
  // one after being issued.  (16-byte aligned: the end of the kernel reuses
  // the Q and dO units as row buffers, 128 rows over the first two units)
  __shared__ __align__(16) __bf16 q_s[3 * kUnit], o_s[3 * kUnit];
  // LSE (log2 domain) and Delta of a half, slot 32 blk + m = query 32 blk +
  // tok_perm(m) (accumulator-row order); read four at a time.
  __shared__ __align__(16) float l0[64], l1[64], l2[64], e0[64], e1[64], e2[64];
  // Column bitmap words of the half's tile: key k's four words (queries
  // 32 w .. 32 w + 31 of the tile, w = 0..3).
  __shared__ __align__(16) uint4 m0[kTile], m1[kTile], m2[kTile];
  // P of each P wave for the dS wave of its key group, [key group][query
  // block][entry half][lane].
  __shared__ __align__(16) bf16x8 p_s[4 * 2 * 2 * 64];
  static_assert(kTile * pitch<D>() <= 2 * kUnit, "the end's row tiles fit two units");

  auto qbuf = [&](auto i) -> __bf16* { return q_s + decltype(i)::value * kUnit; };
  auto obuf = [&](auto i) -> __bf16* { return o_s + decltype(i)::value * kUnit; };
  auto lbuf = [&](auto i) -> float* {
    if constexpr (decltype(i)::value == 0) return l0;
    else if constexpr (decltype(i)::value == 1) return l1;
    else return l2;
  };
  auto ebuf = [&](auto i) -> float* {
    if constexpr (decltype(i)::value == 0) return e0;
    else if constexpr (decltype(i)::value == 1) return e1;
    else return e2;
  };
  auto mbuf = [&](auto i) -> uint4* {
    if constexpr (decltype(i)::value == 0) return m0;
    else if constexpr (decltype(i)::value == 1) return m1;
    else return m2;
  };

  const int hk = blockIdx.x, b = blockIdx.z;
  const int tid = threadIdx.x, wave = uniform(tid >> 6), lane = tid & 63;
  const bool ds_wave = wave >= 4;
  // Waves w and w + 4 share a SIMD: SIMD s runs the P wave of key group s
  // and the dS wave of key group 3 - s, so that a SIMD's load is the work of
  // two key groups from opposite ends of the tile, which evens out tiles
  // whose allowed pairs sit in some key groups only (document boundaries,
  // the causal diagonal).
  const int kw = ds_wave ? 3 - (wave & 3) : (wave & 3);
  const int g = lane >> 5, n = lane & 31;
  const int G = p.Hq / p.Hkv;
  const int mb = p.m.Bm > 1 ? b : 0;
  const int T = p.T, nt = p.m.nt;
  const int kt = uniform(p.m.col_order[(size_t)mb * nt + blockIdx.y]);
  const int k0 = kt * kTile;
  const int kloc = 32 * kw + n;
  const float c = p.scale_log2;

  const size_t col = (size_t)mb * nt + kt;
  const int npart = uniform(p.m.q_num[col]);
  const int nfull = uniform(p.m.full_q_num[col]);
  const int nq = npart + nfull;
  const int nu = G * nq;  // (query head, query tile) items
  const int32_t* pidx = p.m.q_idx + col * nt;
  const int32_t* fidx = p.m.full_q_idx + col * nt;
  const int32_t* pslot = p.m.q_bits_slot + col * nt;
  const uint32_t* bits_tiles = p.m.tile_bits + kTile * 4;  // column-major halves

  // P wave cw copies instructions cw, cw + 4, ... of the Q and dO units, and
  // one more each: the Q unit's last (cw 0), the dO unit's last (cw 1), the
  // LSE row and the bitmap words of keys 0..63 (cw 2), the Delta row and
  // those of keys 64..127 (cw 3).
  const int cw = wave & 3;
  int qoff[KP + 1], ooff[KP + 1];
#pragma unroll
  for (int j = 0; j < KP; ++j) {
    qoff[j] = unit_dma_offset<D>(cw + 4 * j, p.q_st, lane);
    ooff[j] = unit_dma_offset<D>(cw + 4 * j, p.do_st, lane);
  }
  qoff[KP] = unit_dma_offset<D>(UC::kInsts - 1, p.q_st, lane);
  ooff[KP] = unit_dma_offset<D>(UC::kInsts - 1, p.do_st, lane);
  const int lrow4 = 4 * (32 * (lane >> 5) + tok_perm(lane & 31));  // LSE / Delta slot `lane`

  // Query-tile list of the column, 64 entries per chunk (lane j: entry
  // 64 * chunk + j), read back with readlane; reloaded when a chunk changes.
  int chunk = 0;
  auto load_chunk = [&](int ch) __attribute__((always_inline)) {
    const int it = 64 * ch + lane;
    return make_int2(it < npart ? pidx[it] : (it < nq ? fidx[it - npart] : 0),
                     it < npart ? pslot[it] : 0);
  };
  int2 list_v = load_chunk(0);
  // (the wait inside the reload keeps the compiler from waiting -- for every
  // copy in flight -- before each readlane)
  auto entry = [&](int it) __attribute__((always_inline)) {
    if ((it >> 6) != chunk) {
      chunk = it >> 6;
      list_v = load_chunk(chunk);
      __builtin_amdgcn_s_waitcnt(0);
    }
    return make_int2(__builtin_amdgcn_readlane(list_v.x, it & 63),
                     __builtin_amdgcn_readlane(list_v.y, it & 63));
  };

  // The lane's key row of K (P waves) or V (dS waves): the B operand (k = d,
  // n = key) of S = Q K^T or dP = dO V^T at every k-step, loaded once.  Rows
  // at or past T read zero.
  bf16x8 kv[KS];
  {
    const __bf16* base = ds_wave ? p.v + b * p.v_sb + hk * p.v_sh : p.k + b * p.k_sb + hk * p.k_sh;
    const int64_t st = ds_wave ? p.v_st : p.k_st;
    const auto rs = slice_rsrc(base, st, T, D);
    const int off = (int)((((int64_t)(k0 + kloc)) * st + 8 * g) * 2);
#pragma unroll
    for (int s = 0; s < KS; ++s)
      kv[s] = __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(rs, off + 32 * s, 0, 0));
  }

  // Buffer resources of the current query head's Q and dO slices and LSE
  // and Delta rows, rebuilt only when the walk moves to the next head.
  int hh_n = 0;
  u32x4 rq, ro, rl, re;
  auto head_rsrc = [&]() __attribute__((always_inline)) {
    const int h = hk * G + hh_n;
    rq = slice_words(p.q + b * p.q_sb + h * p.q_sh, p.q_st, T, D);
    ro = slice_words(p.dout + b * p.do_sb + h * p.do_sh, p.do_st, T, D);
    rl = rsrc_words(p.lse2 + ((size_t)b * p.Hq + h) * T, (int64_t)T * 4);
    re = rsrc_words(p.delta + ((size_t)b * p.Hq + h) * T, (int64_t)T * 4);
  };
  head_rsrc();
  // Halves h = 0 .. 2 nu - 1: item h / 2, rows 64 (h % 2) of its tile.  The
  // item of the latest half advanced to:
  int it_n = 0;
  int2 e_n = make_int2(0, 0);
  auto advance = [&](int h) __attribute__((always_inline)) {
    if ((h & 1) == 0 && h > 0 && ++it_n == nq) {
      it_n = 0;
      ++hh_n;
      head_rsrc();
    }
    if ((h & 1) == 0) e_n = entry(it_n);
  };
  struct HalfCopies {
    u32x4 q, o, l, e, m;  // buffer resources: Q, dO slices, LSE, Delta rows, bitmap
    int q_ro, o_ro, r4;   // byte offsets of the half's first row
  };
  // Copies of the latest half advanced to (rows r0 .. r0 + 63 of head h).
  auto half_copies = [&](int h_rows) __attribute__((always_inline)) {
    const int r0 = e_n.x * kTile + 64 * (h_rows & 1);
    const bool partial = it_n < npart;
    HalfCopies hc;
    hc.q = rq;
    hc.o = ro;
    hc.l = rl;
    hc.e = re;
    // full tiles have no bitmap: an empty range (the copies write zeros)
    hc.m = rsrc_words(bits_tiles + (size_t)(partial ? e_n.y : 0) * kTileBitsWords,
                      partial ? kTile * 16 : 0);
    hc.q_ro = uniform(r0 * (int)p.q_st * 2);
    hc.o_ro = uniform(r0 * (int)p.do_st * 2);
    hc.r4 = uniform(r0 * 4);
    return hc;
  };
  // A P wave's copies of one half into buffer y: 2 KP + 1 (cw < 2) or
  // 2 KP + 2 (cw >= 2) loads.
  // (LDS addresses as integers: constants plus the wave's offset)
  const uint32_t q_u = lds_u32(q_s), o_u = lds_u32(o_s), cw_u = (uint32_t)cw * 1024u;
  auto issue = [&](auto y, const HalfCopies& hc) __attribute__((always_inline)) {
    constexpr uint32_t yo = decltype(y)::value * kUnit * 2;  // bytes
#pragma unroll
    for (int j = 0; j < KP; ++j) {
      lds_copy16_m0(uniform(q_u + yo + cw_u + 4096u * j), qoff[j] + hc.q_ro, hc.q);
      lds_copy16_m0(uniform(o_u + yo + cw_u + 4096u * j), ooff[j] + hc.o_ro, hc.o);
    }
    constexpr uint32_t last = (UC::kInsts - 1) * 1024u;
    if (cw == 0) {
      lds_copy16_m0(q_u + yo + last, qoff[KP] + hc.q_ro, hc.q);
    } else if (cw == 1) {
      lds_copy16_m0(o_u + yo + last, ooff[KP] + hc.o_ro, hc.o);
    } else if (cw == 2) {
      lds_copy4_m0(lds_u32(lbuf(y)), hc.r4 + lrow4, hc.l);
      lds_copy16_m0(lds_u32(mbuf(y)), 16 * lane, hc.m);
    } else {
      lds_copy4_m0(lds_u32(ebuf(y)), hc.r4 + lrow4, hc.e);
      lds_copy16_m0(lds_u32(mbuf(y)) + 1024u, 1024 + 16 * lane, hc.m);
    }
  };
  // End of a phase: the P waves keep this phase's copies in flight.
  auto end_barrier = [&]() __attribute__((always_inline)) {
    if (ds_wave) vm_barrier<0>();
    else if (cw < 2) vm_barrier<2 * KP + 1>();
    else vm_barrier<2 * KP + 2>();
  };
  // The bar inside a phase: P written.
  auto mid_barrier = [&]() __attribute__((always_inline)) {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  };

  // P waves: dV^T; dS waves: dK^T (rows d, lane = key).
  f32x16 acc[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) acc[dt] = f32x16{};

  // The lane's bitmap words of the half in buffer i (all ones on full tiles).
  auto words = [&](auto i, bool partial, int h) __attribute__((always_inline)) {
    uint2 w2 = make_uint2(~0u, ~0u);
    if (partial) {
      const uint4 w = mbuf(i)[kloc];
      w2 = (h & 1) ? make_uint2(w.z, w.w) : make_uint2(w.x, w.y);
    }
    return w2;
  };

  // One phase on the half in buffer x (compile time), copies into buffer y.
  auto run = [&](auto dsw) __attribute__((always_inline)) {
    constexpr bool kDs = decltype(dsw)::value;
    const int nh = 2 * nu;
    bool pf0 = false, pf1 = false, pf2 = false;  // partial tile of the half in buffer 0 / 1 / 2
    auto set_pf = [&](auto y, bool v) __attribute__((always_inline)) {
      if constexpr (decltype(y)::value == 0) pf0 = v;
      else if constexpr (decltype(y)::value == 1) pf1 = v;
      else pf2 = v;
    };
    auto get_pf = [&](auto x) __attribute__((always_inline)) {
      if constexpr (decltype(x)::value == 0) return pf0;
      else if constexpr (decltype(x)::value == 1) return pf1;
      else return pf2;
    };
    auto phase = [&](auto x, auto y, int k) __attribute__((always_inline)) {
      const uint2 w2 = words(x, get_pf(x), k);
      const __bf16* qu = qbuf(x);
      const __bf16* du = obuf(x);
      if constexpr (!kDs) {
        // S, P -> LDS
        const float* lu = lbuf(x);
        bf16x8 pa[2], pb[2];
#pragma unroll
        for (int blk = 0; blk < 2; ++blk) {
          const uint32_t w = blk ? w2.y : w2.x;
          if (__ballot(w != 0u) == 0ull) continue;
          const bool mixed = __ballot(w != ~0u) != 0ull;
          const int rb = 32 * blk;
          // every operand of the chain read first (the compiler otherwise
          // reads each into the same registers right before its MFMA)
          bf16x8 opd[KS];
#pragma unroll
          for (int s = 0; s < KS; ++s) opd[s] = lds_row8<D>(qu, rb + tok_perm(n), 16 * s + 8 * g);
          f32x16 sacc;
          __builtin_amdgcn_s_setprio(1);
#pragma unroll
          for (int s = 0; s < KS; ++s) sacc = mfma32(opd[s], kv[s], s ? sacc : f32x16{});
          __builtin_amdgcn_s_setprio(0);
          const f32x16 lse = acc_rows(lu + rb, g);
#pragma unroll
          for (int e = 0; e < 16; ++e) sacc[e] = fast_exp2(fmaf(sacc[e], c, -lse[e]));
          if (mixed) masked_clear(sacc, w >> g);
          pa[blk] = pack_half(sacc, 0);
          pb[blk] = pack_half(sacc, 1);
          bf16x8* dst = p_s + ((kw * 2 + blk) * 2) * 64 + lane;
          dst[0] = pa[blk];
          dst[64] = pb[blk];
        }
        mid_barrier();
        // dV^T += dO^T P
#pragma unroll
        for (int blk = 0; blk < 2; ++blk) {
          const uint32_t w = blk ? w2.y : w2.x;
          if (__ballot(w != 0u) == 0ull) continue;
          const int rb = 32 * blk;
          bf16x8 opd[2 * DT];
#pragma unroll
          for (int h2 = 0; h2 < 2; ++h2)
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) opd[h2 * DT + dt] = lds_col8<D>(du, rb + 16 * h2, 32 * dt, lane);
          __builtin_amdgcn_s_setprio(1);
#pragma unroll
          for (int h2 = 0; h2 < 2; ++h2)
#pragma unroll
            for (int dt = 0; dt < DT; ++dt)
              acc[dt] = mfma32(opd[h2 * DT + dt], h2 ? pb[blk] : pa[blk], acc[dt]);
          __builtin_amdgcn_s_setprio(0);
        }
        // the copies of half k + 2 (the last half again when there is none:
        // buffer y is then not read before the kernel ends)
        const int hl = k + 2 < nh ? k + 2 : nh - 1;
        if (k + 2 < nh) advance(k + 2);
        issue(y, half_copies(hl));
        set_pf(y, it_n < npart);
      } else {
        // dP
        const float* dlu = ebuf(x);
        f32x16 dp[2];
#pragma unroll
        for (int blk = 0; blk < 2; ++blk) {
          const uint32_t w = blk ? w2.y : w2.x;
          if (__ballot(w != 0u) == 0ull) continue;
          const int rb = 32 * blk;
          bf16x8 opd[KS];
#pragma unroll
          for (int s = 0; s < KS; ++s) opd[s] = lds_row8<D>(du, rb + tok_perm(n), 16 * s + 8 * g);
          __builtin_amdgcn_s_setprio(1);
#pragma unroll
          for (int s = 0; s < KS; ++s) dp[blk] = mfma32(opd[s], kv[s], s ? dp[blk] : f32x16{});
          __builtin_amdgcn_s_setprio(0);
        }
        // the item bookkeeping of half k + 2 (the P waves copy it)
        if (k + 2 < nh) advance(k + 2);
        set_pf(y, it_n < npart);
        mid_barrier();
        // dS = P (dP - Delta), dK^T += Q^T dS
#pragma unroll
        for (int blk = 0; blk < 2; ++blk) {
          const uint32_t w = blk ? w2.y : w2.x;
          if (__ballot(w != 0u) == 0ull) continue;
          const int rb = 32 * blk;
          const f32x16 dl = acc_rows(dlu + rb, g);
          const bf16x8* src = p_s + ((kw * 2 + blk) * 2) * 64 + lane;
          const bf16x8 xa = src[0], xb = src[64];
          f32x16 ds;
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            ds[j] = (dp[blk][j] - dl[j]) * (float)xa[j];
            ds[8 + j] = (dp[blk][8 + j] - dl[8 + j]) * (float)xb[j];
          }
          const bf16x8 sa = pack_half(ds, 0), sb = pack_half(ds, 1);
          bf16x8 opd[2 * DT];
#pragma unroll
          for (int h2 = 0; h2 < 2; ++h2)
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) opd[h2 * DT + dt] = lds_col8<D>(qu, rb + 16 * h2, 32 * dt, lane);
          __builtin_amdgcn_s_setprio(1);
#pragma unroll
          for (int h2 = 0; h2 < 2; ++h2)
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) acc[dt] = mfma32(opd[h2 * DT + dt], h2 ? sb : sa, acc[dt]);
          __builtin_amdgcn_s_setprio(0);
        }
      }
      end_barrier();
    };
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    using I2 = std::integral_constant<int, 2>;
    // Half 0 into buffer 0, then a wait the compiler sees (it also covers
    // the K / V rows loaded into registers, so no wait for them is left in
    // the loop) and a barrier; then half 1 into buffer 1.
    if (nh > 0) {
      advance(0);
      if constexpr (!kDs) issue(I0{}, half_copies(0));
      set_pf(I0{}, it_n < npart);
    }
    dma_barrier();
    if (nh > 0) {
      const int h1 = nh > 1 ? 1 : 0;
      if (nh > 1) advance(1);
      if constexpr (!kDs) issue(I1{}, half_copies(h1));
      set_pf(I1{}, it_n < npart);
    }
    for (int k = 0; k < nh; k += 3) {
      phase(I0{}, I2{}, k);
      if (k + 1 >= nh) break;
      phase(I1{}, I0{}, k + 1);
      if (k + 2 >= nh) break;
      phase(I2{}, I1{}, k + 2);
    }
  };
  if (ds_wave) run(std::true_type{});
  else run(std::false_type{});

  // dK (dS waves, times the scale) and dV (P waves) of the tile as bf16 rows
  // in LDS (dK over the first two Q units, dV over the first two dO units,
  // padded pitch), then all eight waves store whole rows, 16 bytes per lane.
  dma_barrier();
  {
    __bf16* rows = ds_wave ? q_s : o_s;
    const float mul = ds_wave ? p.scale : 1.f;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        bf16x4 w4;
#pragma unroll
        for (int e = 0; e < 4; ++e) w4[e] = (__bf16)(acc[dt][4 * a + e] * mul);
        *reinterpret_cast<bf16x4*>(rows + kloc * pitch<D>() + 32 * dt + acc_row(4 * a, g)) = w4;
      }
  }
  __syncthreads();
  constexpr int kChunks = D / 8;  // 16-byte pieces per row
  __bf16* dkp = p.dk + b * p.dk_sb + hk * p.dk_sh;
  __bf16* dvp = p.dv + b * p.dv_sb + hk * p.dv_sh;
#pragma unroll
  for (int j = 0; j < kTile * kChunks / (kPairWaves * 64); ++j) {
    const int ci = tid + kPairWaves * 64 * j;
    const int r = ci / kChunks, ch = ci % kChunks;
    if (k0 + r < T) {
      const int64_t row = k0 + r;
      *reinterpret_cast<uint4*>(dkp + row * p.dk_st + 8 * ch) =
          *reinterpret_cast<const uint4*>(q_s + r * pitch<D>() + 8 * ch);
      *reinterpret_cast<uint4*>(dvp + row * p.dv_st + 8 * ch) =
          *reinterpret_cast<const uint4*>(o_s + r * pitch<D>() + 8 * ch);
    }
  }
}

// dQ for one (b, query head, 128-query tile).  Per wave 32 queries; S^T and
// dP^T put the query in the lane, dS^T feeds dQ^T += K^T dS^T as B operand.
// The row's KV tiles stream through LDS as 64-key halves (one unit each for
// K and V rows), refilled by direct global->LDS copies issued right after the
// barrier that retired them, so each copy has one half of compute to land in;
// the tile bitmaps travel one tile ahead the same way.
// With p.fuse_delta the rows' Delta = rowsum(O * dO) is computed here (from
// the dO rows already held in registers and one read of the O rows) and
// written for the dK/dV launch that follows, instead of read from bwd_delta.
template <int D>
__global__ __launch_bounds__(kThreads, 2) void bwd_dq_kernel(BwdParams p) {
  constexpr int KS = D / 16;
  constexpr int DT = D / 32;
  using U = UnitDma<D>;
  constexpr int kUnit = U::kRows * pitch<D>();
  __shared__ __bf16 k_lo[kUnit], k_hi[kUnit], v_lo[kUnit], v_hi[kUnit];
  __shared__ uint32_t bits_lds[2][kTile * 4];

  const int b = blockIdx.z;
  const int tid = threadIdx.x, wave = uniform(tid >> 6), lane = tid & 63;
  const int g = lane >> 5, n = lane & 31;
  const int T = p.T, nt = p.m.nt;
  int h, slot;
  head_and_slot(p.Hq, p.Hkv, nt, h, slot);
  const int hk = h / (p.Hq / p.Hkv);
  const int mb = p.m.Bm > 1 ? b : 0;
  const int qt = uniform(p.m.row_order[(size_t)mb * nt + slot]);
  const int q0 = qt * kTile;
  const int qloc = 32 * wave + n;
  const int qrow = q0 + qloc;
  const bool qvalid = qrow < T;
  const float c = p.scale_log2;

  // The row's KV tile list first: its first chunk is read back (readlane)
  // before the first K/V copy, and loads complete in issue order, so that
  // wait does not also wait for the Q / dO / O rows issued after it.
  const size_t row = (size_t)mb * nt + qt;
  const int npart = uniform(p.m.kv_num[row]);
  const int nfull = uniform(p.m.full_kv_num[row]);
  const int ntiles = npart + nfull;
  const int32_t* pidx = p.m.kv_idx + row * nt;
  const int32_t* fidx = p.m.full_kv_idx + row * nt;
  const uint32_t* bits_row = p.m.tile_bits + (size_t)p.m.kv_bits_off[row] * kTileBitsWords;
  // KV tile indices of the row, 64 iterations per chunk (lane j: iteration
  // 64 * chunk + j), read back with readlane.
  auto load_chunk = [&](int chunk) {
    const int it = 64 * chunk + lane;
    return it < npart ? pidx[it] : (it < ntiles ? fidx[it - npart] : 0);
  };
  int tiles_v = load_chunk(0);

  // Rows past T read row 0: a query row only reaches its own dQ column,
  // which is not stored, and its P is zero (neg_lse = -inf).
  const int qr = qvalid ? qrow : 0;
  const size_t rowstat = ((size_t)b * p.Hq + h) * T + qr;
  bf16x8 qf[KS], dof[KS], of[KS];
  {
    const __bf16* qp = p.q + b * p.q_sb + h * p.q_sh + (int64_t)qr * p.q_st;
    const __bf16* dp = p.dout + b * p.do_sb + h * p.do_sh + (int64_t)qr * p.do_st;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      qf[s] = *reinterpret_cast<const bf16x8*>(qp + 16 * s + 8 * g);
      dof[s] = *reinterpret_cast<const bf16x8*>(dp + 16 * s + 8 * g);
    }
  }
  if (p.fuse_delta) {
    // Lane (g, n) holds elements 16 s + 8 g .. + 7 of its row's dO; the
    // matching O elements give half the row's Delta = rowsum(O * dO).
    const __bf16* op = p.o + b * p.o_sb + h * p.o_sh + (int64_t)qr * p.o_st;
#pragma unroll
    for (int s = 0; s < KS; ++s) of[s] = *reinterpret_cast<const bf16x8*>(op + 16 * s + 8 * g);
  }
  const float lrow = p.lse2[rowstat];
  float delta = p.fuse_delta ? 0.f : p.delta[rowstat];
  // fully masked row (lse2 = -inf) or row past T: P = 0
  const float neg_lse = (!qvalid || lrow == -INFINITY) ? -INFINITY : -lrow;

  const __bf16* kbase = p.k + b * p.k_sb + hk * p.k_sh;
  const __bf16* vbase = p.v + b * p.v_sb + hk * p.v_sh;
  int koff[U::kPerWave + 1], voff[U::kPerWave + 1];
#pragma unroll
  for (int j = 0; j < U::kPerWave; ++j) {
    koff[j] = unit_dma_offset<D>(wave + kWaves * j, p.k_st, lane);
    voff[j] = unit_dma_offset<D>(wave + kWaves * j, p.v_st, lane);
  }
  koff[U::kPerWave] = unit_dma_offset<D>(U::kInsts - 1, p.k_st, lane);
  voff[U::kPerWave] = unit_dma_offset<D>(U::kInsts - 1, p.v_st, lane);

  auto tile_of = [&](int it) { return __builtin_amdgcn_readlane(tiles_v, it & 63); };
  const auto krs = slice_rsrc(kbase, p.k_st, T, D);
  const auto vrs = slice_rsrc(vbase, p.v_st, T, D);
  const int k_row2 = (int)p.k_st * 2, v_row2 = (int)p.v_st * 2;
  // K and V rows [t0, t0 + 64) into one half's units (rows past T read zero).
  auto load_half = [&](__bf16* kd, __bf16* vd, int t0) {
    unit_dma<D>(kd, krs, koff, t0 * k_row2, wave, 0);
    unit_dma<D>(vd, vrs, voff, t0 * v_row2, wave, 1);
  };
  // Row-major half (128 queries x 4 words) of the bitmap of iteration it
  // (KV tile kt, slot kv_bits_off + kt); waves 0 and 1 copy 1 KiB each.
  // Tiles without a bitmap copy zeros.
  auto load_bits = [&](int it, int kt) {
    const bool has = it < npart;
    const auto rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint32_t*>(bits_row + (has ? (size_t)kt * kTileBitsWords : 0)), 0,
        has ? kTile * 16 : 0, 0x00020000);
    if (wave < 2)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rs, (__attribute__((address_space(3))) void*)(&bits_lds[it & 1][wave * 256]), 16,
          wave * 1024 + lane * 16, 0, 0, 0);
  };

  f32x16 dqacc[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) dqacc[dt] = f32x16{};
  // -Delta in every entry: the dP^T chains start from it and end at dP - Delta.
  f32x16 dseed;

  // One 32-key block: rows 32 j .. 32 j + 31 of a half's units; w = the
  // lane's bitmap word (all ones for full tiles).
  auto block = [&](const __bf16* ku, const __bf16* vu, uint32_t w, int j) {
    if (__ballot(w != 0u) == 0ull) return;
    f32x16 sacc, dpacc;
    // The score chain starts from the mask seed (mixed blocks) or from the
    // MFMA's inline zero (no register initialisation): one copy of the run
    // for each start.  MFMA runs at raised wave priority.
    auto score_run = [&](auto seeded) __attribute__((always_inline)) {
      __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        const bf16x8 ka = lds_row8<D>(ku, 32 * j + tok_perm(n), 16 * s + 8 * g);
        const bf16x8 va = lds_row8<D>(vu, 32 * j + tok_perm(n), 16 * s + 8 * g);
        if (decltype(seeded)::value || s > 0)
          sacc = mfma32(ka, qf[s], sacc);
        else
          sacc = mfma32(ka, qf[s], f32x16{});
        dpacc = mfma32(va, dof[s], s > 0 ? dpacc : dseed);
      }
      // LDS reads four MFMAs ahead of their use.
      __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
      for (int i = 0; i < 2 * KS - 4; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
      __builtin_amdgcn_s_setprio(0);
    };
    if (__ballot(w != ~0u) != 0ull) {
      sacc = mask_bias(~(w >> g));
      score_run(std::true_type{});
    } else {
      score_run(std::false_type{});
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const float pv = fast_exp2(fmaf(sacc[i], c, neg_lse));
      dpacc[i] = pv * dpacc[i];  // dS^T
    }
    // dQ^T += K^T dS^T (contraction over the 32 keys of the block).
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int h2 = 0; h2 < 2; ++h2) {
      const bf16x8 sb = pack_half(dpacc, h2);
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const bf16x8 ka = lds_col8<D>(ku, 32 * j + 16 * h2, 32 * dt, lane);
        dqacc[dt] = mfma32(ka, sb, dqacc[dt]);
      }
    }
    __builtin_amdgcn_s_setprio(0);
  };

  int k0_next = ntiles > 0 ? tile_of(0) * kTile : 0;
  if (ntiles > 0) {
    load_half(k_lo, v_lo, k0_next);
    if (npart > 0) load_bits(0, k0_next / kTile);
  }
  if (p.fuse_delta) {
    // While the first K/V half is in flight: the two lane halves of a row
    // each sum half its products; written once per row for dK/dV.
    float acc = 0.f;
#pragma unroll
    for (int s = 0; s < KS; ++s)
#pragma unroll
      for (int j = 0; j < 8; ++j) acc = fmaf((float)of[s][j], (float)dof[s][j], acc);
    delta = halves_sum(acc);
    if (qvalid && g == 0) p.delta[rowstat] = delta;
  }
#pragma unroll
  for (int i = 0; i < 16; ++i) dseed[i] = -delta;
  for (int it = 0; it < ntiles; ++it) {
    const bool partial = it < npart;
    const int k0 = k0_next;
    // Keys [k0, k0 + 64): its units and bitmap have landed; the other half's
    // units are free again.
    dma_barrier();
    uint4 mbits = make_uint4(~0u, ~0u, ~0u, ~0u);
    if (partial) mbits = *reinterpret_cast<const uint4*>(&bits_lds[it & 1][qloc * 4]);
    load_half(k_hi, v_hi, k0 + 64);
    block(k_lo, v_lo, mbits.x, 0);
    block(k_lo, v_lo, mbits.y, 1);

    // Keys [k0 + 64, k0 + 128); the first half's units are free again.
    dma_barrier();
    const bool more = it + 1 < ntiles;
    if (more) {
      if (((it + 1) & 63) == 0) tiles_v = load_chunk((it + 1) >> 6);
      k0_next = tile_of(it + 1) * kTile;
      load_half(k_lo, v_lo, k0_next);
      load_bits(it + 1, k0_next / kTile);
    }
    block(k_hi, v_hi, mbits.z, 0);
    block(k_hi, v_hi, mbits.w, 1);
  }

  if (qvalid) {
    __bf16* dqp = p.dq + b * p.dq_sb + h * p.dq_sh + (int64_t)qrow * p.dq_st;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) store_acc_t(dqp, dqacc[dt], 32 * dt, g, p.scale);
  }
}

namespace {

BwdParams make_bwd_params(const TensorView& q, const TensorView& k, const TensorView& v,
                          const TensorView& o, const TensorView& dout, const float* lse2,
                          float* delta, const TensorView& dq, const TensorView& dk,
                          const TensorView& dv, const AttnDims& dims, const MaskTables& mask) {
  BwdParams p;
  p.q = static_cast<const __bf16*>(q.data); p.q_sb = q.sb; p.q_sh = q.sh; p.q_st = q.st;
  p.k = static_cast<const __bf16*>(k.data); p.k_sb = k.sb; p.k_sh = k.sh; p.k_st = k.st;
  p.v = static_cast<const __bf16*>(v.data); p.v_sb = v.sb; p.v_sh = v.sh; p.v_st = v.st;
  p.o = static_cast<const __bf16*>(o.data); p.o_sb = o.sb; p.o_sh = o.sh; p.o_st = o.st;
  p.dout = static_cast<const __bf16*>(dout.data); p.do_sb = dout.sb; p.do_sh = dout.sh; p.do_st = dout.st;
  p.dq = static_cast<__bf16*>(dq.data); p.dq_sb = dq.sb; p.dq_sh = dq.sh; p.dq_st = dq.st;
  p.dk = static_cast<__bf16*>(dk.data); p.dk_sb = dk.sb; p.dk_sh = dk.sh; p.dk_st = dk.st;
  p.dv = static_cast<__bf16*>(dv.data); p.dv_sb = dv.sb; p.dv_sh = dv.sh; p.dv_st = dv.st;
  p.lse2 = lse2;
  p.delta = delta;
  p.B = dims.B; p.Hq = dims.Hq; p.Hkv = dims.Hkv; p.T = dims.T;
  p.scale = dims.scale;
  p.scale_log2 = dims.scale * kLog2e;
  p.fuse_delta = 0;
  p.m = mask;
  return p;
}

}  // namespace

hipError_t launch_attn_bwd_phase(int phase, const TensorView& q, const TensorView& k,
                                 const TensorView& v, const TensorView& o,
                                 const TensorView& dout, const float* lse2, float* delta,
                                 const TensorView& dq, const TensorView& dk, const TensorView& dv,
                                 const AttnDims& dims, const MaskTables& mask,
                                 hipStream_t stream) {
  const BwdParams p = make_bwd_params(q, k, v, o, dout, lse2, delta, dq, dk, dv, dims, mask);
  const int nt = (dims.T + kTile - 1) / kTile;
  if (nt == 0 || dims.B == 0 || dims.Hq == 0) return hipSuccess;
  const bool d64 = dims.D == 64;
  if (phase == kBwdDelta) {
    const int64_t rows = (int64_t)dims.B * dims.Hq * dims.T;
    const int rows_per_block = kThreads / (dims.D / 8);
    const dim3 grid((unsigned)((rows + rows_per_block - 1) / rows_per_block));
    if (d64) hipLaunchKernelGGL(bwd_delta_kernel<64>, grid, dim3(kThreads), 0, stream, p);
    else hipLaunchKernelGGL(bwd_delta_kernel<128>, grid, dim3(kThreads), 0, stream, p);
  } else if (phase == kBwdDkDv) {
    const dim3 grid(dims.Hkv, nt, dims.B);
#ifdef T2T_DKDV_CLASSIC
    if (d64) hipLaunchKernelGGL(bwd_dkdv_kernel<64>, grid, dim3(kDkdvThreads), 0, stream, p);
    else hipLaunchKernelGGL(bwd_dkdv_kernel<128>, grid, dim3(kDkdvThreads), 0, stream, p);
#else
    if (d64) hipLaunchKernelGGL(bwd_dkdv_pair_kernel<64>, grid, dim3(kPairWaves * 64), 0, stream, p);
    else hipLaunchKernelGGL(bwd_dkdv_kernel<128>, grid, dim3(kDkdvThreads), 0, stream, p);
#endif
  } else {  // kBwdDq, kBwdDqDelta
    BwdParams pq = p;
    pq.fuse_delta = phase == kBwdDqDelta;
    const dim3 grid(dims.Hq, nt, dims.B);
    if (d64) hipLaunchKernelGGL(bwd_dq_kernel<64>, grid, dim3(kThreads), 0, stream, pq);
    else hipLaunchKernelGGL(bwd_dq_kernel<128>, grid, dim3(kThreads), 0, stream, pq);
  }
  return hipGetLastError();
}

}  // namespace t2t
