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
// in the same key order.  The softmax runs in the log2 domain (scores times
// scale * log2 e); LSE is written in that domain, and the host multiplies by
// ln 2 for the natural-log value.  The running reference max only moves when
// a row's max exceeds it by more than 2^8 in probability (lazy rescaling):
// probabilities stay below 256, far inside fp32 / bf16 range, and O is
// rescaled a handful of times per row instead of at every block.
//
// Pipeline: each KV tile is consumed in steps of SK keys (K rows + V rows,
// one LDS unit each): two 64-key halves at D = 64, four 32-key quarters at
// D = 128, where the smaller step's registers and LDS units let three
// work-groups share a CU instead of two.  While a wave computes on one
// step, the other buffer's units are being filled by direct global->LDS
// copies issued right after the barrier that retired them; each lane loads
// its query row's words of the next tile's bitmap into registers at the
// tile's last step.  One barrier per step.  No staging registers and no
// register->LDS stores.
//
// Work-groups are dispatched longest row first (row_order); with grouped-query
// heads the heads of one KV head and row run back to back on one XCD
// (head_and_slot), so their K/V copies are served by that XCD's L2.
#include "attn_kernels.h"

namespace t2t {

namespace {

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

template <int D, int SK>
__global__ __launch_bounds__(kThreads, 2) void attn_fwd_bf16_kernel(FwdParams p) {
  constexpr int KS = D / 16;     // MFMA k-steps over the head dim
  constexpr int DT = D / 32;     // 32-wide output column tiles
  constexpr int NB = SK / 32;    // 32-key blocks per step
  constexpr int NS = kTile / SK; // steps per KV tile
  constexpr int PK = SK / 16;    // P V k-steps per step
  using U = UnitDma<D, kWaves, SK>;
  __shared__ __bf16 k_a[U::kElems], k_b[U::kElems], v_a[U::kElems], v_b[U::kElems];

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

  const __bf16* kbase = p.k + b * p.k_sb + hk * p.k_sh;
  const __bf16* vbase = p.v + b * p.v_sb + hk * p.v_sh;
  int koff[U::kPerWave + 1], voff[U::kPerWave + 1];
#pragma unroll
  for (int j = 0; j < U::kPerWave; ++j) {
    koff[j] = unit_dma_offset<D, SK>(wave + kWaves * j, p.k_st, lane);
    voff[j] = unit_dma_offset<D, SK>(wave + kWaves * j, p.v_st, lane);
  }
  koff[U::kPerWave] = unit_dma_offset<D, SK>(U::kInsts - 1, p.k_st, lane);
  voff[U::kPerWave] = unit_dma_offset<D, SK>(U::kInsts - 1, p.v_st, lane);

  const size_t row = (size_t)mb * nt + qt;
  const int npart = uniform(p.m.kv_num[row]);
  const int nfull = uniform(p.m.full_kv_num[row]);
  const int ntiles = npart + nfull;
  const int32_t* pidx = p.m.kv_idx + row * nt;
  const int32_t* fidx = p.m.full_kv_idx + row * nt;
  const uint32_t* bits_row = p.m.tile_bits + (size_t)p.m.kv_bits_off[row] * kTileBitsWords;

  // KV tile indices of the row, 64 iterations per chunk: lane j of tiles_v
  // holds the tile of iteration 64 * chunk + j (read back with readlane).
  auto load_chunk = [&](int chunk) {
    const int it = 64 * chunk + lane;
    return it < npart ? pidx[it] : (it < ntiles ? fidx[it - npart] : 0);
  };
  int tiles_v = load_chunk(0);
  auto tile_of = [&](int it) { return __builtin_amdgcn_readlane(tiles_v, it & 63); };
  // K and V rows [t0, t0 + SK) into one step's units.
  // (t0 >= T, e.g. past the last tile, copies zeros.)
  const auto krs = slice_rsrc(kbase, p.k_st, T, D);
  const auto vrs = slice_rsrc(vbase, p.v_st, T, D);
  const int k_row2 = (int)p.k_st * 2, v_row2 = (int)p.v_st * 2;
  auto load_step = [&](__bf16* kd, __bf16* vd, int t0) {
    unit_dma<D, kWaves, SK>(kd, krs, koff, t0 * k_row2, wave, 0);
    unit_dma<D, kWaves, SK>(vd, vrs, voff, t0 * v_row2, wave, 1);
  };
  // The lane's four bitmap words (its query row of the tile's row-major
  // bitmap) of iteration it, loaded into registers one tile ahead.  (Tiles
  // without a bitmap, it >= npart, read zeros.)
  auto load_bits = [&](int it, int kt) {
    const bool has = it < npart;
    const auto rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint32_t*>(bits_row + (has ? (size_t)kt * kTileBitsWords : 0)), 0,
        has ? kTile * 16 : 0, 0x00020000);
    return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rs, qloc * 16, 0, 0));
  };

  f32x16 oacc[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) oacc[dt] = f32x16{};
  float m_ref = -INFINITY, l_run = 0.f;  // reference max of raw scores, running sum

  // One step of SK keys (NB 32-key blocks): S^T = K Q^T (+ mask seed),
  // lazy-rescaled online softmax, O^T += V^T P^T.  w0, w1: bitmap words of
  // the step's 32-key blocks (w1 unused when NB = 1).  A step with any
  // allowed pair is computed whole (a block without one gets an all -inf
  // seed), which keeps each contraction one straight-line run of NB
  // interleaved accumulator chains.
  auto step = [&](const __bf16* kt_lds, const __bf16* vt_lds, uint32_t w0, uint32_t w1,
                  bool partial) {
    const uint32_t w_any = NB == 2 ? (w0 | w1) : w0, w_all = NB == 2 ? (w0 & w1) : w0;
    if (partial && __ballot(w_any != 0u) == 0ull) return;
    f32x16 st[NB];
    // The chains start from the mask seeds (mixed steps) or from the MFMA's
    // inline zero (no register initialisation): one copy of the run for each
    // start.  MFMA runs issue at raised wave priority, so that the waves
    // sharing the SIMD fill the gaps with their softmax instead of competing
    // for issue.
    auto score_run = [&](auto seeded) __attribute__((always_inline)) {
      __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int s = 0; s < KS; ++s)
#pragma unroll
        for (int j = 0; j < NB; ++j) {
          const bf16x8 kf = lds_row8<D>(kt_lds, 32 * j + tok_perm(n), 16 * s + 8 * g);
          if (decltype(seeded)::value || s > 0)
            st[j] = mfma32(kf, qf[s], st[j]);
          else
            st[j] = mfma32(kf, qf[s], f32x16{});
        }
      // Issue the K reads a few MFMAs ahead of their use.
      __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
      for (int i = 0; i < NB * KS - 4; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
      __builtin_amdgcn_s_setprio(0);
    };
    if (partial && __ballot(w_all != ~0u) != 0ull) {
      st[0] = mask_bias(~(w0 >> g));
      if constexpr (NB == 2) st[NB - 1] = mask_bias(~(w1 >> g));
      score_run(std::true_type{});
    } else {
      score_run(std::false_type{});
    }

    // Probabilities against the current reference max come first.  The
    // reference moves only when the row max exceeds it by 8 (log2 units),
    // i.e. when a probability would exceed 2^8; a lane whose probabilities
    // sum to at most 2^7 has none near that, so when every lane's sum is
    // that small and every row has a finite reference, no row moves and the
    // probabilities stand -- the row max is not needed at all.  Otherwise
    // the row max decides as before, and rows that move rescale O and the
    // sum and recompute their probabilities.  Either way the values are
    // those of the max-first order.
    auto probs = [&](bf16x8* pf) {
      const float neg = m_ref == -INFINITY ? 0.f : -m_ref * c;
      float rs = 0.f;
#pragma unroll
      for (int s = 0; s < PK; ++s)  // k-step s: entries [8 (s & 1), + 8) of block s >> 1
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          const float e = fast_exp2(fmaf(st[s >> 1][8 * (s & 1) + k], c, neg));
          pf[s][k] = (__bf16)e;
          rs += e;
        }
      return rs;
    };
    bf16x8 pf[PK];
    float rs = probs(pf);
    // (pins the first evaluation ahead of the branch; the compiler would
    // otherwise move it into the branch's fall-through, behind the row max)
    if constexpr (PK == 4)
      asm volatile("" ::"v"(pf[0]), "v"(pf[1]), "v"(pf[2]), "v"(pf[3]), "v"(rs));
    else
      asm volatile("" ::"v"(pf[0]), "v"(pf[1]), "v"(rs));
    if (__ballot(m_ref == -INFINITY || !(rs <= 128.f)) != 0ull) {
      float mx = -INFINITY;
#pragma unroll
      for (int j = 0; j < NB; ++j)
#pragma unroll
        for (int i = 0; i < 16; ++i) mx = fmaxf(mx, st[j][i]);
      mx = halves_max(mx);
      // -inf - -inf compares false, so untouched rows never move.
      const bool move = (mx - m_ref) * c > 8.f;
      if (__ballot(move) != 0ull) {
        const float alpha = move ? fast_exp2((m_ref - mx) * c) : 1.f;  // 0 from -inf
        l_run *= alpha;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) oacc[dt] *= alpha;
        m_ref = move ? mx : m_ref;
        rs = probs(pf);
      }
    }
    l_run += halves_sum(rs);

    // O^T += V^T P^T, 16 keys per k-step.
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int s = 0; s < PK; ++s)
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const bf16x8 vf = lds_col8<D>(vt_lds, 16 * s, 32 * dt, lane);
        oacc[dt] = mfma32(vf, pf[s], oacc[dt]);
      }
    // V transpose reads one k-step (DT MFMAs) ahead.
    __builtin_amdgcn_sched_group_barrier(0x100, 2 * DT, 1);
#pragma unroll
    for (int i = 0; i < (PK - 1) * DT; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 1);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, DT, 1);
    __builtin_amdgcn_s_setprio(0);
  };

  int k0_next = ntiles > 0 ? tile_of(0) * kTile : 0;
  uint4 mb_next = make_uint4(~0u, ~0u, ~0u, ~0u);
  if (ntiles > 0) {
    if (npart > 0) mb_next = load_bits(0, k0_next / kTile);
    load_step(k_a, v_a, k0_next);
  }
  for (int it = 0; it < ntiles; ++it) {
    const bool partial = it < npart;
    const int k0 = k0_next;
    const uint4 mbits = partial ? mb_next : make_uint4(~0u, ~0u, ~0u, ~0u);
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      // Keys [k0 + SK s, + SK): their units (and at s = 0 the tile's bitmap
      // words) have landed; the other buffer's units are free again.
      dma_barrier();
      __bf16 *kc = (s & 1) ? k_b : k_a, *vc = (s & 1) ? v_b : v_a;
      __bf16 *kn = (s & 1) ? k_a : k_b, *vn = (s & 1) ? v_a : v_b;
      if (s + 1 < NS) {
        load_step(kn, vn, k0 + SK * (s + 1));
      } else if (it + 1 < ntiles) {
        if (((it + 1) & 63) == 0) tiles_v = load_chunk((it + 1) >> 6);
        k0_next = tile_of(it + 1) * kTile;
        if (it + 1 < npart) mb_next = load_bits(it + 1, k0_next / kTile);
        load_step(kn, vn, k0_next);
      }
      auto word = [&](int i) { return i == 0 ? mbits.x : i == 1 ? mbits.y : i == 2 ? mbits.z : mbits.w; };
      step(kc, vc, word(NB * s), word(NB * s + NB - 1), partial);
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
          l_run > 0.f ? m_ref * c + __log2f(l_run) : -INFINITY;
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
  // Keys per step: 64 at D = 64 (128 VGPRs, 36 KiB: four work-groups per
  // CU), 32 at D = 128 (158 VGPRs, 36 KiB: three per CU, where 64-key halves
  // hold 180 VGPRs and 68 KiB, two per CU).
  if (dims.D == 64)
    hipLaunchKernelGGL((attn_fwd_bf16_kernel<64, 64>), grid, dim3(kThreads), 0, stream, p);
  else
    hipLaunchKernelGGL((attn_fwd_bf16_kernel<128, 32>), grid, dim3(kThreads), 0, stream, p);
  return hipGetLastError();
}

}  // namespace t2t
