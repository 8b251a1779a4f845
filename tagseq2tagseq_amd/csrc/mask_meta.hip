// Mask-metadata pass: per-token document ids and grant words -> 128 x 128 tile
// classification (skip / partial / full), the ordered index lists of a
// BlockMask, launch orders and per-partial-tile allowed-pair bitmaps.
//
// Semantics restated from
//   * mask_mod:  model/graph_traversal/cross_doc_mask.py:348-357
//                (doc_causal: block_mask_creator.py:121-129, words == 0)
//   * classification: torch/nn/attention/flex_attention.py:979-1022 -- the
//                [T,T] mask padded with False to a multiple of 128; a tile is
//                full iff all 128*128 pairs are allowed, partial iff some but
//                not all are, skip otherwise
//   * index lists: torch/nn/attention/flex_attention.py:429-441 -- num = row
//                sum; indices = set columns ascending, then unset columns
//                ascending (stable descending argsort); q-side lists are the
//                same over the transposed grid.
//
// Instead of materialising the T x T mask, each tile is decided from runs of
// tokens with identical (doc id, grant words): within a (q-run, kv-run)
// rectangle the non-causal part of the predicate is constant, so a tile needs
// one predicate evaluation per run pair plus the causal geometry of the
// rectangle.  Packed documents give 1-3 runs per 128 tokens, so a tile costs a
// handful of evaluations instead of 16384.
//
// Launches: (1) classify every tile, (2) row and column lists, (3) partial-
// tile bitmaps; the third also writes the bitmap slot offsets (each row's
// column-0 work-group) and the launch orders (work-group (0, 0) of each mask
// row), so no launch waits on a single work-group.
#include "attn_kernels.h"

namespace t2t {

namespace {

// Lower-triangle tile of linear index L (row-major over qt, kt <= qt).
__device__ __forceinline__ void tri_tile(int L, int& qt, int& kt) {
  int r = (int)((sqrtf(8.f * (float)L + 1.f) - 1.f) * 0.5f);
  while ((r + 1) * (r + 2) / 2 <= L) ++r;  // exact despite float rounding
  while (r * (r + 1) / 2 > L) --r;
  qt = r;
  kt = L - r * (r + 1) / 2;
}

struct TokSig {
  int32_t doc;
  uint64_t bits[kMaxWords];
};

__device__ __forceinline__ void load_sig(TokSig& s, const int32_t* doc, const uint64_t* bits,
                                         int words, int T, int t) {
  s.doc = doc[t];
#pragma unroll
  for (int w = 0; w < kMaxWords; ++w) s.bits[w] = (w < words) ? bits[(size_t)w * T + t] : 0ull;
}

__device__ __forceinline__ bool sig_eq(const TokSig& a, const TokSig& b, int words) {
  if (a.doc != b.doc) return false;
#pragma unroll
  for (int w = 0; w < kMaxWords; ++w)
    if (w < words && a.bits[w] != b.bits[w]) return false;
  return true;
}

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }

__device__ __forceinline__ int lanes_below(uint64_t mask) {
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32),
                                   __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0));
}

// One wave: tokens base+lane and base+64+lane (those < T).  Writes the start
// offsets (relative to base) of runs of identical signatures into starts[],
// terminated by starts[n] = number of valid tokens; returns n.
__device__ int wave_runs(const int32_t* doc, const uint64_t* bits, int words, int T,
                         int base, int* starts) {
  const int lane = lane_id();
  const int nvalid = min(kTile, T - base);
  int flag[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int t = lane + 64 * h;
    flag[h] = 0;
    if (t < nvalid) {
      if (t == 0) {
        flag[h] = 1;
      } else {
        TokSig cur, prev;
        load_sig(cur, doc, bits, words, T, base + t);
        load_sig(prev, doc, bits, words, T, base + t - 1);
        flag[h] = !sig_eq(cur, prev, words);
      }
    }
  }
  const uint64_t m0 = __ballot(flag[0]);
  const uint64_t m1 = __ballot(flag[1]);
  const int n0 = __popcll(m0);
  if (flag[0]) starts[lanes_below(m0)] = lane;
  if (flag[1]) starts[n0 + lanes_below(m1)] = lane + 64;
  const int n = n0 + __popcll(m1);
  if (lane == 0) starts[n] = nvalid;
  return n;
}

__device__ __forceinline__ bool sig_pair_allowed(const int32_t* doc, const uint64_t* qbits,
                                                 const uint64_t* kvbits, int words, int T,
                                                 int q, int kv) {
  if (doc[q] == doc[kv]) return true;
  for (int w = 0; w < words; ++w)
    if (qbits[(size_t)w * T + q] & kvbits[(size_t)w * T + kv]) return true;
  return false;
}

// Compact one 0/1 row of `n` byte flags (flag = (cls == want)) into the
// ordered list of torch's _dense_to_ordered: set positions ascending, then
// unset positions ascending.  One wave; `cls` is read with stride `stride`.
__device__ void wave_ordered(const int8_t* cls, int stride, int n, int8_t want,
                             int32_t* num_out, int32_t* idx_out) {
  const int lane = lane_id();
  int total = 0;
  for (int c = 0; c < n; c += 64) {
    const int i = c + lane;
    const bool f = (i < n) && cls[(size_t)i * stride] == want;
    total += __popcll(__ballot(f));
  }
  int set_base = 0, unset_base = total;
  for (int c = 0; c < n; c += 64) {
    const int i = c + lane;
    const bool in = i < n;
    const bool f = in && cls[(size_t)i * stride] == want;
    const uint64_t ms = __ballot(f);
    const uint64_t mu = __ballot(in && !f);
    if (f) idx_out[set_base + lanes_below(ms)] = i;
    else if (in) idx_out[unset_base + lanes_below(mu)] = i;
    set_base += __popcll(ms);
    unset_base += __popcll(mu);
  }
  if (lane == 0) *num_out = total;
}

}  // namespace

// (1) grid (nt (nt + 1) / 2, Bm); block 64: one wave decides one tile of the
// lower triangle (kt <= qt) and writes its mirror above the diagonal as skip
// (every pair there has kv > q).
__global__ __launch_bounds__(64) void mask_classify_tiles(
    const int32_t* __restrict__ doc_all, const uint64_t* __restrict__ qbits_all,
    const uint64_t* __restrict__ kvbits_all, int T, int words, MaskOut out) {
  __shared__ int q_starts[kTile + 1];
  __shared__ int kv_starts[kTile + 1];
  const int nt = out.nt;
  const int b = blockIdx.y;
  int qt, kt;
  tri_tile(blockIdx.x, qt, kt);
  const int lane = threadIdx.x;
  int8_t* dst = out.tile_class + ((size_t)b * nt + qt) * nt + kt;
  if (lane == 0 && kt < qt) out.tile_class[((size_t)b * nt + kt) * nt + qt] = kSkip;
  const int32_t* doc = doc_all + (size_t)b * T;
  const uint64_t* qbits = qbits_all + (size_t)b * words * T;
  const uint64_t* kvbits = kvbits_all + (size_t)b * words * T;
  const int q0 = qt * kTile, k0 = kt * kTile;
  const int qvalid = min(kTile, T - q0), kvalid = min(kTile, T - k0);
  const int nqr = wave_runs(doc, qbits, words, T, q0, q_starts);
  const int nkr = wave_runs(doc, kvbits, words, T, k0, kv_starts);
  __syncthreads();
  // Padding rows/columns are False pairs: such a tile can never be full.
  bool any_true = false;
  bool any_false = (qvalid < kTile) || (kvalid < kTile);
  const int npairs = nqr * nkr;
  for (int p0 = 0; p0 < npairs; p0 += 64) {
    const int p = p0 + lane;
    bool t = false, f = false;
    if (p < npairs) {
      const int r = p / nkr, s = p - r * nkr;
      const int qa = q0 + q_starts[r], qb = q0 + q_starts[r + 1];
      const int ka = k0 + kv_starts[s], kb = k0 + kv_starts[s + 1];
      const bool v = sig_pair_allowed(doc, qbits, kvbits, words, T, qa, ka);
      const bool exists_ge = (qb - 1) >= ka;   // some pair with q >= kv
      const bool exists_lt = qa < (kb - 1);    // some pair with q < kv
      t = v && exists_ge;
      f = !v || exists_lt;
    }
    any_true = any_true || (__ballot(t) != 0);
    any_false = any_false || (__ballot(f) != 0);
    if (any_true && any_false) break;
  }
  if (lane == 0) *dst = any_true ? (any_false ? kPartial : kFull) : kSkip;
}

// (2) grid (nt, Bm); block 256.  Wave 0/1: partial / full list of row x;
// wave 2/3: partial / full list of column x.
__global__ __launch_bounds__(kThreads) void mask_lists(MaskOut out) {
  const int nt = out.nt;
  const int i = blockIdx.x, b = blockIdx.y;
  const int wave = threadIdx.x >> 6;
  const int8_t* grid = out.tile_class + (size_t)b * nt * nt;
  const size_t r = (size_t)b * nt + i;
  if (wave == 0)
    wave_ordered(grid + (size_t)i * nt, 1, nt, kPartial, out.kv_num + r, out.kv_idx + r * nt);
  else if (wave == 1)
    wave_ordered(grid + (size_t)i * nt, 1, nt, kFull, out.full_kv_num + r, out.full_kv_idx + r * nt);
  else if (wave == 2)
    wave_ordered(grid + i, nt, nt, kPartial, out.q_num + r, out.q_idx + r * nt);
  else
    wave_ordered(grid + i, nt, nt, kFull, out.full_q_num + r, out.full_q_idx + r * nt);
}

namespace {

constexpr int kRankChunk = 512;

// Launch orders of mask row b, by the whole work-group: rows / columns ranked
// by descending non-skip tile count in buckets of kOrderBucket tiles, rows of
// one bucket by descending index and columns by ascending index -- longest
// first for the load balance, and within a bucket neighbouring rows (which
// mostly read the same K/V tiles) or columns back to back, so that a cache
// serves the shared tiles.  The counts are staged through LDS in chunks.
constexpr int kOrderBucket = 2;

__device__ void rank_orders(const MaskOut& out, int b, int* rtot, int* ctot) {
  const int nt = out.nt, tid = threadIdx.x;
  const int32_t* rn = out.kv_num + (size_t)b * nt;
  const int32_t* rf = out.full_kv_num + (size_t)b * nt;
  const int32_t* cn = out.q_num + (size_t)b * nt;
  const int32_t* cf = out.full_q_num + (size_t)b * nt;
  for (int i0 = 0; i0 < nt; i0 += kThreads) {
    const int i = i0 + tid;
    const int ri = i < nt ? (rn[i] + rf[i]) / kOrderBucket : 0;
    const int ci = i < nt ? (cn[i] + cf[i]) / kOrderBucket : 0;
    int rr = 0, rc = 0;
    for (int j0 = 0; j0 < nt; j0 += kRankChunk) {
      const int m = min(kRankChunk, nt - j0);
      __syncthreads();
      for (int j = tid; j < m; j += kThreads) {
        rtot[j] = (rn[j0 + j] + rf[j0 + j]) / kOrderBucket;
        ctot[j] = (cn[j0 + j] + cf[j0 + j]) / kOrderBucket;
      }
      __syncthreads();
      for (int j = 0; j < m; ++j) {
        const int rj = rtot[j], cj = ctot[j];
        rr += (rj > ri) || (rj == ri && j0 + j > i);
        rc += (cj > ci) || (cj == ci && j0 + j < i);
      }
    }
    if (i < nt) {
      out.row_order[(size_t)b * nt + rr] = i;
      out.col_order[(size_t)b * nt + rc] = i;
    }
  }
}

// Exclusive prefix of kv_num over (mask row, row) up to entry e = b * nt + qt,
// by one wave: the first bitmap slot of that row's partial tiles.
__device__ int row_slot_offset(const MaskOut& out, int e, int lane) {
  int sum = 0;
  for (int c = 0; c < e; c += 64) {
    const int j = c + lane;
    sum += j < e ? out.kv_num[j] : 0;
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off, 64);
  return sum;
}

}  // namespace

namespace {

// Set bits [lo, hi) of a 128-bit mask held as four 32-bit words.
__device__ __forceinline__ void set_bit_range(uint32_t acc[4], int lo, int hi) {
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const int a = max(lo - 32 * w, 0), z = min(hi - 32 * w, 32);
    if (a < z) {
      const uint32_t upto = z == 32 ? ~0u : ((1u << z) - 1u);
      acc[w] |= upto & ~((1u << a) - 1u);
    }
  }
}

__device__ __forceinline__ bool lds_pair_allowed(int32_t da, int32_t db, const uint64_t* ba,
                                                 const uint64_t* bb, int stride_a, int stride_b,
                                                 int words) {
  if (da == db) return true;
  for (int w = 0; w < words; ++w)
    if (ba[w * stride_a] & bb[w * stride_b]) return true;
  return false;
}

}  // namespace

// (3) grid (nt (nt + 1) / 2, Bm); block 256.  For a partial tile of the lower
// triangle: its
// slot (row-major numbering over (b, qt, list position)), both bitmap
// orientations, and its entry in the column's slot list.  A row of the
// bitmap is built run by run: within a run of keys with one signature the
// non-causal predicate is constant, so one evaluation sets a whole bit range;
// the causal and padding limits are applied last.
__global__ __launch_bounds__(kThreads) void mask_tile_bits(
    const int32_t* __restrict__ doc_all, const uint64_t* __restrict__ qbits_all,
    const uint64_t* __restrict__ kvbits_all, int T, int words, MaskOut out) {
  __shared__ int32_t qdoc[kTile], kdoc[kTile];
  __shared__ uint64_t qb[kMaxWords][kTile], kb[kMaxWords][kTile];
  __shared__ int q_starts[kTile + 1], kv_starts[kTile + 1];
  __shared__ int n_qr, n_kr, pos_row, pos_col, row_off;
  __shared__ int rtot[kRankChunk], ctot[kRankChunk];
  const int nt = out.nt;
  const int b = blockIdx.y;
  int qt, kt;
  tri_tile(blockIdx.x, qt, kt);
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  // Work-group (0, 0) of a mask row also writes its launch orders, and
  // work-group (0, qt) the row's first bitmap slot (kv_bits_off).
  if (kt == 0 && qt == 0) rank_orders(out, b, rtot, ctot);
  if (kt == 0 && wave == 0) {
    const int off = row_slot_offset(out, b * nt + qt, lane);
    if (lane == 0) out.kv_bits_off[(size_t)b * nt + qt] = off;
  }
  const int8_t* grid = out.tile_class + (size_t)b * nt * nt;
  if (grid[(size_t)qt * nt + kt] != kPartial) return;
  const int32_t* doc = doc_all + (size_t)b * T;
  const uint64_t* qbits = qbits_all + (size_t)b * words * T;
  const uint64_t* kvbits = kvbits_all + (size_t)b * words * T;
  const int q0 = qt * kTile, k0 = kt * kTile;

  if (wave == 0) {  // position among the row's partial tiles (columns < kt)
    int cnt = 0;
    for (int c = 0; c < kt; c += 64) {
      const int j = c + lane;
      cnt += __popcll(__ballot(j < kt && grid[(size_t)qt * nt + j] == kPartial));
    }
    const int off = row_slot_offset(out, b * nt + qt, lane);
    if (lane == 0) {
      pos_row = cnt;
      row_off = off;
    }
  } else if (wave == 1) {  // position among the column's partial tiles (rows < qt)
    int cnt = 0;
    for (int c = 0; c < qt; c += 64) {
      const int j = c + lane;
      cnt += __popcll(__ballot(j < qt && grid[(size_t)j * nt + kt] == kPartial));
    }
    if (lane == 0) pos_col = cnt;
  } else if (wave == 2) {
    const int n = wave_runs(doc, qbits, words, T, q0, q_starts);
    if (lane == 0) n_qr = n;
  } else {
    const int n = wave_runs(doc, kvbits, words, T, k0, kv_starts);
    if (lane == 0) n_kr = n;
  }
  if (tid < kTile) {
    const int t = q0 + tid;
    qdoc[tid] = t < T ? doc[t] : 0;
    for (int w = 0; w < words; ++w) qb[w][tid] = t < T ? qbits[(size_t)w * T + t] : 0ull;
  } else {
    const int c = tid - kTile, t = k0 + c;
    kdoc[c] = t < T ? doc[t] : 0;
    for (int w = 0; w < words; ++w) kb[w][c] = t < T ? kvbits[(size_t)w * T + t] : 0ull;
  }
  __syncthreads();
  const int slot = row_off + pos_row;
  uint32_t acc[4] = {0u, 0u, 0u, 0u};
  if (tid < kTile) {
    // row orientation: query q0 + tid against the tile's keys
    const int r = tid, q = q0 + r;
    if (q < T) {
      for (int s = 0; s < n_kr; ++s) {
        const int a = kv_starts[s], z = kv_starts[s + 1];
        if (lds_pair_allowed(qdoc[r], kdoc[a], &qb[0][r], &kb[0][a], kTile, kTile, words))
          set_bit_range(acc, a, z);
      }
      // causal: keys k0 + kk <= q; padding keys (>= T) are outside every run
      const int lim = q - k0 + 1;  // allowed kk < lim
      uint32_t cm[4] = {0u, 0u, 0u, 0u};
      set_bit_range(cm, 0, min(max(lim, 0), kTile));
#pragma unroll
      for (int w = 0; w < 4; ++w) acc[w] &= cm[w];
    }
  } else {
    // column orientation: key k0 + c against the tile's queries
    const int c = tid - kTile, key = k0 + c;
    if (key < T) {
      for (int s = 0; s < n_qr; ++s) {
        const int a = q_starts[s], z = q_starts[s + 1];
        if (lds_pair_allowed(qdoc[a], kdoc[c], &qb[0][a], &kb[0][c], kTile, kTile, words))
          set_bit_range(acc, a, z);
      }
      // causal: queries q0 + qq >= key
      const int from = key - q0;  // allowed qq >= from
      uint32_t cm[4] = {0u, 0u, 0u, 0u};
      set_bit_range(cm, min(max(from, 0), kTile), kTile);
#pragma unroll
      for (int w = 0; w < 4; ++w) acc[w] &= cm[w];
    }
  }
  uint32_t* dst = out.tile_bits + (size_t)slot * kTileBitsWords +
                  (tid < kTile ? tid * 4 : kTile * 4 + (tid - kTile) * 4);
  *reinterpret_cast<uint4*>(dst) = make_uint4(acc[0], acc[1], acc[2], acc[3]);
  if (tid == 0) out.q_bits_slot[((size_t)b * nt + kt) * nt + pos_col] = slot;
}

hipError_t launch_mask_meta(const int32_t* doc, const uint64_t* qbits, const uint64_t* kvbits,
                            int T, int words, const MaskOut& out, hipStream_t stream) {
  const int nt = out.nt;
  if (nt == 0 || out.Bm == 0) return hipSuccess;
  const dim3 tiles((unsigned)(nt * (nt + 1) / 2), out.Bm);
  hipLaunchKernelGGL(mask_classify_tiles, tiles, dim3(64), 0, stream, doc, qbits, kvbits, T,
                     words, out);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(mask_lists, dim3(nt, out.Bm), dim3(kThreads), 0, stream, out);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(mask_tile_bits, tiles, dim3(kThreads), 0, stream, doc, qbits, kvbits, T,
                     words, out);
  return hipGetLastError();
}

}  // namespace t2t
