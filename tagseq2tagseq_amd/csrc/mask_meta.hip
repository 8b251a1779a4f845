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
// Launches: (1) classify every tile, (2) row and column lists with the
// bitmap slot tables, (3) partial-tile bitmaps; in the third each row's
// column-0 work-group also ranks its row and column for the launch orders,
// so no launch waits on a single work-group.  The bitmap of tile (b, qt, kt) lives in slot
// b * nt (nt + 1) / 2 + qt (qt + 1) / 2 + kt (a fixed position in the lower
// triangle), so no work-group has to count the partial tiles before its own.
// Every work-group first copies the signatures (doc id, grant words) of its
// tokens into LDS with one load per token and word, and finds the runs and
// evaluates the predicate from there.
#include "attn_kernels.h"

namespace t2t {

namespace {

// Lower-triangle tile of linear index L (row-major over qt, kt <= qt).
__device__ __forceinline__ void tri_tile(int L, int& qt, int& kt) {
  int r = (int)((sqrtf(8.f * (float)L + 1.f) - 1.f) * 0.5f);
  while ((int64_t)(r + 1) * (r + 2) / 2 <= L) ++r;  // exact despite float rounding
  while ((int64_t)r * (r + 1) / 2 > L) --r;
  qt = r;
  kt = L - (int)((int64_t)r * (r + 1) / 2);
}

// Signatures (doc id, grant words) of the 128 tokens of one tile side, in
// dynamic LDS: doc[i], bits[w * 128 + i].
struct TileSigs {
  int32_t* doc;
  uint64_t* bits;
};

// Bytes of dynamic LDS for the query and key signatures of one tile.
__host__ __device__ constexpr int sig_lds_bytes(int words) {
  return 2 * kTile * (int)(sizeof(int32_t) + words * sizeof(uint64_t));
}

// The query-side and key-side views of that LDS (bits first: 8-byte aligned).
__device__ __forceinline__ void sig_views(unsigned char* lds, int words, TileSigs& q,
                                          TileSigs& k) {
  q.bits = reinterpret_cast<uint64_t*>(lds);
  k.bits = q.bits + words * kTile;
  q.doc = reinterpret_cast<int32_t*>(k.bits + words * kTile);
  k.doc = q.doc + kTile;
}

// Thread `i` (< 128) copies the signature of token base + i (zeros past T).
__device__ __forceinline__ void load_sigs(const TileSigs& s, const int32_t* doc,
                                          const uint64_t* bits, int words, int T, int base,
                                          int i) {
  const int t = base + i;
  s.doc[i] = t < T ? doc[t] : 0;
  for (int w = 0; w < words; ++w) s.bits[w * kTile + i] = t < T ? bits[(size_t)w * T + t] : 0ull;
}

__device__ __forceinline__ bool sigs_eq(const TileSigs& s, int a, int b, int words) {
  if (s.doc[a] != s.doc[b]) return false;
  for (int w = 0; w < words; ++w)
    if (s.bits[w * kTile + a] != s.bits[w * kTile + b]) return false;
  return true;
}

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }

__device__ __forceinline__ int lanes_below(uint64_t mask) {
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32),
                                   __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0));
}

// One wave over the LDS signatures of one tile side (the first nvalid tokens
// are real): writes the start offsets of runs of identical signatures into
// starts[], terminated by starts[n] = nvalid; returns n.
__device__ int wave_runs(const TileSigs& s, int words, int nvalid, int* starts) {
  const int lane = lane_id();
  int flag[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int t = lane + 64 * h;
    flag[h] = t < nvalid && (t == 0 || !sigs_eq(s, t, t - 1, words));
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

// The non-causal part of the predicate for query-side token a and key-side
// token c of a tile: same document, or a shared grant bit.
__device__ __forceinline__ bool sigs_allowed(const TileSigs& q, int a, const TileSigs& k, int c,
                                             int words) {
  if (q.doc[a] == k.doc[c]) return true;
  for (int w = 0; w < words; ++w)
    if (q.bits[w * kTile + a] & k.bits[w * kTile + c]) return true;
  return false;
}

// First bitmap slot of mask row b's tile row qt (slot of tile (qt, kt) =
// this + kt).
// (t2t_mask_meta keeps every slot index below 2^31.)
__device__ __forceinline__ int tri_slot(int b, int nt, int qt) {
  return (int)((int64_t)b * ((int64_t)nt * (nt + 1) / 2) + (int64_t)qt * (qt + 1) / 2);
}

// Compact one 0/1 row of `n` byte flags (flag = (cls == want)) into the
// ordered list of torch's _dense_to_ordered: set positions ascending, then
// unset positions ascending.  One wave; `cls` is read with stride `stride`.
__device__ void wave_ordered(const int8_t* cls, int stride, int n, int8_t want,
                             int32_t* num_out, int32_t* idx_out, int32_t* slot_out = nullptr,
                             int slot_b = 0, int slot_col = 0) {
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
    if (f) {
      idx_out[set_base + lanes_below(ms)] = i;
      // bitmap slot of the column's partial tile in row i
      if (slot_out) slot_out[set_base + lanes_below(ms)] = tri_slot(slot_b, n, i) + slot_col;
    } else if (in) {
      idx_out[unset_base + lanes_below(mu)] = i;
    }
    set_base += __popcll(ms);
    unset_base += __popcll(mu);
  }
  if (lane == 0) *num_out = total;
}

}  // namespace

// (1) grid (nt (nt + 1) / 2, Bm); block 128: one work-group decides one tile
// of the lower triangle (kt <= qt) and writes its mirror above the diagonal
// as skip (every pair there has kv > q).  Thread i copies the signatures of
// query q0 + i and key k0 + i; waves 0 and 1 then find the query and key runs
// side by side, and wave 0 evaluates the run pairs.
__global__ __launch_bounds__(128) void mask_classify_tiles(
    const int32_t* __restrict__ doc_all, const uint64_t* __restrict__ qbits_all,
    const uint64_t* __restrict__ kvbits_all, int T, int words, MaskOut out) {
  extern __shared__ __align__(16) unsigned char sig_lds[];
  __shared__ int q_starts[kTile + 1], kv_starts[kTile + 1];
  __shared__ int n_qr, n_kr;
  TileSigs qs, ks;
  sig_views(sig_lds, words, qs, ks);
  const int nt = out.nt;
  const int b = blockIdx.y;
  int qt, kt;
  tri_tile(blockIdx.x, qt, kt);
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  int8_t* dst = out.tile_class + ((size_t)b * nt + qt) * nt + kt;
  if (tid == 0 && kt < qt) out.tile_class[((size_t)b * nt + kt) * nt + qt] = kSkip;
  const int32_t* doc = doc_all + (size_t)b * T;
  const int q0 = qt * kTile, k0 = kt * kTile;
  const int qvalid = min(kTile, T - q0), kvalid = min(kTile, T - k0);
  load_sigs(qs, doc, qbits_all + (size_t)b * words * T, words, T, q0, tid);
  load_sigs(ks, doc, kvbits_all + (size_t)b * words * T, words, T, k0, tid);
  __syncthreads();
  if (wave == 0) {
    const int n = wave_runs(qs, words, qvalid, q_starts);
    if (lane == 0) n_qr = n;
  } else {
    const int n = wave_runs(ks, words, kvalid, kv_starts);
    if (lane == 0) n_kr = n;
  }
  __syncthreads();
  if (wave != 0) return;
  const int nqr = n_qr, nkr = n_kr;
  // Padding rows/columns are False pairs: such a tile can never be full.
  bool any_true = false;
  bool any_false = (qvalid < kTile) || (kvalid < kTile);
  const int npairs = nqr * nkr;
  for (int p0 = 0; p0 < npairs; p0 += 64) {
    const int p = p0 + lane;
    bool t = false, f = false;
    if (p < npairs) {
      const int r = p / nkr, s = p - r * nkr;
      const int qa = q_starts[r], qb = q_starts[r + 1];
      const int ka = kv_starts[s], kb = kv_starts[s + 1];
      const bool v = sigs_allowed(qs, qa, ks, ka, words);
      const bool exists_ge = (q0 + qb - 1) >= (k0 + ka);  // some pair with q >= kv
      const bool exists_lt = (q0 + qa) < (k0 + kb - 1);   // some pair with q < kv
      t = v && exists_ge;
      f = !v || exists_lt;
    }
    any_true = any_true || (__ballot(t) != 0);
    any_false = any_false || (__ballot(f) != 0);
    if (any_true && any_false) break;
  }
  if (lane == 0) *dst = any_true ? (any_false ? kPartial : kFull) : kSkip;
}

// (2) grid (nt, Bm); block 256.  Wave 0/1: partial / full list of row x
// (and the row's first bitmap slot); wave 2/3: partial / full list of column
// x (and the slots of the column's partial tiles).
__global__ __launch_bounds__(kThreads) void mask_lists(MaskOut out) {
  const int nt = out.nt;
  const int i = blockIdx.x, b = blockIdx.y;
  const int wave = threadIdx.x >> 6;
  const int8_t* grid = out.tile_class + (size_t)b * nt * nt;
  const size_t r = (size_t)b * nt + i;
  if (threadIdx.x == 0) out.kv_bits_off[r] = tri_slot(b, nt, i);
  if (wave == 0)
    wave_ordered(grid + (size_t)i * nt, 1, nt, kPartial, out.kv_num + r, out.kv_idx + r * nt);
  else if (wave == 1)
    wave_ordered(grid + (size_t)i * nt, 1, nt, kFull, out.full_kv_num + r, out.full_kv_idx + r * nt);
  else if (wave == 2)
    wave_ordered(grid + i, nt, nt, kPartial, out.q_num + r, out.q_idx + r * nt,
                 out.q_bits_slot + r * nt, b, i);
  else
    wave_ordered(grid + i, nt, nt, kFull, out.full_q_num + r, out.full_q_idx + r * nt);
}

namespace {

// Launch orders: rows / columns ranked by descending non-skip tile count in
// buckets of kOrderBucket tiles, rows of one bucket by descending index and
// columns by ascending index -- longest first for the load balance, and
// within a bucket neighbouring rows (which mostly read the same K/V tiles)
// or columns back to back, so that a cache serves the shared tiles.
constexpr int kOrderBucket = 2;

// By the whole work-group: the rank of row i and of column i of mask row b
// in those orders, written as row_order[rank] = i and col_order[rank] = i
// (by each row's own work-group, so the ranking is spread over the launch
// instead of one work-group doing all of it).
__device__ void rank_row_col(const MaskOut& out, int b, int i, int* red) {
  const int nt = out.nt, tid = threadIdx.x;
  const int32_t* rn = out.kv_num + (size_t)b * nt;
  const int32_t* rf = out.full_kv_num + (size_t)b * nt;
  const int32_t* cn = out.q_num + (size_t)b * nt;
  const int32_t* cf = out.full_q_num + (size_t)b * nt;
  const int kr = (rn[i] + rf[i]) / kOrderBucket, kc = (cn[i] + cf[i]) / kOrderBucket;
  int rr = 0, rc = 0;
  for (int j = tid; j < nt; j += kThreads) {
    const int jr = (rn[j] + rf[j]) / kOrderBucket, jc = (cn[j] + cf[j]) / kOrderBucket;
    rr += (jr > kr) || (jr == kr && j > i);
    rc += (jc > kc) || (jc == kc && j < i);
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    rr += __shfl_xor(rr, off, 64);
    rc += __shfl_xor(rc, off, 64);
  }
  if ((tid & 63) == 0) {
    red[2 * (tid >> 6)] = rr;
    red[2 * (tid >> 6) + 1] = rc;
  }
  __syncthreads();
  if (tid == 0) {
    int sr = 0, sc = 0;
    for (int w = 0; w < kThreads / 64; ++w) {
      sr += red[2 * w];
      sc += red[2 * w + 1];
    }
    out.row_order[(size_t)b * nt + sr] = i;
    out.col_order[(size_t)b * nt + sc] = i;
  }
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

}  // namespace

// (3) grid (nt (nt + 1) / 2, Bm); block 256.  For a partial tile of the lower
// triangle: both bitmap orientations, into slot tri_slot(b, nt, qt) + kt.
// Work-group (qt, 0) also ranks row qt and column qt for the launch orders.
// Threads 0..127 copy the query signatures, 128..255 the key signatures;
// waves 0 and 1 find the runs.  A row of the bitmap is built run by run:
// within a run of keys with one signature the non-causal predicate is
// constant, so one evaluation sets a whole bit range; the causal and padding
// limits are applied last.
__global__ __launch_bounds__(kThreads) void mask_tile_bits(
    const int32_t* __restrict__ doc_all, const uint64_t* __restrict__ qbits_all,
    const uint64_t* __restrict__ kvbits_all, int T, int words, MaskOut out) {
  extern __shared__ __align__(16) unsigned char sig_lds[];
  __shared__ int q_starts[kTile + 1], kv_starts[kTile + 1];
  __shared__ int n_qr, n_kr;
  __shared__ int red[2 * kThreads / 64];
  TileSigs qs, ks;
  sig_views(sig_lds, words, qs, ks);
  const int nt = out.nt;
  const int b = blockIdx.y;
  int qt, kt;
  tri_tile(blockIdx.x, qt, kt);
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  if (kt == 0) rank_row_col(out, b, qt, red);
  if (out.tile_class[((size_t)b * nt + qt) * nt + kt] != kPartial) return;
  const int32_t* doc = doc_all + (size_t)b * T;
  const int q0 = qt * kTile, k0 = kt * kTile;
  if (tid < kTile)
    load_sigs(qs, doc, qbits_all + (size_t)b * words * T, words, T, q0, tid);
  else
    load_sigs(ks, doc, kvbits_all + (size_t)b * words * T, words, T, k0, tid - kTile);
  __syncthreads();
  if (wave == 0) {
    const int n = wave_runs(qs, words, min(kTile, T - q0), q_starts);
    if (lane == 0) n_qr = n;
  } else if (wave == 1) {
    const int n = wave_runs(ks, words, min(kTile, T - k0), kv_starts);
    if (lane == 0) n_kr = n;
  }
  __syncthreads();
  uint32_t acc[4] = {0u, 0u, 0u, 0u};
  if (tid < kTile) {
    // row orientation: query q0 + tid against the tile's keys
    const int r = tid, q = q0 + r;
    if (q < T) {
      for (int s = 0; s < n_kr; ++s) {
        const int a = kv_starts[s], z = kv_starts[s + 1];
        if (sigs_allowed(qs, r, ks, a, words)) set_bit_range(acc, a, z);
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
        if (sigs_allowed(qs, a, ks, c, words)) set_bit_range(acc, a, z);
      }
      // causal: queries q0 + qq >= key
      const int from = key - q0;  // allowed qq >= from
      uint32_t cm[4] = {0u, 0u, 0u, 0u};
      set_bit_range(cm, min(max(from, 0), kTile), kTile);
#pragma unroll
      for (int w = 0; w < 4; ++w) acc[w] &= cm[w];
    }
  }
  const int slot = tri_slot(b, nt, qt) + kt;
  uint32_t* dst = out.tile_bits + (size_t)slot * kTileBitsWords +
                  (tid < kTile ? tid * 4 : kTile * 4 + (tid - kTile) * 4);
  *reinterpret_cast<uint4*>(dst) = make_uint4(acc[0], acc[1], acc[2], acc[3]);
}

hipError_t launch_mask_meta(const int32_t* doc, const uint64_t* qbits, const uint64_t* kvbits,
                            int T, int words, const MaskOut& out, hipStream_t stream) {
  const int nt = out.nt;
  if (nt == 0 || out.Bm == 0) return hipSuccess;
  const dim3 tiles((unsigned)((int64_t)nt * (nt + 1) / 2), out.Bm);
  const int sig_bytes = sig_lds_bytes(words);
  hipLaunchKernelGGL(mask_classify_tiles, tiles, dim3(128), sig_bytes, stream, doc, qbits, kvbits,
                     T, words, out);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(mask_lists, dim3(nt, out.Bm), dim3(kThreads), 0, stream, out);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(mask_tile_bits, tiles, dim3(kThreads), sig_bytes, stream, doc, qbits, kvbits,
                     T, words, out);
  return hipGetLastError();
}

}  // namespace t2t
