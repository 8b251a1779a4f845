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
// Launches: (1) one wave per tile of the lower triangle: its class and, for a
// partial tile, both orientations of its bitmap; (2) row and column lists with
// the bitmap slot tables; (3) launch orders, each row's work-group ranking
// its row and its column (no launch waits on a single work-group).  The
// bitmap of tile (b, qt, kt) lives in slot b * nt (nt + 1) / 2 + qt (qt + 1) / 2
// + kt (a fixed position in the lower triangle), so no wave has to count the
// partial tiles before its own.
// The runs are found in registers: lane l of a wave holds the signatures
// (doc id, grant words) of tokens l and 64 + l of a tile side, a whole-wave
// lane shift compares each token with the one before it, and a ballot marks
// the run starts of the 128 tokens as a 128-bit mask; a run's signature is
// that of its first token, read from the lane holding it.  The grant-word
// count is a template parameter, so a signature is exactly the registers it
// needs and no loop over words is decided at run time.
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

// First bitmap slot of mask row b's tile row qt (slot of tile (qt, kt) =
// this + kt).
// (t2t_mask_meta keeps every slot index below 2^31.)
__device__ __forceinline__ int tri_slot(int b, int nt, int qt) {
  return (int)((int64_t)b * ((int64_t)nt * (nt + 1) / 2) + (int64_t)qt * (qt + 1) / 2);
}

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

// A token's signature: document id and W grant words (zeros past T).
template <int W>
struct Sig {
  int32_t doc;
  uint64_t w[W > 0 ? W : 1];
};

template <int W>
__device__ __forceinline__ Sig<W> load_sig(const int32_t* doc, const uint64_t* bits, int T,
                                           int t) {
  // loads from a clamped index (T >= 1), so that none sits in a branch
  const int tc = min(t, T - 1);
  const bool in = t < T;
  Sig<W> g;
  const int32_t d = doc[tc];
  g.doc = in ? d : 0;
#pragma unroll
  for (int w = 0; w < W; ++w) {
    const uint64_t v = bits[(size_t)w * T + tc];
    g.w[w] = in ? v : 0ull;
  }
  return g;
}

template <int W>
__device__ __forceinline__ bool sig_eq(const Sig<W>& a, const Sig<W>& b) {
  bool eq = a.doc == b.doc;
#pragma unroll
  for (int w = 0; w < W; ++w) eq = eq && a.w[w] == b.w[w];
  return eq;
}

// The non-causal part of the predicate for a query-side signature q and a
// key-side signature k: same document, or a shared grant bit.
template <int W>
__device__ __forceinline__ bool sig_allowed(const Sig<W>& q, const Sig<W>& k) {
  bool ok = q.doc == k.doc;
#pragma unroll
  for (int w = 0; w < W; ++w) ok = ok || (q.w[w] & k.w[w]) != 0ull;
  return ok;
}

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }

__device__ __forceinline__ int lanes_below(uint64_t mask) {
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32),
                                   __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0));
}

__device__ __forceinline__ uint64_t join64(uint32_t lo, uint32_t hi) {
  return ((uint64_t)hi << 32) | lo;
}

// Lane src's signature (src the same for every lane).
template <int W>
__device__ __forceinline__ Sig<W> readlane_sig(const Sig<W>& g, int src) {
  Sig<W> r;
  r.doc = __builtin_amdgcn_readlane(g.doc, src);
#pragma unroll
  for (int w = 0; w < W; ++w)
    r.w[w] = join64((uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)g.w[w], src),
                    (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(g.w[w] >> 32), src));
  return r;
}

// Every lane's predecessor within the wave (lane l gets lane l - 1's
// signature; lane 0 gets `first`): a whole-wave right shift by one lane (DPP).
__device__ __forceinline__ int shift_up(int first, int v) {
  return __builtin_amdgcn_update_dpp(first, v, 0x138, 0xf, 0xf, false);
}

template <int W>
__device__ __forceinline__ Sig<W> shift_up_sig(const Sig<W>& g, const Sig<W>& first) {
  Sig<W> r;
  r.doc = shift_up(first.doc, g.doc);
#pragma unroll
  for (int w = 0; w < W; ++w)
    r.w[w] = join64((uint32_t)shift_up((int)(uint32_t)first.w[w], (int)(uint32_t)g.w[w]),
                    (uint32_t)shift_up((int)(uint32_t)(first.w[w] >> 32),
                                       (int)(uint32_t)(g.w[w] >> 32)));
  return r;
}

// The 128 tokens base .. base + 127 of one tile side (the first nvalid are
// real), held by one wave: lane l holds tokens base + l (sig[0]) and
// base + 64 + l (sig[1]).  Bit i of the 128-bit run mask (m[0] bits 0-63,
// m[1] bits 64-127) is set iff token base + i starts a run of identical
// signatures.
template <int W>
struct TileSide {
  Sig<W> sig[2];
  uint64_t m[2];
};

// Marks the run starts of a side whose signatures the wave already holds.
template <int W>
__device__ __forceinline__ TileSide<W> mark_runs(const Sig<W>& s0, const Sig<W>& s1, int nvalid) {
  const int lane = lane_id();
  TileSide<W> s;
  s.sig[0] = s0;
  s.sig[1] = s1;
  // predecessor of each token: lane - 1 of the same half; lane 0 of the
  // second half takes lane 63 of the first (lane 0 of the first half starts
  // a run whatever it is compared with)
  const Sig<W> last0 = readlane_sig(s0, 63);
  const Sig<W> p0 = shift_up_sig(s0, last0);
  const Sig<W> p1 = shift_up_sig(s1, last0);
  const bool f0 = lane < nvalid && (lane == 0 || !sig_eq(s0, p0));
  const bool f1 = 64 + lane < nvalid && !sig_eq(s1, p1);
  s.m[0] = __ballot(f0);
  s.m[1] = __ballot(f1);
  return s;
}

// Calls f(a, z, sig) for every run [a, z) of the side in order (a
// wave-uniform loop; sig = the run's signature) while go() holds.
template <int W, class F, class G>
__device__ __forceinline__ void for_each_run(const TileSide<W>& s, int nvalid, G go, F f) {
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    for (uint64_t m = s.m[h]; m && go(); m &= m - 1) {
      const int a = 64 * h + __ffsll((long long)m) - 1;
      const uint64_t rest = m & (m - 1);
      const int z = rest ? 64 * h + __ffsll((long long)rest) - 1
                         : (h == 0 && s.m[1] ? 64 + __ffsll((long long)s.m[1]) - 1 : nvalid);
      f(a, z, readlane_sig(s.sig[h], a & 63));
    }
  }
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

// (1) grid (ceil(nt (nt + 1) / 2 / 4), Bm); block 256: each wave takes one
// tile of the lower triangle (kt <= qt; linear index 4 x + wave, row-major)
// and writes its mirror above the diagonal as skip (every pair there has
// kv > q).  Class: each query run against every key token (lanes over key
// tokens, a loop over query runs), stopping once the tile is known to be
// partial.
// Bitmap of a partial tile: lane l builds rows l and 64 + l (those queries
// against the key runs) and columns l and 64 + l (those keys against the
// query runs); within a run the non-causal predicate is constant, so one
// evaluation sets a whole bit range; the causal and padding limits come last.
constexpr int kTileWaves = kThreads / 64;

template <int W>
__global__ __launch_bounds__(kThreads) void mask_tiles(const int32_t* __restrict__ doc_all,
                                                       const uint64_t* __restrict__ qbits_all,
                                                       const uint64_t* __restrict__ kvbits_all,
                                                       int T, MaskOut out) {
  const int nt = out.nt;
  const int b = blockIdx.y;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t L = (int64_t)blockIdx.x * kTileWaves + wave;
  if (L >= (int64_t)nt * (nt + 1) / 2) return;
  int qt, kt;
  tri_tile((int)L, qt, kt);
  const int lane = lane_id();
  if (lane == 0 && kt < qt) out.tile_class[((size_t)b * nt + kt) * nt + qt] = kSkip;
  const int32_t* doc = doc_all + (size_t)b * T;
  const int q0 = qt * kTile, k0 = kt * kTile;
  const int qvalid = min(kTile, T - q0), kvalid = min(kTile, T - k0);
  // query tokens q0 + lane and q0 + 64 + lane, key tokens k0 + lane and
  // k0 + 64 + lane
  const uint64_t* qbits = qbits_all + (size_t)b * W * T;
  const uint64_t* kbits = kvbits_all + (size_t)b * W * T;
  const Sig<W> qsig[2] = {load_sig<W>(doc, qbits, T, q0 + lane),
                          load_sig<W>(doc, qbits, T, q0 + 64 + lane)};
  const Sig<W> ksig[2] = {load_sig<W>(doc, kbits, T, k0 + lane),
                          load_sig<W>(doc, kbits, T, k0 + 64 + lane)};
  const TileSide<W> qs = mark_runs(qsig[0], qsig[1], qvalid);
  // Padding rows/columns are False pairs: such a tile can never be full.
  bool any_true = false;
  bool any_false = (qvalid < kTile) || (kvalid < kTile);
  auto open = [&]() { return !(any_true && any_false); };
  // each query run against every key token: within the run the non-causal
  // predicate is constant, and the run's first and last query bound the
  // causal part
  for_each_run(qs, qvalid, open, [&](int qa, int qb, const Sig<W>& rsig) {
    bool t = false, f = false;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int kk = lane + 64 * i;
      const bool v = sig_allowed(rsig, ksig[i]);
      const bool exists_ge = q0 + qb - 1 >= k0 + kk;  // some pair with q >= kv
      const bool exists_lt = q0 + qa < k0 + kk;       // some pair with q < kv
      t = t || (kk < kvalid && v && exists_ge);
      f = f || (kk < kvalid && (!v || exists_lt));
    }
    any_true = any_true || (__ballot(t) != 0);
    any_false = any_false || (__ballot(f) != 0);
  });
  const int8_t cls = any_true ? (any_false ? kPartial : kFull) : kSkip;
  if (lane == 0) out.tile_class[((size_t)b * nt + qt) * nt + kt] = cls;
  if (cls != kPartial) return;

  const TileSide<W> ks = mark_runs(ksig[0], ksig[1], kvalid);
  auto always = []() { return true; };
  uint32_t rows[2][4] = {}, cols[2][4] = {};
  for_each_run(ks, kvalid, always, [&](int a, int z, const Sig<W>& rsig) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
      if (sig_allowed(qsig[i], rsig)) set_bit_range(rows[i], a, z);
  });
  for_each_run(qs, qvalid, always, [&](int a, int z, const Sig<W>& rsig) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
      if (sig_allowed(rsig, ksig[i])) set_bit_range(cols[i], a, z);
  });
  uint32_t* dst = out.tile_bits + (size_t)(tri_slot(b, nt, qt) + kt) * kTileBitsWords;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int t = lane + 64 * i;
    // causal: query q0 + t sees keys k0 + kk <= q0 + t; key k0 + t is seen by
    // queries q0 + qq >= k0 + t; tokens past T keep no bit (padding keys and
    // queries lie outside every run)
    uint32_t rm[4] = {}, cm[4] = {};
    if (kt < qt) {
      // below the diagonal every key precedes every query
      const uint32_t all = q0 + t < T ? ~0u : 0u;
      rm[0] = rm[1] = rm[2] = rm[3] = all;
      cm[0] = cm[1] = cm[2] = cm[3] = ~0u;
    } else {
      if (q0 + t < T) set_bit_range(rm, 0, min(max(q0 + t - k0 + 1, 0), kTile));
      if (k0 + t < T) set_bit_range(cm, min(max(k0 + t - q0, 0), kTile), kTile);
    }
    *reinterpret_cast<uint4*>(dst + t * 4) =
        make_uint4(rows[i][0] & rm[0], rows[i][1] & rm[1], rows[i][2] & rm[2], rows[i][3] & rm[3]);
    *reinterpret_cast<uint4*>(dst + (kTile + t) * 4) =
        make_uint4(cols[i][0] & cm[0], cols[i][1] & cm[1], cols[i][2] & cm[2], cols[i][3] & cm[3]);
  }
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

// (3) grid (nt, Bm); block 256: the launch-order ranks of row x and column x.
__global__ __launch_bounds__(kThreads) void mask_rank(MaskOut out) {
  __shared__ int red[2 * kThreads / 64];
  rank_row_col(out, blockIdx.y, blockIdx.x, red);
}

hipError_t launch_mask_meta(const int32_t* doc, const uint64_t* qbits, const uint64_t* kvbits,
                            int T, int words, const MaskOut& out, hipStream_t stream) {
  const int nt = out.nt;
  if (nt == 0 || out.Bm == 0) return hipSuccess;
  if (words < 0 || words > kMaxWords) return hipErrorInvalidValue;
  const int64_t n_tri = (int64_t)nt * (nt + 1) / 2;
  const dim3 tiles((unsigned)((n_tri + kTileWaves - 1) / kTileWaves), out.Bm);
  using TilesFn = void (*)(const int32_t*, const uint64_t*, const uint64_t*, int, MaskOut);
  static constexpr TilesFn kTilesByWords[kMaxWords + 1] = {
      mask_tiles<0>, mask_tiles<1>, mask_tiles<2>, mask_tiles<3>, mask_tiles<4>,
      mask_tiles<5>, mask_tiles<6>, mask_tiles<7>, mask_tiles<8>};
  static_assert(kMaxWords == 8, "one instantiation per grant-word count");
  hipLaunchKernelGGL(kTilesByWords[words], tiles, dim3(kThreads), 0, stream, doc, qbits, kvbits,
                     T, out);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(mask_lists, dim3(nt, out.Bm), dim3(kThreads), 0, stream, out);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(mask_rank, dim3(nt, out.Bm), dim3(kThreads), 0, stream, out);
  return hipGetLastError();
}

}  // namespace t2t
