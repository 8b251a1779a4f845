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
// The runs are found in registers: each lane loads the signatures (doc id,
// grant words) of its tokens and of the tokens just before them, a ballot of
// "differs from the previous token" marks the run starts of 128 tokens as a
// 128-bit mask, and the signature of a run is read at its first token (a
// cached load); no work-group stages signatures in LDS or waits at a barrier
// for them.
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

// A token's signature: document id and grant words (zeros past T).  KW is
// the compile-time bound on the words (registers are held for KW of them);
// the `words` arguments below give how many are real (words <= KW).
template <int KW>
struct Sig {
  int32_t doc;
  uint64_t w[KW > 0 ? KW : 1];
};

template <int KW>
__device__ __forceinline__ Sig<KW> load_sig(const int32_t* doc, const uint64_t* bits, int words,
                                            int T, int t) {
  Sig<KW> g;
  const bool in = t < T;
  g.doc = in ? doc[t] : 0;
#pragma unroll
  for (int w = 0; w < KW; ++w) g.w[w] = (in && w < words) ? bits[(size_t)w * T + t] : 0ull;
  return g;
}

template <int KW>
__device__ __forceinline__ bool sig_eq(const Sig<KW>& a, const Sig<KW>& b, int words) {
  bool eq = a.doc == b.doc;
#pragma unroll
  for (int w = 0; w < KW; ++w)
    if (w < words) eq = eq && a.w[w] == b.w[w];
  return eq;
}

// The non-causal part of the predicate for a query-side signature q and a
// key-side signature k: same document, or a shared grant bit.
template <int KW>
__device__ __forceinline__ bool sig_allowed(const Sig<KW>& q, const Sig<KW>& k, int words) {
  bool ok = q.doc == k.doc;
#pragma unroll
  for (int w = 0; w < KW; ++w)
    if (w < words) ok = ok || (q.w[w] & k.w[w]) != 0ull;
  return ok;
}

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }

__device__ __forceinline__ int lanes_below(uint64_t mask) {
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32),
                                   __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0));
}

// Lane src's signature, fetched by every lane (src may differ per lane).
template <int KW>
__device__ __forceinline__ Sig<KW> shfl_sig(const Sig<KW>& g, int src, int words) {
  Sig<KW> r;
  r.doc = __shfl(g.doc, src, 64);
#pragma unroll
  for (int w = 0; w < KW; ++w) {
    r.w[w] = 0ull;
    if (w < words) {
      const uint32_t lo = (uint32_t)__shfl((int)(uint32_t)g.w[w], src, 64);
      const uint32_t hi = (uint32_t)__shfl((int)(uint32_t)(g.w[w] >> 32), src, 64);
      r.w[w] = ((uint64_t)hi << 32) | lo;
    }
  }
  return r;
}

// Lane src's signature (src the same for every lane).
template <int KW>
__device__ __forceinline__ Sig<KW> readlane_sig(const Sig<KW>& g, int src, int words) {
  Sig<KW> r;
  r.doc = __builtin_amdgcn_readlane(g.doc, src);
#pragma unroll
  for (int w = 0; w < KW; ++w) {
    r.w[w] = 0ull;
    if (w < words) {
      const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)g.w[w], src);
      const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(g.w[w] >> 32), src);
      r.w[w] = ((uint64_t)hi << 32) | lo;
    }
  }
  return r;
}

// The 128 tokens base .. base + 127 of one tile side (the first nvalid are
// real), held by one wave: lane l holds tokens base + l (sig[0]) and
// base + 64 + l (sig[1]).  Bit i of the 128-bit run mask (m[0] bits 0-63,
// m[1] bits 64-127) is set iff token base + i starts a run of identical
// signatures.
template <int KW>
struct TileSide {
  Sig<KW> sig[2];
  uint64_t m[2];
};

template <int KW>
__device__ __forceinline__ TileSide<KW> wave_tile_side(const int32_t* doc, const uint64_t* bits,
                                                       int words, int T, int base, int nvalid) {
  const int lane = lane_id();
  TileSide<KW> s;
  s.sig[0] = load_sig<KW>(doc, bits, words, T, base + lane);
  s.sig[1] = load_sig<KW>(doc, bits, words, T, base + 64 + lane);
  // predecessor of each token: lane - 1 of the same half; lane 0 of the
  // second half takes lane 63 of the first
  const int up = (lane + 63) & 63;
  const Sig<KW> p0 = shfl_sig(s.sig[0], up, words);
  const Sig<KW> t1 = shfl_sig(s.sig[1], up, words);
  const Sig<KW> p1 = lane == 0 ? p0 : t1;
  const bool f0 = lane < nvalid && (lane == 0 || !sig_eq(s.sig[0], p0, words));
  const bool f1 = 64 + lane < nvalid && !sig_eq(s.sig[1], p1, words);
  s.m[0] = __ballot(f0);
  s.m[1] = __ballot(f1);
  return s;
}

// The signature of token i of the side, for every lane's own i.
template <int KW>
__device__ __forceinline__ Sig<KW> side_sig(const TileSide<KW>& s, int i, int words) {
  const Sig<KW> lo = shfl_sig(s.sig[0], i & 63, words);
  const Sig<KW> hi = shfl_sig(s.sig[1], i & 63, words);
  return i < 64 ? lo : hi;
}

// The run starts as a mask pair, for the helpers below.
struct RunMask {
  uint64_t m[2];
};

template <int KW>
__device__ __forceinline__ RunMask run_mask(const TileSide<KW>& s) {
  return RunMask{{s.m[0], s.m[1]}};
}

__device__ __forceinline__ int run_count(const RunMask& r) {
  return __popcll(r.m[0]) + __popcll(r.m[1]);
}

// Position of the n-th (0-based) run start, or `none` when there are n or
// fewer starts (the end of the last run).
__device__ __forceinline__ int nth_start(const RunMask& r, int n, int none) {
  const int c0 = __popcll(r.m[0]);
  uint64_t m = r.m[0];
  int pos = 0;
  if (n >= c0) {
    m = r.m[1];
    pos = 64;
    n -= c0;
  }
  if (n >= __popcll(m)) return none;
#pragma unroll
  for (int width = 32; width >= 1; width >>= 1) {
    const int c = __popcll(m & ((1ull << width) - 1ull));
    if (n >= c) {
      n -= c;
      m >>= width;
      pos += width;
    }
  }
  return pos;
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

// (1) grid (ceil(nt (nt + 1) / 2 / 4), Bm); block 256: each wave decides one
// tile of the lower triangle (kt <= qt; linear index 4 x + wave, row-major)
// and writes its mirror above the diagonal as skip (every pair there has
// kv > q).  The wave finds the query and key run starts and evaluates the
// run pairs, 64 at a time, stopping once the tile is known to be partial.
constexpr int kClassifyWaves = kThreads / 64;

template <int KW>
__global__ __launch_bounds__(kThreads) void mask_classify_tiles(
    const int32_t* __restrict__ doc_all, const uint64_t* __restrict__ qbits_all,
    const uint64_t* __restrict__ kvbits_all, int T, int words, MaskOut out) {
  const int nt = out.nt;
  const int b = blockIdx.y;
  const int64_t L = (int64_t)blockIdx.x * kClassifyWaves + (threadIdx.x >> 6);
  if (L >= (int64_t)nt * (nt + 1) / 2) return;
  int qt, kt;
  tri_tile((int)L, qt, kt);
  const int lane = lane_id();
  if (lane == 0 && kt < qt) out.tile_class[((size_t)b * nt + kt) * nt + qt] = kSkip;
  const int32_t* doc = doc_all + (size_t)b * T;
  const uint64_t* qbits = qbits_all + (size_t)b * words * T;
  const uint64_t* kbits = kvbits_all + (size_t)b * words * T;
  const int q0 = qt * kTile, k0 = kt * kTile;
  const int qvalid = min(kTile, T - q0), kvalid = min(kTile, T - k0);
  const TileSide<KW> qs = wave_tile_side<KW>(doc, qbits, words, T, q0, qvalid);
  const TileSide<KW> ks = wave_tile_side<KW>(doc, kbits, words, T, k0, kvalid);
  const RunMask qr = run_mask(qs), kr = run_mask(ks);
  const int nqr = run_count(qr), nkr = run_count(kr);
  // Padding rows/columns are False pairs: such a tile can never be full.
  bool any_true = false;
  bool any_false = (qvalid < kTile) || (kvalid < kTile);
  const int npairs = nqr * nkr;
  for (int p0 = 0; p0 < npairs; p0 += 64) {
    const int p = p0 + lane;
    const int r = min(p, npairs - 1) / nkr, c = min(p, npairs - 1) - r * nkr;
    const int qa = nth_start(qr, r, 0), qb = nth_start(qr, r + 1, qvalid);
    const int ka = nth_start(kr, c, 0), kb = nth_start(kr, c + 1, kvalid);
    // every lane takes part in the shuffles (lanes past the last pair
    // repeat it)
    const bool v = sig_allowed(side_sig(qs, qa, words), side_sig(ks, ka, words), words);
    const bool exists_ge = (q0 + qb - 1) >= (k0 + ka);  // some pair with q >= kv
    const bool exists_lt = (q0 + qa) < (k0 + kb - 1);   // some pair with q < kv
    const bool t = v && exists_ge;
    const bool f = !v || exists_lt;
    any_true = any_true || (__ballot(t) != 0);
    any_false = any_false || (__ballot(f) != 0);
    if (any_true && any_false) break;
  }
  if (lane == 0)
    out.tile_class[((size_t)b * nt + qt) * nt + kt] =
        any_true ? (any_false ? kPartial : kFull) : kSkip;
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
// Threads 0..127 build the rows (query q0 + tid against the tile's keys),
// threads 128..255 the columns (key k0 + tid - 128 against the queries); each
// wave finds the run starts of the other side itself.  A row is built run by
// run: within a run of keys with one signature the non-causal predicate is
// constant, so one evaluation sets a whole bit range; the causal and padding
// limits are applied last.
template <int KW>
__global__ __launch_bounds__(kThreads) void mask_tile_bits(
    const int32_t* __restrict__ doc_all, const uint64_t* __restrict__ qbits_all,
    const uint64_t* __restrict__ kvbits_all, int T, int words, MaskOut out) {
  __shared__ int red[2 * kThreads / 64];
  const int nt = out.nt;
  const int b = blockIdx.y;
  int qt, kt;
  tri_tile(blockIdx.x, qt, kt);
  const int tid = threadIdx.x;
  if (kt == 0) rank_row_col(out, b, qt, red);
  if (out.tile_class[((size_t)b * nt + qt) * nt + kt] != kPartial) return;
  const int32_t* doc = doc_all + (size_t)b * T;
  const uint64_t* qbits = qbits_all + (size_t)b * words * T;
  const uint64_t* kbits = kvbits_all + (size_t)b * words * T;
  const int q0 = qt * kTile, k0 = kt * kTile;
  const bool rows = tid < kTile;
  // this thread's token and the other side of the tile
  const int mine = rows ? q0 + tid : k0 + tid - kTile;
  const int obase = rows ? k0 : q0;
  const uint64_t* mbits = rows ? qbits : kbits;
  const uint64_t* obits = rows ? kbits : qbits;
  const int ovalid = min(kTile, T - obase);
  const TileSide<KW> os = wave_tile_side<KW>(doc, obits, words, T, obase, ovalid);
  const Sig<KW> my = load_sig<KW>(doc, mbits, words, T, mine);
  uint32_t acc[4] = {0u, 0u, 0u, 0u};
  // run starts of the other side, in order (a wave-uniform loop over every
  // lane); a run's signature is that of its first token, read from the lane
  // holding it
  for (int h = 0; h < 2; ++h) {
    for (uint64_t m = os.m[h]; m; m &= m - 1) {
      const int a = 64 * h + __ffsll((long long)m) - 1;
      const uint64_t rest = m & (m - 1);
      const int z = rest ? 64 * h + __ffsll((long long)rest) - 1
                         : (h == 0 && os.m[1] ? __ffsll((long long)os.m[1]) - 1 + 64 : ovalid);
      const Sig<KW> other = readlane_sig(os.sig[h], a & 63, words);
      if (rows ? sig_allowed(my, other, words) : sig_allowed(other, my, words))
        set_bit_range(acc, a, z);
    }
  }
  uint32_t cm[4] = {0u, 0u, 0u, 0u};
  if (mine < T) {
    if (rows) {
      // causal: keys k0 + kk <= q; padding keys (>= T) are outside every run
      set_bit_range(cm, 0, min(max(mine - k0 + 1, 0), kTile));
    } else {
      // causal: queries q0 + qq >= key
      set_bit_range(cm, min(max(mine - q0, 0), kTile), kTile);
    }
  }
  // (a token past T keeps no bit: its causal mask is empty)
#pragma unroll
  for (int w = 0; w < 4; ++w) acc[w] &= cm[w];
  const int slot = tri_slot(b, nt, qt) + kt;
  uint32_t* dst = out.tile_bits + (size_t)slot * kTileBitsWords + tid * 4;
  *reinterpret_cast<uint4*>(dst) = make_uint4(acc[0], acc[1], acc[2], acc[3]);
}

hipError_t launch_mask_meta(const int32_t* doc, const uint64_t* qbits, const uint64_t* kvbits,
                            int T, int words, const MaskOut& out, hipStream_t stream) {
  const int nt = out.nt;
  if (nt == 0 || out.Bm == 0) return hipSuccess;
  const int64_t n_tri = (int64_t)nt * (nt + 1) / 2;
  const dim3 tiles((unsigned)n_tri, out.Bm);
  const dim3 tile_quads((unsigned)((n_tri + kClassifyWaves - 1) / kClassifyWaves), out.Bm);
  // signature registers sized for the smallest bound >= words
  auto classify = mask_classify_tiles<8>;
  auto bits = mask_tile_bits<8>;
  if (words == 0) {
    classify = mask_classify_tiles<0>;
    bits = mask_tile_bits<0>;
  } else if (words == 1) {
    classify = mask_classify_tiles<1>;
    bits = mask_tile_bits<1>;
  } else if (words == 2) {
    classify = mask_classify_tiles<2>;
    bits = mask_tile_bits<2>;
  } else if (words == 3) {
    classify = mask_classify_tiles<3>;
    bits = mask_tile_bits<3>;
  } else if (words == 4) {
    classify = mask_classify_tiles<4>;
    bits = mask_tile_bits<4>;
  }
  hipLaunchKernelGGL(classify, tile_quads, dim3(kThreads), 0, stream, doc, qbits, kvbits, T,
                     words, out);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(mask_lists, dim3(nt, out.Bm), dim3(kThreads), 0, stream, out);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(bits, tiles, dim3(kThreads), 0, stream, doc, qbits, kvbits, T, words, out);
  return hipGetLastError();
}

}  // namespace t2t
