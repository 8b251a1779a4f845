// Mask-metadata pass: per-token document ids and grant words -> 128 x 128 tile
// classification (skip / partial / full) and the ordered index lists of a
// BlockMask.
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
#include "t2t_common.h"

namespace t2t {

namespace {

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

// grid (nt, Bm); block 256; dynamic LDS: nt bytes of row classes.
__global__ __launch_bounds__(kThreads) void mask_classify_rows(
    const int32_t* __restrict__ doc_all, const uint64_t* __restrict__ qbits_all,
    const uint64_t* __restrict__ kvbits_all, int T, int words, int nt,
    int8_t* __restrict__ tile_class, int32_t* __restrict__ kv_num,
    int32_t* __restrict__ kv_idx, int32_t* __restrict__ full_kv_num,
    int32_t* __restrict__ full_kv_idx) {
  extern __shared__ int8_t row_cls[];
  __shared__ int q_starts[kTile + 1];
  __shared__ int kv_starts[kWaves][kTile + 1];
  __shared__ int n_qruns;

  const int qt = blockIdx.x;
  const int b = blockIdx.y;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int32_t* doc = doc_all + (size_t)b * T;
  const uint64_t* qbits = qbits_all + (size_t)b * words * T;
  const uint64_t* kvbits = kvbits_all + (size_t)b * words * T;
  const int q0 = qt * kTile;
  const int qvalid = min(kTile, T - q0);

  if (wave == 0) {
    const int n = wave_runs(doc, qbits, words, T, q0, q_starts);
    if (lane == 0) n_qruns = n;
  }
  __syncthreads();
  const int nqr = n_qruns;

  for (int kt = wave; kt < nt; kt += kWaves) {
    int8_t cls = kSkip;
    if (kt <= qt) {
      const int k0 = kt * kTile;
      const int kvalid = min(kTile, T - k0);
      const int nkr = wave_runs(doc, kvbits, words, T, k0, kv_starts[wave]);
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
          const int ka = k0 + kv_starts[wave][s], kb = k0 + kv_starts[wave][s + 1];
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
      cls = any_true ? (any_false ? kPartial : kFull) : kSkip;
    }
    if (lane == 0) row_cls[kt] = cls;
  }
  __syncthreads();

  int8_t* out_row = tile_class + ((size_t)b * nt + qt) * nt;
  for (int i = threadIdx.x; i < nt; i += kThreads) out_row[i] = row_cls[i];
  const size_t row = (size_t)b * nt + qt;
  if (wave == 0) {
    wave_ordered(row_cls, 1, nt, kPartial, kv_num + row, kv_idx + row * nt);
  } else if (wave == 1) {
    wave_ordered(row_cls, 1, nt, kFull, full_kv_num + row, full_kv_idx + row * nt);
  }
}

// grid (nt, Bm); block 128 (wave 0: partial list, wave 1: full list).
__global__ __launch_bounds__(128) void mask_columns(
    const int8_t* __restrict__ tile_class, int nt, int32_t* __restrict__ q_num,
    int32_t* __restrict__ q_idx, int32_t* __restrict__ full_q_num,
    int32_t* __restrict__ full_q_idx) {
  const int kt = blockIdx.x;
  const int b = blockIdx.y;
  const int wave = threadIdx.x >> 6;
  const int8_t* col = tile_class + (size_t)b * nt * nt + kt;
  const size_t row = (size_t)b * nt + kt;
  if (wave == 0)
    wave_ordered(col, nt, nt, kPartial, q_num + row, q_idx + row * nt);
  else
    wave_ordered(col, nt, nt, kFull, full_q_num + row, full_q_idx + row * nt);
}

hipError_t launch_mask_meta(const int32_t* doc, const uint64_t* qbits, const uint64_t* kvbits,
                            int Bm, int T, int words, int8_t* tile_class, int32_t* kv_num,
                            int32_t* kv_idx, int32_t* full_kv_num, int32_t* full_kv_idx,
                            int32_t* q_num, int32_t* q_idx, int32_t* full_q_num,
                            int32_t* full_q_idx, hipStream_t stream) {
  const int nt = (T + kTile - 1) / kTile;
  if (nt == 0 || Bm == 0) return hipSuccess;
  hipLaunchKernelGGL(mask_classify_rows, dim3(nt, Bm), dim3(kThreads), nt, stream, doc, qbits,
                     kvbits, T, words, nt, tile_class, kv_num, kv_idx, full_kv_num, full_kv_idx);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(mask_columns, dim3(nt, Bm), dim3(128), 0, stream, tile_class, nt, q_num,
                     q_idx, full_q_num, full_q_idx);
  return hipGetLastError();
}

}  // namespace t2t
