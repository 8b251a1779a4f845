// Per-token inputs of the metadata pass, built on the device from span and
// grant lists: the document-id map and the query / key grant words.
//
// Replaces the per-span and per-grant Python loops of the reference's mask
// creators, which issue one or two device slice operations per span / grant:
//   document_ids  (model/graph_traversal/block_mask_creator.py:107-117):
//     ids = -1; for span: ids[max(0, start):min(T, end)] = span.doc_id
//     (later spans overwrite earlier ones)
//   grant words   (model/graph_traversal/cross_doc_mask.py:240-294):
//     grant k: q_bm[k // 64][q_start:q_end] |= 1 << (k % 64),
//              kv_bm[k // 64][kv_start:kv_end] |= 1 << (k % 64)
// and adds the doc x doc link-bitmask form of the cross_doc_link mask
// (q_bits[t] = links[span(t)], kv_bits[t] = 1 << span(t)).
//
// One thread per (batch row, token): the row's spans and grants are staged
// through LDS in chunks of 256; each wave marks which of its 64 entries touch
// the work-group's 256 tokens (a ballot), and every thread then walks only the
// marked entries, in list order, so the result follows the reference's
// sequential semantics for any span / grant list (overlapping or unsorted
// included) while a token reads a handful of entries instead of the whole list.
#include "attn_kernels.h"

namespace t2t {

namespace {

constexpr int kTokThreads = 256;

struct TokenArgs {
  const int32_t* spans;      // [B][max_spans][3]: start, end, doc id
  const int32_t* n_spans;    // [B]
  int max_spans;
  const int32_t* grants;     // [B][max_grants][5]: bit, q_start, q_end, kv_start, kv_end
  const int32_t* n_grants;   // [B] (NULL: no grants)
  int max_grants;
  const uint64_t* links;     // [B][max_spans][words] or NULL
  int B, T, words;
  int32_t* doc;              // [B][T]
  uint64_t* q_bits;          // [B][words][T]
  uint64_t* kv_bits;         // [B][words][T]
};

constexpr int kTokWaves = kTokThreads / 64;

// Marks, per wave, the staged entries for which `hit` holds (lane i of wave w
// for entry 64 w + i); returns after every thread can read the masks.
__device__ __forceinline__ void mark_entries(bool hit, uint64_t* marks) {
  const uint64_t m = __ballot(hit);
  if ((threadIdx.x & 63) == 0) marks[threadIdx.x >> 6] = m;
  __syncthreads();
}

__global__ __launch_bounds__(kTokThreads) void token_inputs_kernel(TokenArgs a) {
  __shared__ int32_t stage[kTokThreads * 5];
  __shared__ uint64_t marks[kTokWaves];
  const int b = blockIdx.y;
  const int t0 = blockIdx.x * kTokThreads;
  const int t = t0 + threadIdx.x;
  const int t1 = min(a.T, t0 + kTokThreads);  // this work-group's tokens: [t0, t1)
  // Counts come from device memory: clamp them to the declared capacities.
  const int ns = max(0, min(a.n_spans[b], a.max_spans));

  // Last span covering t (spans are clipped to [0, T) by the comparison).
  int span = -1, doc_id = -1;
  for (int base = 0; base < ns; base += kTokThreads) {
    const int cnt = min(kTokThreads, ns - base);
    __syncthreads();
    bool hit = false;
    if ((int)threadIdx.x < cnt) {
      const int32_t* s = a.spans + ((size_t)b * a.max_spans + base + threadIdx.x) * 3;
      const int s0 = s[0], s1 = s[1];
      stage[3 * threadIdx.x + 0] = s0;
      stage[3 * threadIdx.x + 1] = s1;
      stage[3 * threadIdx.x + 2] = s[2];
      hit = s0 < t1 && s1 > t0;
    }
    mark_entries(hit, marks);
    for (int w = 0; w < kTokWaves; ++w) {
      for (uint64_t m = marks[w]; m; m &= m - 1) {
        const int i = 64 * w + __ffsll((long long)m) - 1;
        if (stage[3 * i] <= t && t < stage[3 * i + 1]) {
          span = base + i;
          doc_id = stage[3 * i + 2];
        }
      }
    }
  }

  uint64_t qw[kMaxWords], kw[kMaxWords];
#pragma unroll
  for (int w = 0; w < kMaxWords; ++w) { qw[w] = 0; kw[w] = 0; }
  if (a.links && span >= 0) {
    const uint64_t* row = a.links + ((size_t)b * a.max_spans + span) * a.words;
#pragma unroll
    for (int w = 0; w < kMaxWords; ++w)
      if (w < a.words) qw[w] = row[w];
#pragma unroll
    for (int w = 0; w < kMaxWords; ++w)
      if (w == (span >> 6)) kw[w] = 1ull << (span & 63);
  }

  const int ng = a.n_grants ? max(0, min(a.n_grants[b], a.max_grants)) : 0;
  for (int base = 0; base < ng; base += kTokThreads) {
    const int cnt = min(kTokThreads, ng - base);
    __syncthreads();
    bool hit = false;
    if ((int)threadIdx.x < cnt) {
      const int32_t* g = a.grants + ((size_t)b * a.max_grants + base + threadIdx.x) * 5;
      int e5[5];
#pragma unroll
      for (int e = 0; e < 5; ++e) stage[5 * threadIdx.x + e] = e5[e] = g[e];
      hit = (e5[1] < t1 && e5[2] > t0) || (e5[3] < t1 && e5[4] > t0);
    }
    mark_entries(hit, marks);
    for (int w = 0; w < kTokWaves; ++w) {
      for (uint64_t mk = marks[w]; mk; mk &= mk - 1) {
        const int i = 64 * w + __ffsll((long long)mk) - 1;
        const int bit = stage[5 * i];
        const uint64_t m = 1ull << (bit & 63);
        const bool inq = stage[5 * i + 1] <= t && t < stage[5 * i + 2];
        const bool ink = stage[5 * i + 3] <= t && t < stage[5 * i + 4];
#pragma unroll
        for (int w2 = 0; w2 < kMaxWords; ++w2) {
          if (w2 == (bit >> 6)) {
            if (inq) qw[w2] |= m;
            if (ink) kw[w2] |= m;
          }
        }
      }
    }
  }

  if (t >= a.T) return;
  a.doc[(size_t)b * a.T + t] = doc_id;
#pragma unroll
  for (int w = 0; w < kMaxWords; ++w) {
    if (w < a.words) {
      a.q_bits[((size_t)b * a.words + w) * a.T + t] = qw[w];
      a.kv_bits[((size_t)b * a.words + w) * a.T + t] = kw[w];
    }
  }
}

}  // namespace

hipError_t launch_token_inputs(const int32_t* spans, const int32_t* n_spans, int max_spans,
                               const int32_t* grants, const int32_t* n_grants, int max_grants,
                               const uint64_t* links, int B, int T, int words, int32_t* doc,
                               uint64_t* q_bits, uint64_t* kv_bits, hipStream_t stream) {
  if (B == 0 || T == 0) return hipSuccess;
  TokenArgs a{spans, n_spans, max_spans, grants, n_grants, max_grants, links,
              B,     T,       words,     doc,    q_bits,   kv_bits};
  const dim3 grid((unsigned)((T + kTokThreads - 1) / kTokThreads), (unsigned)B);
  hipLaunchKernelGGL(token_inputs_kernel, grid, dim3(kTokThreads), 0, stream, a);
  return hipGetLastError();
}

}  // namespace t2t
