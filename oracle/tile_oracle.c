/* Brute-force tile pair counts for the masked-attention BlockMask.
 * TEST INFRASTRUCTURE ONLY: used by tests/ and bench.py's cpu_baseline leg as
 * a checker; nothing in the product links it.
 *
 * Restates, pair by pair, the mask_mod of
 *   model/graph_traversal/cross_doc_mask.py:348-357
 *     causal & (doc[q] == doc[kv] | OR_c (q_bm[c][q] & kv_bm[c][kv]) != 0)
 * (doc_causal, block_mask_creator.py:121-129, is the case words == 0), and the
 * per-tile sum of torch/nn/attention/flex_attention.py:990-1013 over the
 * False-padded [T,T] mask with 128 x 128 tiles.
 *
 * doc:      int32[T]
 * q_bits:   uint64[words][T]   (word-major, as the reference's chunk list)
 * kv_bits:  uint64[words][T]
 * counts:   int64[nt][nt], nt = ceil(T / block), written in full.
 */
#include <stdint.h>
#include <string.h>

int oracle_tile_counts(const int32_t *doc, const uint64_t *q_bits,
                       const uint64_t *kv_bits, int64_t T, int64_t words,
                       int64_t block, int64_t *counts) {
  if (T < 0 || words < 0 || block <= 0) return -1;
  const int64_t nt = (T + block - 1) / block;
  memset(counts, 0, (size_t)(nt * nt) * sizeof(int64_t));
  for (int64_t q = 0; q < T; ++q) {
    const int64_t qt = q / block;
    const int32_t dq = doc[q];
    for (int64_t kv = 0; kv <= q; ++kv) {  /* causal: kv <= q */
      int ok = (doc[kv] == dq);
      for (int64_t w = 0; !ok && w < words; ++w)
        ok = (q_bits[w * T + q] & kv_bits[w * T + kv]) != 0;
      if (ok) counts[qt * nt + kv / block] += 1;
    }
  }
  return 0;
}
