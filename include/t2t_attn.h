/*
 * t2t_attn.h -- C ABI of libt2t_attn.so, the gfx950 masked flash-attention
 * path (doc_causal / cross_doc_link) of tagseq2tagseq.
 *
 * Plain pointers and sizes only.  Every pointer argument is a device pointer
 * unless stated otherwise; the caller owns all memory (the library allocates
 * and frees nothing).  All work is enqueued on `stream` (a hipStream_t passed
 * as void*; NULL = the null stream) with no host synchronisation.  Functions
 * return T2T_OK (0) or a negative status; t2t_last_error() then returns a
 * thread-local message.
 *
 * Mask model (the reference's mask_mod, model/graph_traversal/cross_doc_mask.py:348-357):
 *   allowed(q, kv) = q >= kv && (doc[q] == doc[kv] ||
 *                                OR_w (q_bits[w][q] & kv_bits[w][kv]) != 0)
 * doc_causal (model/graph_traversal/block_mask_creator.py:121-129) is words == 0.
 * Per-token inputs are laid out doc int32[Bm][T], q_bits / kv_bits
 * uint64[Bm][words][T] (word-major, the reference's chunk list), with Bm = 1
 * (one mask for every batch row, the reference's B=None) or Bm = B.
 */
#ifndef T2T_ATTN_H
#define T2T_ATTN_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define T2T_OK 0
#define T2T_EINVAL (-1)       /* bad pointer, size or stride */
#define T2T_EUNSUPPORTED (-2) /* shape / dtype outside what the kernels implement */
#define T2T_EHIP (-3)         /* a HIP launch or runtime call failed */

#define T2T_DTYPE_BF16 0
#define T2T_DTYPE_F32 1

#define T2T_TILE 128   /* BlockMask tile edge (torch/nn/attention/flex_attention.py:395) */
#define T2T_MAX_WORDS 8

/* Tile classes in tile_class[]: torch's partial / full int8 grids
 * (torch/nn/attention/flex_attention.py:1014-1018) folded into one byte. */
#define T2T_TILE_SKIP 0
#define T2T_TILE_PARTIAL 1
#define T2T_TILE_FULL 2

/* Words of one tile bitmap: [2][128][4] uint32 (row-major then column-major). */
#define T2T_TILE_BITS_WORDS 1024

/* [B, H, T, D] tensor with unit stride along D; strides in elements. */
typedef struct t2t_tensor {
  void *data;
  int64_t stride_b;
  int64_t stride_h;
  int64_t stride_t;
} t2t_tensor;

/*
 * Block-sparse mask tables, nt = ceil(T / 128).  The first eight match
 * torch's BlockMask (kv_num_blocks, kv_indices, full_kv_num_blocks,
 * full_kv_indices, q_num_blocks, q_indices, full_q_num_blocks, full_q_indices;
 * torch/nn/attention/flex_attention.py:586-657) with the head dimension
 * dropped: *_num int32[Bm][nt], *_idx int32[Bm][nt][nt].  The rest are this
 * library's additions:
 *   row_order / col_order int32[Bm][nt]: launch orders -- tile rows /
 *       columns by descending count of non-skip tiles taken in buckets of
 *       two (count / 2), within a bucket rows by descending and columns by
 *       ascending index (longest first for load balance, neighbours back to
 *       back for cache reuse of the tiles they share);
 *   kv_bits_off int32[Bm][nt]: bitmap slots of a tile row: partial tile
 *       (r, c) uses slot kv_bits_off[r] + c, and distinct partial tiles must
 *       get distinct slots.  t2t_mask_meta writes b nt (nt + 1) / 2 +
 *       r (r + 1) / 2, the tile's position in the lower triangle, which is
 *       distinct only because its masks are causal (every partial tile has
 *       c <= r); a caller filling the tables for a mask with partial tiles
 *       above the diagonal uses b nt^2 + r nt (one slot per tile);
 *   q_bits_slot int32[Bm][nt][nt]: bitmap slot of the i-th partial tile of a
 *       column (entries past q_num unspecified);
 *   tile_bits uint32[tile_bits_slots][2][128][4]: per partial tile, the
 *       allowed pairs as bits -- [0][q][w] bit j = allowed(q0 + q, k0 + 32 w + j),
 *       [1][k][w] bit j = allowed(q0 + 32 w + j, k0 + k);
 *   tile_bits_slots: capacity; Bm * nt * (nt + 1) / 2 always suffices for
 *       t2t_mask_meta's layout (Bm * nt * nt for the square one).
 */
typedef struct t2t_block_mask {
  int32_t mask_batch; /* Bm */
  int32_t num_tiles;  /* nt */
  int32_t *kv_num;
  int32_t *kv_idx;
  int32_t *full_kv_num;
  int32_t *full_kv_idx;
  int32_t *q_num;
  int32_t *q_idx;
  int32_t *full_q_num;
  int32_t *full_q_idx;
  int32_t *row_order;
  int32_t *col_order;
  int32_t *kv_bits_off;
  int32_t *q_bits_slot;
  uint32_t *tile_bits;
  int64_t tile_bits_slots;
} t2t_block_mask;

/* Library version string (host memory, static). */
const char *t2t_version(void);

/* Thread-local message for the last non-OK status on this thread. */
const char *t2t_last_error(void);

/*
 * Per-token inputs of t2t_mask_meta, built on the device from span and grant
 * lists.  Replaces the per-span loop of document_ids
 * (model/graph_traversal/block_mask_creator.py:107-117) and the per-grant
 * device slice-ORs of CrossDocLinkMaskCreator._build_grant_bitmasks
 * (model/graph_traversal/cross_doc_mask.py:240-294), and builds the doc x doc
 * link-bitmask form of the cross_doc_link mask.
 *   spans   int32[B][max_spans][3] = (start, end, doc_id), n_spans int32[B]:
 *           span i covers tokens [start, end) clipped to [0, T); later spans
 *           overwrite earlier ones; tokens no span covers get doc id -1.
 *   grants  int32[B][max_grants][5] = (bit, q_start, q_end, kv_start, kv_end),
 *           n_grants int32[B]; both NULL for no grants.  Bit `bit` of word
 *           bit / 64 is set in q_bits over [q_start, q_end) and in kv_bits over
 *           [kv_start, kv_end), clipped to [0, T); bits >= 64 * words are ignored.
 *   links   uint64[B][max_spans][words] or NULL: q_bits[t] |= links[span(t)],
 *           kv_bits[t] |= bit span(t) (span(t) = index of the span covering t;
 *           spans past 64 * words set no key bit).
 * Counts above max_spans / max_grants are clamped.  Outputs doc int32[B][T]
 * and, when words > 0, q_bits / kv_bits uint64[B][words][T] (the layout
 * t2t_mask_meta reads).
 */
int t2t_token_inputs(const int32_t *spans, const int32_t *n_spans, int32_t max_spans,
                     const int32_t *grants, const int32_t *n_grants, int32_t max_grants,
                     const uint64_t *links, int32_t B, int32_t T, int32_t words,
                     int32_t *doc, uint64_t *q_bits, uint64_t *kv_bits, void *stream);

/*
 * Metadata pass: tile classification, the BlockMask tables and the partial
 * tile bitmaps, written into the buffers `out` points at.
 * Replaces create_block_mask(mask_mod, B=None, H=None, T, T)
 * (torch/nn/attention/flex_attention.py:1144-1225) as called by
 * create_doc_causal_block_mask (model/graph_traversal/block_mask_creator.py:132-139)
 * and CrossDocLinkMaskCreator.__call__ (model/graph_traversal/cross_doc_mask.py:359-366),
 * without materialising the [T, T] mask.
 * tile_class: int8[Bm][nt][nt] out.  out->mask_batch / num_tiles must equal
 * mask_batch / ceil(T / 128); mask_batch * nt (nt + 1) / 2 bitmap slots
 * must fit int32 (T2T_EUNSUPPORTED otherwise).
 */
int t2t_mask_meta(const int32_t *doc, const uint64_t *q_bits, const uint64_t *kv_bits,
                  int32_t mask_batch, int32_t T, int32_t words, int8_t *tile_class,
                  const t2t_block_mask *out, void *stream);

/*
 * Masked attention forward.  Replaces the flex_attention forward
 * (torch/nn/attention/flex_attention.py:1396-1676; eager arithmetic
 * torch/_higher_order_ops/flex_attention.py:202-267) that FlexSelfAttention
 * calls from model/modules/layer.py:33.
 * q [B,Hq,T,D], k/v [B,Hkv,T,D], o [B,Hq,T,D] (dtype), lse2 float[B][Hq][T]
 * (contiguous) = log2-sum-exp2 of the masked row of (Q K^T * scale * log2 e);
 * natural-log LSE = lse2 * ln 2; fully masked rows give o = 0, lse2 = -inf.
 * Supported: dtype T2T_DTYPE_BF16 or T2T_DTYPE_F32 (q, k, v, o all of that
 * type; float32 is computed in float32 throughout), D in {64, 128},
 * Hq % Hkv == 0, and a positive finite normal scale (every attention entry
 * point rejects other scales with T2T_EINVAL: the kernels fold the scale
 * into -inf mask seeds and -LSE / scale row seeds; torch's flex_attention
 * would also take zero or negative scales).
 */
int t2t_attn_fwd(const t2t_tensor *q, const t2t_tensor *k, const t2t_tensor *v,
                 const t2t_tensor *o, float *lse2, int32_t B, int32_t Hq, int32_t Hkv,
                 int32_t T, int32_t D, int32_t dtype, float scale, const t2t_block_mask *mask,
                 void *stream);

/*
 * Masked attention backward.  Replaces flex_attention_backward as driven by
 * FlexAttentionAutogradOp.backward (torch/_higher_order_ops/flex_attention.py:689-767;
 * eager arithmetic sdpa_dense_backward :825-994).
 * delta: float[B][Hq][T] workspace, overwritten with rowsum(O * dO) by the dQ
 * launch (which runs first and computes it) and read by dK/dV.  dtype
 * T2T_DTYPE_BF16 or T2T_DTYPE_F32 (all tensors of that type; float32 is
 * computed in float32 throughout).  dq like q; dk/dv like k/v
 * (summed over each GQA group, written, not accumulated).  No atomics: the
 * result is bitwise deterministic.
 */
int t2t_attn_bwd(const t2t_tensor *q, const t2t_tensor *k, const t2t_tensor *v,
                 const t2t_tensor *o, const t2t_tensor *dout, const float *lse2,
                 float *delta, const t2t_tensor *dq, const t2t_tensor *dk,
                 const t2t_tensor *dv, int32_t B, int32_t Hq, int32_t Hkv, int32_t T,
                 int32_t D, int32_t dtype, float scale, const t2t_block_mask *mask,
                 void *stream);

/*
 * t2t_attn_bwd without the caller's Delta workspace, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid allocation).  No counterpart in the reference.
 * Delta lives in a file-scope device array of the library (one 16 MiB copy
 * per GPU, held until the process ends), so B * Hq * T must be at most
 * 4194304 (4 * 2^20) rows; larger shapes return T2T_EINVAL.  The call
 * allocates and frees nothing.  Every call on one GPU shares that GPU's
 * array: calls that overlap on one GPU (concurrent streams, or a second call
 * enqueued on another stream before the first finished) race.  The first call
 * on a device looks up the array's address with that device current.
 * Arguments and results otherwise as t2t_attn_bwd (bitwise identical outputs).
 */
int t2t_attn_bwd_noalloc(const t2t_tensor *q, const t2t_tensor *k, const t2t_tensor *v,
                         const t2t_tensor *o, const t2t_tensor *dout, const float *lse2,
                         const t2t_tensor *dq, const t2t_tensor *dk, const t2t_tensor *dv,
                         int32_t B, int32_t Hq, int32_t Hkv, int32_t T, int32_t D, int32_t dtype,
                         float scale, const t2t_block_mask *mask, void *stream);

/*
 * The backward's phases, callable separately (for example to run dK/dV and
 * dQ on two streams once Delta is ready; t2t_attn_bwd itself runs a dQ that
 * also writes Delta, then dK/dV).  bf16 only (float32 runs as one
 * t2t_attn_bwd call).  Same conventions:
 *   preprocess: delta[b][h][t] = sum_d o * dout  (sdpa_dense_backward :910-914)
 *   dkdv:       dk, dv  (KV-tile-major, walks q_num/q_idx + full_q_*)
 *   dq:         dq      (Q-tile-major, walks kv_num/kv_idx + full_kv_*)
 */
int t2t_attn_bwd_preprocess(const t2t_tensor *o, const t2t_tensor *dout, float *delta,
                            int32_t B, int32_t Hq, int32_t T, int32_t D, int32_t dtype,
                            void *stream);

int t2t_attn_bwd_dkdv(const t2t_tensor *q, const t2t_tensor *k, const t2t_tensor *v,
                      const t2t_tensor *dout, const float *lse2, const float *delta,
                      const t2t_tensor *dk, const t2t_tensor *dv, int32_t B, int32_t Hq,
                      int32_t Hkv, int32_t T, int32_t D, int32_t dtype, float scale,
                      const t2t_block_mask *mask, void *stream);

int t2t_attn_bwd_dq(const t2t_tensor *q, const t2t_tensor *k, const t2t_tensor *v,
                    const t2t_tensor *dout, const float *lse2, const float *delta,
                    const t2t_tensor *dq, int32_t B, int32_t Hq, int32_t Hkv, int32_t T,
                    int32_t D, int32_t dtype, float scale, const t2t_block_mask *mask,
                    void *stream);

/*
 * Attention-module prologue: QKV split + rotary embedding.  Replaces the
 * head split and rotary embedding inside the reference's attention module
 * (tunalab FlexSelfAttention as constructed and called at
 * model/modules/layer.py:16-21,33; that package's source is not in the
 * reference, so the rotary variant is the half-split form below).
 *   qkv   bf16 [B][T][3][H][D]: token rows of 3*H*D elements with element
 *         strides qkv_sb (batch) and qkv_st (token); within a row q, k, v
 *         head blocks are contiguous (the nn.Linear(C, 3C) output viewed as
 *         [B, T, 3, H, D]).
 *   cos, sin  float [table_rows][D/2] (contiguous); token t uses row pos0 + t.
 *   q, k, v   [B, H, T, D] outputs: for i < D/2, with c, s = cos, sin[pos0 + t][i],
 *             y[i] = x[i] c + x[i + D/2] s,  y[i + D/2] = x[i + D/2] c - x[i] s
 *             on q and k (fp32 arithmetic, one bf16 rounding); v is copied.
 * Supported: bf16, D % 16 == 0 and D <= 256; rows and views 16-byte aligned.
 */
int t2t_qkv_rope(const void *qkv, int64_t qkv_sb, int64_t qkv_st, int32_t B, int32_t T,
                 int32_t H, int32_t D, const float *cos, const float *sin, int32_t table_rows,
                 int32_t pos0, const t2t_tensor *q, const t2t_tensor *k, const t2t_tensor *v,
                 void *stream);

/*
 * Gradient of t2t_qkv_rope: dqkv (layout of qkv) from dq, dk, dv, applying the
 * transposed rotation dx[i] = dy[i] c - dy[i + D/2] s,
 * dx[i + D/2] = dy[i] s + dy[i + D/2] c to dq and dk and copying dv.  Every
 * element of dqkv is written (not accumulated).
 */
int t2t_qkv_rope_backward(const t2t_tensor *dq, const t2t_tensor *dk, const t2t_tensor *dv,
                          const float *cos, const float *sin, int32_t table_rows, int32_t pos0,
                          int32_t B, int32_t T, int32_t H, int32_t D, void *dqkv,
                          int64_t dqkv_sb, int64_t dqkv_st, void *stream);

/*
 * Decode step: attention of Tq new query rows per batch row against a
 * key/value cache, for generation with cached keys and values.  Replaces the
 * per-token full recompute of TS2TSModel.forward_inference
 * (model/model.py:214-237) driven by the generation loop
 * (model/generation_loop.py:90-92), whose last rows are the only ones used.
 *   q        [B, Hq, Tq, D] new query rows (rotated), o [B, Hq, Tq, D] out,
 *            lse2 float[B][Hq][Tq] out (log2 domain, as t2t_attn_fwd).
 *   k, v     [B, Hkv, cap, D] caches; positions 0 .. Tkv - 1 are read.
 *   key_doc  int32[Bm][key_stride], key_bits uint64[Bm][words][key_stride]:
 *            per cached position its doc id and kv words.
 *   q_pos    int32[Bm][Tq] absolute positions of the new rows, q_doc
 *            int32[Bm][Tq], q_bits uint64[Bm][words][Tq].
 *   Key j is allowed for new row t iff j <= q_pos[t] and (key_doc[j] ==
 *   q_doc[t] or q_bits[.][t] & key_bits[.][j] != 0 in some word) -- the
 *   doc_causal / cross_doc_link mask_mod.
 *   workspace: float[t2t_attn_decode_workspace(B, Hq, Tq, Tkv, D) / 4].
 * Supported: bf16, D in {64, 128}, (Hq / Hkv) * Tq <= 8, words <= 8.
 */
int64_t t2t_attn_decode_workspace(int32_t B, int32_t Hq, int32_t Tq, int32_t Tkv, int32_t D);

int t2t_attn_decode(const t2t_tensor *q, const t2t_tensor *k, const t2t_tensor *v,
                    const t2t_tensor *o, float *lse2, const int32_t *key_doc,
                    const uint64_t *key_bits, int64_t key_stride, const int32_t *q_pos,
                    const int32_t *q_doc, const uint64_t *q_bits, int32_t mask_batch,
                    int32_t words, int32_t B, int32_t Hq, int32_t Hkv, int32_t Tq, int32_t Tkv,
                    int32_t D, int32_t dtype, float scale, void *workspace,
                    int64_t workspace_bytes, void *stream);

/*
 * RMS normalisation of token rows: y = x / sqrt(mean(x^2) + eps) * weight in
 * fp32, rounded once to bf16.  Replaces the RMSNorm modules of the reference's
 * layers and head (model/modules/layer.py:14,19; training_module.py:122-123;
 * tunalab's RMSNorm, not part of the reference).
 *   x, y     bf16 rows [N][C] with row strides (elements); C % 8 == 0, C <= 4096.
 *   weight   [C], weight_dtype 0 = bf16, 1 = float32.
 *   rstd     float[N] out: 1 / rms per row (input of the backward).
 */
int t2t_rms_norm(const void *x, int64_t x_stride, const void *weight, int32_t weight_dtype,
                 void *y, int64_t y_stride, float *rstd, int32_t N, int32_t C, float eps,
                 void *stream);

/* Workspace (bytes) of t2t_rms_norm_backward for N rows of C. */
int64_t t2t_rms_norm_backward_workspace(int32_t N, int32_t C);

/*
 * Gradient of t2t_rms_norm: dx = r (g - xh mean(g xh)) with r = rstd,
 * xh = x r, g = dy weight; dweight = sum over rows of dy xh (weight dtype),
 * reduced in a fixed order (deterministic, no atomics).  dx and dweight are
 * written, not accumulated.
 */
int t2t_rms_norm_backward(const void *dy, int64_t dy_stride, const void *x, int64_t x_stride,
                          const void *weight, int32_t weight_dtype, const float *rstd, void *dx,
                          int64_t dx_stride, void *dweight, void *workspace,
                          int64_t workspace_bytes, int32_t N, int32_t C, void *stream);

/* Epilogues of t2t_rows_linear. */
#define T2T_ROWS_STORE 0  /* y = W xin */
#define T2T_ROWS_ADD 1    /* y = res + bf16(W xin) */
#define T2T_ROWS_SWIGLU 2 /* y = bf16(silu(g)) u, g = W[0:N] xin, u = W[N:2N] xin */

/*
 * Linear map of a few token rows for a generation step, with the work around
 * it fused in.  Replaces, at M <= 8 rows, the nn.Linear products of a layer
 * (model/modules/layer.py:32-35: tunalab FlexSelfAttention's out-projection,
 * GLU's gate_up and down, and the head's lm_head at model/model.py:227-237)
 * together with the RMSNorm before them and the residual add or SwiGLU after.
 *   x        bf16 rows [M][K] (row stride x_stride >= K, elements); 1 <= K <=
 *            4096, 0 <= M <= 8; rows are read as 16-byte vectors when K and
 *            x_stride are multiples of 8 and x, weight (and a float32 norm
 *            weight) are 16-byte aligned, element by element otherwise.
 *   weight   bf16 [N][K] row-major (nn.Linear layout); [2N][K] for SWIGLU
 *            (gate rows, then up rows: the gate_up output chunked in two).
 *   norm_weight  optional RMSNorm weight [K] (norm_dtype 0 bf16, 1 float32):
 *            xin = bf16(x / sqrt(mean(x^2) + eps) * norm_weight), as
 *            t2t_rms_norm writes it; NULL: xin = x.
 *   res, y   bf16 rows [M][N]; y may be res (in place), nothing else may alias.
 *   skip_weight  optional (ADD only) device scalar w (skip_weight_dtype 0 bf16,
 *            1 float32): y = bf16(t + bf16(w * s)) with t = the add's result and
 *            s = skip rows [M][N] (skip_stride), or s = t when skip is NULL --
 *            the backbone's weighted skip connection
 *            (model/modules/backbone.py:93-104) of the next layer folded in.
 * Products are summed in fp32 and rounded to bf16 before the epilogue.
 */
int t2t_rows_linear(const void *x, int64_t x_stride, int32_t M, int32_t K, const void *weight,
                    int32_t N, const void *norm_weight, int32_t norm_dtype, float eps,
                    int32_t epilogue, const void *res, int64_t res_stride, const void *skip,
                    int64_t skip_stride, const void *skip_weight, int32_t skip_weight_dtype,
                    void *y, int64_t y_stride, void *stream);

/*
 * qkv projection of a few rows with the rotary embedding and the key/value
 * cache write: replaces, in a generation step, the attention module's qkv
 * nn.Linear, its head split and rotation (t2t_qkv_rope) and the writes of the
 * new k and v rows into the cache, with the layer's RMSNorm before them
 * (model/modules/layer.py:33).
 *   x, norm_weight, eps   as for t2t_rows_linear (K = model dim).
 *   weight   bf16 [3 H D][K] (q, k, v head blocks, nn.Linear(C, 3C) layout).
 *   cos, sin float [table_rows][D/2]; row m uses position p = pos[m] (device
 *            int64[M]) or pos0 + m when pos is NULL.
 *   q        [H][M][D] view (t axis = row; the b stride is unused) of the
 *            rotated query rows.
 *   k_cache, v_cache  [H][cache_rows][D] views: row m's rotated k and plain v
 *            go to slot p.  A row whose p lies outside
 *            [0, min(table_rows, cache_rows)) writes nothing (q included).
 * Rotation as t2t_qkv_rope, on the bf16-rounded products.
 */
int t2t_rows_qkv_rope(const void *x, int64_t x_stride, int32_t M, int32_t K, const void *weight,
                      const void *norm_weight, int32_t norm_dtype, float eps, int32_t H,
                      int32_t D, const float *cos, const float *sin, int32_t table_rows,
                      const int64_t *pos, int32_t pos0, const t2t_tensor *q,
                      const t2t_tensor *k_cache, const t2t_tensor *v_cache, int32_t cache_rows,
                      void *stream);

/*
 * First position p < n at which two copies of a sequence's per-token inputs
 * differ -- token ids, doc ids, or any q / kv grant word -- or n when they
 * agree: the check of the generation key/value cache against the inputs of
 * a new TS2TSModel.forward_inference_last call (no counterpart in the
 * reference, which recomputes every position per token: generation_loop.py:90-92).
 *   tokens_*  int64[n], doc_* int32[n], q_bits_* / kv_bits_* uint64
 *             [words][bits_stride_*] (bits_stride >= n; NULL when words == 0).
 *   out       int32[1] (device): must hold n (or any value >= n) when the call
 *             runs (e.g. a fill on the same stream); the call lowers it to the
 *             first differing position with an atomic min, so it ends as the
 *             result.  0 <= words <= T2T_MAX_WORDS.
 */
int t2t_first_input_diff(const int64_t *tokens_a, const int64_t *tokens_b, const int32_t *doc_a,
                         const int32_t *doc_b, const uint64_t *q_bits_a, const uint64_t *q_bits_b,
                         const uint64_t *kv_bits_a, const uint64_t *kv_bits_b,
                         int64_t bits_stride_a, int64_t bits_stride_b, int32_t words, int32_t n,
                         int32_t *out, void *stream);

/*
 * Weight gradient of a linear map over many rows: C[m][n] = sum over k of
 * A[k][m] B[k][n], i.e. dW = dY^T X for y = x W^T with dY [K][M] and X [K][N].
 * Replaces the weight-gradient product of nn.Linear's backward for the
 * layers' projections (tunalab FlexSelfAttention's qkv / out projections and
 * GLU's gate_up / down, called from model/modules/layer.py:33-35), which
 * torch runs as one library product with only (M / 128) (N / 128) output
 * tiles.  K is split across work-groups into fp32 partials (the workspace),
 * summed in a fixed order by a second launch: deterministic, no atomics.
 *   a, b     bf16 row-major with row strides lda, ldb (elements, % 8 == 0,
 *            >= M / >= N), 16-byte aligned.
 *   out      [M][N] row-major, out_dtype T2T_DTYPE_BF16 or T2T_DTYPE_F32.
 *   M, N     multiples of 128; K a multiple of 64 (T2T_EUNSUPPORTED otherwise).
 *   workspace  t2t_wgrad_workspace(M, N, K) bytes, 16-byte aligned.
 */
int64_t t2t_wgrad_workspace(int32_t M, int32_t N, int32_t K);

int t2t_wgrad(const void *a, int64_t lda, const void *b, int64_t ldb, void *out,
              int32_t out_dtype, int32_t M, int32_t N, int32_t K, void *workspace,
              int64_t workspace_bytes, void *stream);

/*
 * SwiGLU of the MLP: h = silu(g) * u, computed in fp32 and rounded once, from
 * the gate / up product's rows [g | u] (g = the first H columns, u = the next
 * H).  Replaces the activation and product inside tunalab's GLU
 * (model/modules/layer.py:23-28; GLU(..., activation="silu")), i.e. torch's
 * chunk + silu + multiply.
 *   gu  bf16 [N][2H] with row stride gu_stride (elements); h bf16 [N][H] with
 *       row stride h_stride.  H % 8 == 0, strides % 8 == 0, pointers 16-byte
 *       aligned.
 */
int t2t_swiglu(const void *gu, int64_t gu_stride, void *h, int64_t h_stride, int32_t N,
               int32_t H, void *stream);

/*
 * Gradient of t2t_swiglu with s = sigmoid(g): dg = dh u s (1 + g (1 - s)),
 * du = dh g s, written as one [N][2H] buffer [dg | du] (the gate / up
 * product's gradient).  Same layout rules as t2t_swiglu.
 */
int t2t_swiglu_backward(const void *gu, int64_t gu_stride, const void *dh, int64_t dh_stride,
                        void *dgu, int64_t dgu_stride, int32_t N, int32_t H, void *stream);

/*
 * Cross-entropy rows of a linear head: loss and logit gradient in one pass.
 * Replaces, per chunk of rows, torch's F.cross_entropy(logits.float(),
 * targets, ignore_index, reduction="sum") and its backward inside the
 * reference's FusedLinearCELoss (tunalab; constructed at
 * model/modules/training_module.py:127-133, called at :209), which produces
 * the gradient during the forward so that dX and dW follow without
 * recomputing the logits.
 *   logits   bf16 [rows][ld] (device, 16-byte aligned); columns 0 .. V-1
 *            are the logits, columns V .. ld-1 are ignored.  ld % 8 == 0,
 *            1 <= V <= ld.
 *   grad     bf16 [rows][ld] out (may be `logits` itself): (softmax - onehot)
 *            * (*scale) in columns < V, 0 in the rest.
 *   target   int64[rows]; a row whose target equals ignore_index has loss 0
 *            and a zero gradient; any other target outside [0, V) gives a NaN
 *            loss (and a zero gradient).
 *   scale    float[1] (device): the gradient's factor (e.g. 1 / number of
 *            counted rows for a mean).
 *   row_loss float[rows] out: logsumexp(row) - row[target], computed in fp32.
 */
int t2t_ce_rows(const void *logits, void *grad, int64_t rows, int32_t V, int64_t ld,
                const int64_t *target, int64_t ignore_index, const float *scale,
                float *row_loss, void *stream);

/*
 * Engine-clock probe.  No counterpart in the reference: measurement support
 * for re-deriving the MFMA peak from the clock a box actually runs at.
 * Enqueues one kernel in which every SIMD runs two waves of back-to-back
 * v_mfma_f32_32x32x16_bf16 chains for `iters` iterations (1 .. 10^7) and one
 * wave records its shader-cycle (s_memtime) and wall-clock (s_memrealtime)
 * tick counts around its loop into out (uint64[2], device memory); wall_khz
 * (host pointer) receives the wall-clock counter's rate.  Engine clock in MHz
 * = out[0] / out[1] * wall_khz / 1000, read after the stream has finished.
 */
int t2t_clock_probe(uint64_t *out, int32_t iters, int32_t *wall_khz, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* T2T_ATTN_H */
