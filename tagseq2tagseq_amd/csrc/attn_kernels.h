// Argument blocks and launchers for the masked-attention kernels.
#pragma once

#include "t2t_common.h"

namespace t2t {

// A [B, H, T, D] tensor view with unit stride along D (element strides).
struct TensorView {
  void* data;
  int64_t sb, sh, st;
};

// BlockMask tables produced by the metadata pass ([Bm][nt] / [Bm][nt][nt]).
struct MaskTables {
  int Bm;
  int nt;
  const int32_t* kv_num;
  const int32_t* kv_idx;
  const int32_t* full_kv_num;
  const int32_t* full_kv_idx;
  const int32_t* q_num;
  const int32_t* q_idx;
  const int32_t* full_q_num;
  const int32_t* full_q_idx;
  const int32_t* row_order;
  const int32_t* col_order;
  const int32_t* kv_bits_off;
  const int32_t* q_bits_slot;
  const uint32_t* tile_bits;  // [slot][2][128][4]
};

// Writable view of the same tables for the metadata pass.
struct MaskOut {
  int Bm;
  int nt;
  int8_t* tile_class;
  int32_t* kv_num;
  int32_t* kv_idx;
  int32_t* full_kv_num;
  int32_t* full_kv_idx;
  int32_t* q_num;
  int32_t* q_idx;
  int32_t* full_q_num;
  int32_t* full_q_idx;
  int32_t* row_order;
  int32_t* col_order;
  int32_t* kv_bits_off;
  int32_t* q_bits_slot;
  uint32_t* tile_bits;
};

struct AttnDims {
  int B, Hq, Hkv, T, D;
  float scale;  // softmax scale applied to Q K^T
};

constexpr int kTileBitsWords = 2 * kTile * 4;  // uint32 words per tile bitmap slot

hipError_t launch_token_inputs(const int32_t* spans, const int32_t* n_spans, int max_spans,
                               const int32_t* grants, const int32_t* n_grants, int max_grants,
                               const uint64_t* links, int B, int T, int words, int32_t* doc,
                               uint64_t* q_bits, uint64_t* kv_bits, hipStream_t stream);

hipError_t launch_mask_meta(const int32_t* doc, const uint64_t* qbits, const uint64_t* kvbits,
                            int T, int words, const MaskOut& out, hipStream_t stream);

hipError_t launch_attn_fwd_bf16(const TensorView& q, const TensorView& k, const TensorView& v,
                                const TensorView& o, float* lse2, const AttnDims& dims,
                                const MaskTables& mask, hipStream_t stream);

// Float32 q / k / v / o (D in {64, 128}); same tables and LSE convention.
hipError_t launch_attn_fwd_f32(const TensorView& q, const TensorView& k, const TensorView& v,
                               const TensorView& o, float* lse2, const AttnDims& dims,
                               const MaskTables& mask, hipStream_t stream);

// Whole float32 backward: dQ (writing Delta), then dK/dV.
hipError_t launch_attn_bwd_f32(const TensorView& q, const TensorView& k, const TensorView& v,
                               const TensorView& o, const TensorView& dout, const float* lse2,
                               float* delta, const TensorView& dq, const TensorView& dk,
                               const TensorView& dv, const AttnDims& dims, const MaskTables& mask,
                               hipStream_t stream);

// kBwdDqDelta: dQ that also computes and writes Delta (run before dK/dV).
enum BwdPhase { kBwdDelta = 0, kBwdDkDv = 1, kBwdDq = 2, kBwdDqDelta = 3 };

// One backward phase.  Views a phase does not read may be empty (delta: o,
// dout; dkdv: q, k, v, dout, lse2, delta, dk, dv; dq: q, k, v, dout, lse2,
// delta, dq).
hipError_t launch_attn_bwd_phase(int phase, const TensorView& q, const TensorView& k,
                                 const TensorView& v, const TensorView& o,
                                 const TensorView& dout, const float* lse2, float* delta,
                                 const TensorView& dq, const TensorView& dk, const TensorView& dv,
                                 const AttnDims& dims, const MaskTables& mask,
                                 hipStream_t stream);

// Attention-module prologue: qkv [B][T][3][H][D] rows (strides sb, st) to
// rotated q, k and plain v views, and the transposed map for the gradients.
hipError_t launch_qkv_rope(const __bf16* qkv, int64_t sb, int64_t st, const TensorView& q,
                           const TensorView& k, const TensorView& v, const float* cos,
                           const float* sin, int B, int T, int H, int D, int pos0,
                           hipStream_t stream);
hipError_t launch_qkv_rope_bwd(const TensorView& dq, const TensorView& dk, const TensorView& dv,
                               const float* cos, const float* sin, int B, int T, int H, int D,
                               int pos0, __bf16* dqkv, int64_t sb, int64_t st,
                               hipStream_t stream);

// Decode step: Tq new query rows per batch row against a key/value cache of
// Tkv filled positions, mask evaluated per key from doc ids and words.
constexpr int kDecodeMaxRows = 8;  // (Hq / Hkv) * Tq per launch
int64_t decode_workspace_floats(int B, int Hq, int Tq, int Tkv, int D);
hipError_t launch_attn_decode(const TensorView& q, const TensorView& k, const TensorView& v,
                              const TensorView& o, float* lse2, const int32_t* key_doc,
                              const uint64_t* key_bits, int64_t key_stride, const int32_t* q_pos,
                              const int32_t* q_doc, const uint64_t* q_bits, int Bm, int W,
                              int B, int Hq, int Hkv, int Tq, int Tkv, int D, float scale,
                              float* workspace, hipStream_t stream);

// Weight gradient C = A^T B over K rows (split-K, fp32 partials summed in order).
int wgrad_splits(int M, int N, int K);
hipError_t launch_wgrad(const __bf16* a, int64_t lda, const __bf16* b, int64_t ldb, float* part,
                        void* out, bool out_f32, int M, int N, int K, hipStream_t stream);

// SwiGLU: h = silu(g) u from [g | u] rows, and [dg | du] from dh.
hipError_t launch_swiglu_fwd(const __bf16* gu, int64_t gs, __bf16* h, int64_t hs, int N, int H,
                             hipStream_t stream);
hipError_t launch_swiglu_bwd(const __bf16* gu, int64_t gs, const __bf16* dh, int64_t dhs,
                             __bf16* dgu, int64_t dgs, int N, int H, hipStream_t stream);

// Cross-entropy rows: loss and (softmax - onehot) * scale per bf16 row.
hipError_t launch_ce_rows(const uint16_t* logits, uint16_t* grad, int64_t rows, int V, int64_t ld,
                          const int64_t* target, int64_t ignore_index, const float* scale,
                          float* row_loss, hipStream_t stream);

// RMS normalisation of token rows (bf16 rows, bf16 or fp32 weight).
int rmsnorm_bwd_groups(int N, int C);
hipError_t launch_rmsnorm_fwd(const __bf16* x, int64_t xs, const void* w, bool w_f32, __bf16* y,
                              int64_t ys, float* rstd, int N, int C, float eps,
                              hipStream_t stream);
hipError_t launch_rmsnorm_bwd(const __bf16* dy, int64_t dys, const __bf16* x, int64_t xs,
                              const void* w, bool w_f32, const float* rstd, __bf16* dx,
                              int64_t dxs, void* dw, float* part, int N, int C,
                              hipStream_t stream);

// Linear maps of M <= 8 token rows (K % 8 == 0, K <= 4096) with an optional
// RMSNorm of the input and a fused epilogue; the modes match T2T_ROWS_*.
enum RowsMode { kRowsStore = 0, kRowsAdd = 1, kRowsSwiglu = 2, kRowsQkvRope = 3 };
constexpr int kRowsMaxRows = 8;
// kRowsAdd: y = res + W x, then, when skip_w is given, + skip_w * skip
// (skip NULL: the sum itself), each step rounded to bf16.
hipError_t launch_rows_linear(int mode, const __bf16* x, int64_t xs, int M, int K,
                              const __bf16* w, int N, const void* norm_w, bool norm_f32,
                              float eps, const __bf16* res, int64_t rs, const __bf16* skip,
                              int64_t ss, const void* skip_w, bool skip_w_f32, __bf16* y,
                              int64_t ys, hipStream_t stream);
// qkv projection of the rows, rotated q rows to q [H][M][D] and rotated k /
// plain v rows to the cache views at the rows' positions (pos[m], or
// pos0 + m when pos is NULL); positions outside [0, max_pos) are not written.
hipError_t launch_rows_qkv_rope(const __bf16* x, int64_t xs, int M, int K, const __bf16* w,
                                const void* norm_w, bool norm_f32, float eps, int H, int D,
                                const float* cos, const float* sin, const int64_t* pos, int pos0,
                                int max_pos, const TensorView& q, const TensorView& k,
                                const TensorView& v, hipStream_t stream);

// Engine-clock probe: out[0] / out[1] = shader cycles / wall-clock ticks of
// one wave while every SIMD runs two waves of MFMA chains (iters iterations).
hipError_t launch_clock_probe(uint64_t* out, int iters, hipStream_t stream);
hipError_t wall_clock_khz(int* khz);

// First position < n at which two copies of per-token inputs differ: lowers
// *out (preset to n by the caller) to it (bits arrays [words][stride]).
hipError_t launch_first_input_diff(const int64_t* ta, const int64_t* tb, const int32_t* da,
                                   const int32_t* db, const uint64_t* qa, const uint64_t* qb,
                                   const uint64_t* ka, const uint64_t* kb, int64_t sa, int64_t sb,
                                   int words, int n, int32_t* out, hipStream_t stream);

}  // namespace t2t
