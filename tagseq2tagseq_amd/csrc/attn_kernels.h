// Argument blocks and launchers for the masked-attention kernels.
#pragma once

#include "t2t_common.h"

namespace t2t {

// A [B, H, T, D] tensor view with unit stride along D (element strides).
struct TensorView {
  void* data;
  int64_t sb, sh, st;
};

// Per-token mask inputs plus the BlockMask tables produced by the metadata pass.
// Tables are laid out [Bm][nt] (counts) and [Bm][nt][nt] (indices); Bm is 1
// (one mask shared by every batch row) or B.
struct MaskTables {
  const int32_t* doc;       // [Bm][T]
  const uint64_t* qbits;    // [Bm][words][T]
  const uint64_t* kvbits;   // [Bm][words][T]
  int words;
  int Bm;
  const int32_t* kv_num;
  const int32_t* kv_idx;
  const int32_t* full_kv_num;
  const int32_t* full_kv_idx;
  const int32_t* q_num;
  const int32_t* q_idx;
  const int32_t* full_q_num;
  const int32_t* full_q_idx;
};

struct AttnDims {
  int B, Hq, Hkv, T, D;
  float scale;  // softmax scale applied to Q K^T
};

hipError_t launch_mask_meta(const int32_t* doc, const uint64_t* qbits, const uint64_t* kvbits,
                            int Bm, int T, int words, int8_t* tile_class, int32_t* kv_num,
                            int32_t* kv_idx, int32_t* full_kv_num, int32_t* full_kv_idx,
                            int32_t* q_num, int32_t* q_idx, int32_t* full_q_num,
                            int32_t* full_q_idx, hipStream_t stream);

hipError_t launch_attn_fwd_bf16(const TensorView& q, const TensorView& k, const TensorView& v,
                                const TensorView& o, float* lse2, const AttnDims& dims,
                                const MaskTables& mask, hipStream_t stream);

enum BwdPhase { kBwdDelta = 0, kBwdDkDv = 1, kBwdDq = 2 };

// One backward phase.  Unused views may be empty for a phase that does not
// read them (delta: o, dout; dkdv: q, k, v, dout, lse2, delta, dk, dv; dq: q,
// k, v, dout, lse2, delta, dq).
hipError_t launch_attn_bwd_phase(int phase, const TensorView& q, const TensorView& k,
                                 const TensorView& v, const TensorView& o,
                                 const TensorView& dout, const float* lse2, float* delta,
                                 const TensorView& dq, const TensorView& dk, const TensorView& dv,
                                 const AttnDims& dims, const MaskTables& mask,
                                 hipStream_t stream);

}  // namespace t2t
