// Shared device helpers for the gfx950 masked-attention kernels.
//
// Tile geometry: the BlockMask granularity is 128 x 128 (the reference's
// create_block_mask default, torch/nn/attention/flex_attention.py:395).  Every
// attention work-group owns one 128-token tile and runs 4 waves of 64 lanes;
// each wave owns 32 rows of that tile.  All dense contractions use the CDNA4
// v_mfma_f32_32x32x16_bf16 instruction, whose lane layout is
//   A (32x16, M x K): lane l holds A[l % 32][8 * (l / 32) + j], j = 0..7
//   B (16x32, K x N): lane l holds B[8 * (l / 32) + j][l % 32]
//   C (32x32, f32):   lane l, acc i holds C[8 * (i / 4) + 4 * (l / 32) + i % 4][l % 32]
// Operand tiles live row-major in LDS ([token][d], d contiguous).  A "row"
// operand (contraction over d) is one 16-byte ds_read_b128 per lane; a
// "column" operand (contraction over tokens) is two ds_read_b64_tr_b16 reads,
// whose result in each 16-lane group is out[i][j] = mem[addr[4 j + i / 4] + i % 4].
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace t2t {

constexpr int kTile = 128;      // BlockMask tile edge (tokens)
constexpr int kWaves = 4;       // waves per work-group
constexpr int kThreads = 256;   // threads per work-group
constexpr int kMaxWords = 8;    // grant words per token supported (512 grants)

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x4_ld __attribute__((__vector_size__(4 * sizeof(__bf16))));
typedef __attribute__((address_space(3))) bf16x4_ld* lds_bf16x4_ptr;

// Tile-class codes written by the metadata pass.
enum : int8_t { kSkip = 0, kPartial = 1, kFull = 2 };

__device__ __forceinline__ f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// Row operand: 8 consecutive bf16 from an LDS row.
__device__ __forceinline__ bf16x8 lds_row8(const __bf16* p) {
  return *reinterpret_cast<const bf16x8*>(p);
}

// Column operand for the A or B slot of mfma32: lane (g = l/32, c = l%32)
// receives tile[r0 + j][col0 + c] for j = 0..3 and tile[r1 + j][col0 + c] for
// j = 4..7, where r0 = base_row + 4 g, r1 = r0 + second_off.  `tile` is a
// row-major LDS tile with `pitch` elements per row.
__device__ __forceinline__ bf16x8 lds_col8(const __bf16* tile, int pitch, int base_row,
                                           int second_off, int col0, int lane) {
  const int grp = lane >> 4;                 // 16-lane group 0..3
  const int r = lane & 15;                   // lane within group
  const int g = grp >> 1;                    // k-group of the MFMA operand
  const int c = col0 + 16 * (grp & 1) + 4 * (r & 3);
  const int row = base_row + 4 * g + (r >> 2);
  const __bf16* p0 = tile + row * pitch + c;
  const __bf16* p1 = p0 + second_off * pitch;
  bf16x4_ld lo = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4_ptr)(p0));
  bf16x4_ld hi = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4_ptr)(p1));
  bf16x8 out;
  out[0] = lo[0]; out[1] = lo[1]; out[2] = lo[2]; out[3] = lo[3];
  out[4] = hi[0]; out[5] = hi[1]; out[6] = hi[2]; out[7] = hi[3];
  return out;
}

// Pack accumulator entries [8h, 8h+8) of a 32x32 f32 tile into a bf16 operand.
__device__ __forceinline__ bf16x8 pack_half(const f32x16& acc, int h) {
  bf16x8 out;
#pragma unroll
  for (int j = 0; j < 8; ++j) out[j] = (__bf16)acc[8 * h + j];
  return out;
}

// Token row of accumulator entry i for lane group g (see layout above).
__device__ __forceinline__ constexpr int acc_row(int i, int g) {
  return 8 * (i >> 2) + 4 * g + (i & 3);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Value held by lane (l ^ 32).
__device__ __forceinline__ float swap_halves(float x) {
  return __shfl_xor(x, 32, 64);
}

// Per-token mask data for one mask row.
struct MaskRow {
  const int32_t* doc;      // [T]
  const uint64_t* qbits;   // [W][T]
  const uint64_t* kvbits;  // [W][T]
  int words;
  int T;
};

// mask_mod of model/graph_traversal/cross_doc_mask.py:348-357 for one pair,
// with per-token data already at hand (doc_causal: words == 0).
__device__ __forceinline__ bool pair_allowed(int q, int kv, int32_t dq, int32_t dk,
                                             const uint64_t* qb, const uint64_t* kb,
                                             int words) {
  if (kv > q) return false;
  if (dq == dk) return true;
  for (int w = 0; w < words; ++w)
    if (qb[w] & kb[w]) return true;
  return false;
}

}  // namespace t2t
