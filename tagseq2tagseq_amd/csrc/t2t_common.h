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
// Operand tiles live row-major in LDS ([token][d], d contiguous, no padding)
// with the 16-byte chunks of row r XOR-permuted by swz(r), so that both read
// patterns below hit distinct banks.  A "row" operand (contraction over d) is
// one 16-byte ds_read_b128 per lane (16 lanes read 16 rows of one chunk); a
// "column" operand (contraction over tokens) is two ds_read_b64_tr_b16 reads,
// whose result in each 16-lane group is out[i][j] = mem[addr[4 j + i / 4] + i % 4]
// (4 rows x 32 bytes per 16 lanes).
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

// Chunk permutation of LDS row r for a D-wide bf16 tile: rows r .. r+15 map a
// given chunk to 16 distinct positions, and rows 4a .. 4a+3 map the chunk
// pairs (2m, 2m+1), (2m+2, 2m+3) to distinct positions.
template <int D>
__device__ __forceinline__ constexpr int swz(int r) {
  return (4 * (r & 3) + ((r >> 2) & 3)) & (D / 8 - 1);
}

// Element offset of (row r, column col) in a swizzled LDS tile.
template <int D>
__device__ __forceinline__ int lds_off(int r, int col) {
  return r * D + ((((col >> 3) ^ swz<D>(r))) << 3) + (col & 7);
}

// Row operand: 8 consecutive bf16 (col a multiple of 8) of row r.
template <int D>
__device__ __forceinline__ bf16x8 lds_row8(const __bf16* tile, int r, int col) {
  return *reinterpret_cast<const bf16x8*>(tile + lds_off<D>(r, col));
}

// Column operand for the A or B slot of mfma32: lane (g = l/32, c = l%32)
// receives tile[r0 + j][col0 + c] for j = 0..3 and tile[r1 + j][col0 + c] for
// j = 4..7, where r0 = base_row + 4 g, r1 = r0 + second_off.
template <int D>
__device__ __forceinline__ bf16x8 lds_col8(const __bf16* tile, int base_row, int second_off,
                                           int col0, int lane) {
  const int grp = lane >> 4;                 // 16-lane group 0..3
  const int r = lane & 15;                   // lane within group
  const int g = grp >> 1;                    // k-group of the MFMA operand
  const int c = col0 + 16 * (grp & 1) + 4 * (r & 3);
  const int row = base_row + 4 * g + (r >> 2);
  const __bf16* p0 = tile + lds_off<D>(row, c);
  const __bf16* p1 = tile + lds_off<D>(row + second_off, c);
  bf16x4_ld lo = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4_ptr)(p0));
  bf16x4_ld hi = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4_ptr)(p1));
  return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
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

// Value known to be equal in every lane (lets the compiler keep it in SGPRs).
__device__ __forceinline__ int uniform(int x) { return __builtin_amdgcn_readfirstlane(x); }

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Combine x of lanes l and l ^ 32 (the two halves of a 32x32 accumulator
// column) with v_permlane32_swap: the returned pair holds both values in
// every lane.
__device__ __forceinline__ float halves_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float halves_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// MFMA accumulator seed for a mixed 32x32 block: 0 where the pair is allowed,
// -inf where it is masked.  `sw` is the lane's bitmap word shifted right by 4 g.
__device__ __forceinline__ f32x16 mask_bias(uint32_t sw) {
  f32x16 c;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    // bit set -> keep = 0 -> +0.0; bit clear -> keep = ~0 -> 0xff800000 = -inf
    const uint32_t keep = ((sw >> (8 * (i >> 2) + (i & 3))) & 1u) - 1u;
    c[i] = __uint_as_float(keep & 0xff800000u);
  }
  return c;
}

constexpr float kLog2e = 1.4426950408889634f;

// Buffer resource over one [T, D] slice (row stride `st` elements): raw
// buffer loads past the last row return zeros, which pads the final tile
// without branches.  0x00020000 is the gfx9-family resource word 3.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t slice_rsrc(const __bf16* base, int64_t st,
                                                              int T, int D) {
  const int64_t bytes = T > 0 ? ((int64_t)(T - 1) * st + D) * 2 : 0;
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<__bf16*>(base), 0,
                                           (int)(bytes < 0x7fffffff ? bytes : 0x7fffffff),
                                           0x00020000);
}

// Copy token rows [t0, t0 + 128) of a slice into a swizzled LDS tile; rows
// past the slice end read as zeros.  Each thread moves 16-byte chunks; a wave
// covers four whole rows.
template <int D>
__device__ __forceinline__ void load_tile_lds(__bf16* dst, __amdgpu_buffer_rsrc_t src,
                                              int64_t st, int t0, int tid) {
  constexpr int kChunks = D / 8;
  constexpr int kIters = kTile * kChunks / kThreads;
  const int soff = (int)((int64_t)t0 * st * 2);
  uint4 buf[kIters];
#pragma unroll
  for (int it = 0; it < kIters; ++it) {
    const int c = tid + it * kThreads;
    const int r = c / kChunks, col = (c % kChunks) * 8;
    buf[it] = __builtin_bit_cast(
        uint4, __builtin_amdgcn_raw_buffer_load_b128(src, (int)((r * st + col) * 2), soff, 0));
  }
#pragma unroll
  for (int it = 0; it < kIters; ++it) {
    const int c = tid + it * kThreads;
    const int r = c / kChunks, col = (c % kChunks) * 8;
    *reinterpret_cast<uint4*>(dst + lds_off<D>(r, col)) = buf[it];
  }
}

// Bit of a tile-bitmap word for accumulator entry i, after the word has been
// shifted right by 4 * g (entries 8 c + r, c = i / 4, r = i % 4).
__device__ __forceinline__ constexpr int acc_bit(int i) { return 8 * (i >> 2) + (i & 3); }

}  // namespace t2t
