// Shared device helpers for the gfx950 masked-attention kernels.
//
// Tile geometry: the BlockMask granularity is 128 x 128 (the reference's
// create_block_mask default, torch/nn/attention/flex_attention.py:395).  All
// dense contractions use the CDNA4 v_mfma_f32_32x32x16_bf16 instruction, whose
// lane layout is
//   A (32x16, M x K): lane l holds A[l % 32][8 * (l / 32) + j], j = 0..7
//   B (16x32, K x N): lane l holds B[8 * (l / 32) + j][l % 32]
//   C (32x32, f32):   lane l, acc i holds C[8 * (i / 4) + 4 * (l / 32) + i % 4][l % 32]
//
// LDS tiles are row-major [token][d] with rows padded by 16 bytes (pitch
// D + 8 elements).  A "row" operand (contraction over d) is one 16-byte
// ds_read_b128 per lane; a "column" operand (contraction over tokens) is two
// ds_read_b64_tr_b16 reads, whose result in each 16-lane group is
// out[i][j] = mem[addr[4 j + i / 4] + i % 4].
//
// The first contraction of every kernel puts tokens on the MFMA M side.  Its
// A-operand lane m reads token tok_perm(m) of the 32-token block instead of
// token m, so accumulator row m holds token tok_perm(m).  The permutation is
// chosen so that each column read touches rows four apart: with the 16-byte
// row padding, the 16 rows of a row read and the 4 x 64 bytes of a 32-lane
// column read then fall on distinct LDS banks, while every address stays a
// per-lane base plus an immediate offset.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

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

// LDS row pitch (elements) of a D-wide bf16 tile.
template <int D>
__device__ __forceinline__ constexpr int pitch() { return D + 8; }

// Token of A-operand row m (0..31) within a 32-token block:
// m = 16 h + 8 b + 4 g + r  ->  16 h + 4 r + 2 b + g.
__device__ __forceinline__ constexpr int tok_perm(int m) {
  return 16 * (m >> 4) + 4 * (m & 3) + 2 * ((m >> 3) & 1) + ((m >> 2) & 1);
}

// Token of accumulator entry i of lane group g (tok_perm of its C row).
__device__ __forceinline__ constexpr int acc_tok(int i, int g) {
  return 16 * (i >> 3) + 4 * (i & 3) + 2 * ((i >> 2) & 1) + g;
}

// Direct global -> LDS copies (buffer_load ... lds, no staging registers) of
// Rows token rows (64 or 32) into a padded LDS unit [Rows][D + 8].  One
// instruction moves 64 lanes x 16 bytes into 64 consecutive 16-byte LDS
// slots; a padded row is kSlots = D / 8 + 1 slots (the last one is the pad,
// loaded from an offset past any buffer so that it reads zero and touches no
// memory).  A 64-row unit is exactly kSlots instructions; a 32-row unit is
// kSlots / 2 + 1 of them, the second half of its last instruction landing in
// 32 sink slots after the rows (kElems counts them).  Instruction i, lane l
// covers slot 64 i + l.
template <int D, int NW = kWaves, int Rows = 64>
struct UnitDma {
  static constexpr int kRows = Rows;
  static constexpr int kSlots = D / 8 + 1;                 // 17 (D = 128) or 9 (D = 64)
  static constexpr int kInsts = (Rows * kSlots + 63) / 64; // 17 / 9 (64 rows), 9 / 5 (32 rows)
  static constexpr int kElems = kInsts * 64 * 8;           // LDS elements, sink included
  static constexpr int kPerWave = kInsts / NW;             // + 1 for one wave
  static_assert(Rows == 64 || Rows == 32, "64- or 32-row units");
  static_assert(kInsts % NW == 1, "one remainder instruction per unit");
};

// Per-lane byte offset of unit instruction i (relative to the unit's first
// row); pad and sink slots get an offset past any buffer (zero fill).
template <int D, int Rows = 64>
__device__ __forceinline__ int unit_dma_offset(int i, int64_t st, int lane) {
  using U = UnitDma<D, kWaves, Rows>;
  const int slot = 64 * i + lane;
  const int row = slot / U::kSlots, chunk = slot % U::kSlots;
  return (chunk < D / 8 && row < Rows) ? (int)((row * st + chunk * 8) * 2) : 0x7ffffff0;
}

// Wave `wave`'s share of a unit copy by NW waves: instructions wave + NW j,
// and the unit's last instruction in wave `extra_wave` only (a wave-uniform
// branch; the other waves issue nothing for it).  voff[j] =
// unit_dma_offset(wave + NW j), voff[kPerWave] = unit_dma_offset(kInsts - 1).
// `src` covers the whole [T, D] slice (slice_rsrc) and `row_off` is the byte
// offset of the unit's first row; it is added to the per-lane offset, whose
// range check then zero-fills rows at or past T (the host keeps every such
// offset below 2^31).
template <int D, int NW = kWaves, int Rows = 64>
__device__ __forceinline__ void unit_dma(__bf16* dst, __amdgpu_buffer_rsrc_t src, const int* voff,
                                         int row_off, int wave, int extra_wave) {
  using U = UnitDma<D, NW, Rows>;
#pragma unroll
  for (int j = 0; j < U::kPerWave; ++j)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        src, (__attribute__((address_space(3))) void*)(dst + (wave + NW * j) * 64 * 8), 16,
        voff[j] + row_off, 0, 0, 0);
  if (wave == extra_wave)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        src, (__attribute__((address_space(3))) void*)(dst + (U::kInsts - 1) * 64 * 8), 16,
        voff[U::kPerWave] + row_off, 0, 0, 0);
}

// Raw buffer resource as four scalar words: [base, base + bytes), stride 0,
// word 3 as slice_rsrc; loads past `bytes` return zeros.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ u32x4 rsrc_words(const void* base, int64_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  u32x4 r;
  r.x = __builtin_amdgcn_readfirstlane((uint32_t)a);
  r.y = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32) & 0xffffu);
  r.z = __builtin_amdgcn_readfirstlane((uint32_t)(bytes < 0x7fffffff ? bytes : 0x7fffffff));
  r.w = 0x00020000u;
  return r;
}

// rsrc_words over one [T, D] slice (row stride `st` elements), as slice_rsrc.
__device__ __forceinline__ u32x4 slice_words(const __bf16* base, int64_t st, int T, int D) {
  return rsrc_words(base, T > 0 ? ((int64_t)(T - 1) * st + D) * 2 : 0);
}

// One direct global -> LDS copy (lane l's 16 bytes at byte offset voff into
// LDS bytes [lds + 16 l, lds + 16 l + 16)) as inline assembly.  The
// compiler's wait-count pass does not track copies it cannot see, so no LDS
// read is made to wait for them; a kernel using this form relies on an
// explicit vmcnt wait before reading what the copies wrote (dma_barrier,
// vm_barrier).  M0 holds the LDS base; a scalar write of M0 needs one wait
// state before the copy reads it.  M0 is a reserved register the compiler
// does not let assembly clobber, and the compiler writes it only for its own
// LDS copies (__builtin_amdgcn_raw_ptr_buffer_load_lds): a kernel uses
// either these copies or the builtin ones, never both.
__device__ __forceinline__ void lds_copy16(const void* lds, int voff, u32x4 rsrc) {
  const uint32_t m0 = __builtin_amdgcn_readfirstlane(
      (uint32_t)reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const void*)lds));
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
               :
               : "s"(m0), "v"(voff), "s"(rsrc));
}

// lds_copy16 / lds_copy4 with the LDS byte address given as a wave-uniform
// integer (e.g. a __shared__ array's lds_u32 plus a constant offset), which
// keeps pointer conversions off the issuing path.
__device__ __forceinline__ void lds_copy16_m0(uint32_t m0, int voff, u32x4 rsrc) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
               :
               : "s"(m0), "v"(voff), "s"(rsrc));
}
__device__ __forceinline__ void lds_copy4_m0(uint32_t m0, int voff, u32x4 rsrc) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dword %1, %2, 0 offen lds"
               :
               : "s"(m0), "v"(voff), "s"(rsrc));
}

// LDS byte address of a __shared__ object (a constant for a named array).
__device__ __forceinline__ uint32_t lds_u32(const void* x) {
  return (uint32_t)reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const void*)x);
}

// lds_copy16 for 4-byte elements: lane l's dword at byte offset voff into
// LDS bytes [lds + 4 l, lds + 4 l + 4).
__device__ __forceinline__ void lds_copy4(const void* lds, int voff, u32x4 rsrc) {
  const uint32_t m0 = __builtin_amdgcn_readfirstlane(
      (uint32_t)reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const void*)lds));
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dword %1, %2, 0 offen lds"
               :
               : "s"(m0), "v"(voff), "s"(rsrc));
}

// Work-group barrier after this wave's LDS accesses have completed and at
// most N of its vector-memory loads (the newest ones: loads complete in
// issue order) are still outstanding -- for pipelines whose copies run more
// than one barrier ahead.  The compiler does not see the copies issued by
// lds_copy16 / lds_copy4, so the wait is written here.
template <int N>
__device__ __forceinline__ void vm_barrier() {
  static_assert(N >= 0 && N < 64, "vmcnt is a 6-bit count");
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" : : "n"(N) : "memory");
}

// Work-group barrier that first drains this wave's outstanding global->LDS
// copies and LDS accesses (the plain __syncthreads fence would also wait for
// them, but the explicit form keeps the compiler from hoisting LDS reads
// across it and documents what the pipeline relies on).
__device__ __forceinline__ void dma_barrier() {
  // The same wait as a builtin first: the compiler's wait-count tracking does
  // not read inline assembly, and without it would still count the loads
  // issued before the barrier as outstanding afterwards -- and place waits
  // for them (with counts that can also cover the copies issued after the
  // barrier) in front of the next compute.
  __builtin_amdgcn_s_waitcnt(0);
  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Bit of accumulator entry i in a bitmap word already shifted right by g.
__device__ __forceinline__ constexpr int acc_tok_bit(int i) {
  return 16 * (i >> 3) + 4 * (i & 3) + 2 * ((i >> 2) & 1);
}

// Row operand: 8 consecutive bf16 (col a multiple of 8) of row r.
template <int D>
__device__ __forceinline__ bf16x8 lds_row8(const __bf16* tile, int r, int col) {
  return *reinterpret_cast<const bf16x8*>(tile + r * pitch<D>() + col);
}

// Column operand (A or B slot of mfma32) over the 16 tokens [base, base + 16)
// of a block, in accumulator order: lane (g = l/32, c = l%32) receives
// tile[base + g + 4 j][col0 + c] for j = 0..3 and tile[base + 2 + g + 4 j][col0 + c]
// for j = 4..7, i.e. the tokens acc_tok(8 h + j, g) - 16 h of a half h whose
// first token is base.
template <int D>
__device__ __forceinline__ bf16x8 lds_col8(const __bf16* tile, int base, int col0, int lane) {
  const int grp = lane >> 4;                 // 16-lane group 0..3
  const int r = lane & 15;                   // lane within group
  const int g = grp >> 1;                    // k-group of the MFMA operand
  const int c = col0 + 16 * (grp & 1) + 4 * (r & 3);
  const int row = base + g + 4 * (r >> 2);
  const __bf16* p0 = tile + row * pitch<D>() + c;
  const __bf16* p1 = p0 + 2 * pitch<D>();
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

// (query head h, launch-order position y) of this work-group in a grid of
// (Hq, nt) blocks per batch row.  The hardware hands work-groups to the 8
// XCDs round-robin in dispatch order.  With grouped-query heads (G = Hq / Hkv
// > 1) the G heads that share a KV head and a query tile are placed 8
// dispatch slots apart, so one XCD runs them back to back and its L2 serves
// their identical K/V copies after the first; the groups themselves keep
// launch order (KV head fastest).  Without grouping, or when the Hkv * nt
// groups do not fill whole rounds of 8, heads stay the fastest dimension.
__device__ __forceinline__ void head_and_slot(int Hq, int Hkv, int nt, int& h, int& y) {
  const int G = Hq / Hkv;
  if (G == 1 || ((Hkv * nt) & 7) != 0) {
    h = blockIdx.x;
    y = blockIdx.y;
    return;
  }
  const int L = blockIdx.x + Hq * blockIdx.y;
  const int round = L / (8 * G), r = L - round * 8 * G;
  const int grp = 8 * round + (r & 7);  // (KV head, position) group
  h = (grp % Hkv) * G + (r >> 3);
  y = grp / Hkv;
}

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

// Sign-extended bit `bit` of x (0 or -1) as one v_bfe_i32; written as inline
// assembly because the compiler otherwise expands the and-mask of a one-bit
// field into a compare and a select.
template <int bit>
__device__ __forceinline__ int sbfe1_c(uint32_t x) {
  int r;
  asm("v_bfe_i32 %0, %1, %2, 1" : "=v"(r) : "v"(x), "i"(bit));
  return r;
}

// MFMA accumulator seed for a mixed 32x32 block: 0 where the pair is allowed,
// -inf where it is masked.  `nw` is the complement of the lane's bitmap word
// (bit t = token t of the block) shifted right by the lane group g, so a set
// bit marks a masked pair: its sign-extended bit field is all ones, which
// masks in the -inf pattern.
template <int I = 0>
__device__ __forceinline__ void mask_bias_fill(f32x16& c, uint32_t nw) {
  if constexpr (I < 16) {
    c[I] = __int_as_float(sbfe1_c<acc_tok_bit(I)>(nw) & (int)0xff800000);
    mask_bias_fill<I + 1>(c, nw);
  }
}

__device__ __forceinline__ f32x16 mask_bias(uint32_t nw) {
  f32x16 c;
  mask_bias_fill(c, nw);
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

}  // namespace t2t
