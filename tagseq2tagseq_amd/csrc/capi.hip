// extern "C" boundary of libt2t_attn.so: argument validation, error
// reporting and dispatch to the gfx950 kernels.  No allocation happens here.
#include <algorithm>
#include <cfloat>
#include <cstdarg>
#include <cstdio>
#include <mutex>

#include "../../include/t2t_attn.h"
#include "attn_kernels.h"

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int hip_status(hipError_t e, const char* what) {
  if (e == hipSuccess) return T2T_OK;
  return fail(T2T_EHIP, "%s: %s", what, hipGetErrorString(e));
}

// A [B, H, T, D] view the kernels can address: 16-byte aligned rows, and each
// [T, D] slice, extended by one 128-row tile, spans less than 2 GiB, since the
// kernels address a slice through a buffer resource with 31-bit byte offsets
// (a tile starting at or past T is addressed, and reads as zeros).
// A [B, H, T, D] view of elements of `esize` bytes: 16-byte aligned base and
// strides, and one (b, h) slice (plus a tile of padding rows) under 2 GiB so
// that 32-bit buffer offsets reach it.
bool view_ok(const t2t_tensor* t, int T, int D, int esize = 2) {
  const int64_t align = 16 / esize;
  if (!(t && t->data && t->stride_b >= 0 && t->stride_h >= 0 && t->stride_t > 0 &&
        (reinterpret_cast<uintptr_t>(t->data) % 16) == 0 && (t->stride_t % align) == 0 &&
        (t->stride_h % align) == 0 && (t->stride_b % align) == 0))
    return false;
  const int64_t span_bytes = (((int64_t)T + t2t::kTile) * t->stride_t + (int64_t)D) * esize;
  return span_bytes <= 0x7fffffffLL - 16;
}

t2t::TensorView as_view(const t2t_tensor* t) {
  return t2t::TensorView{t->data, t->stride_b, t->stride_h, t->stride_t};
}

int check_mask(const t2t_block_mask* m, int B, int T, bool need_rows, bool need_cols) {
  if (!m) return fail(T2T_EINVAL, "mask is NULL");
  if (!(m->mask_batch == 1 || m->mask_batch == B))
    return fail(T2T_EINVAL, "mask.mask_batch=%d must be 1 or B=%d", m->mask_batch, B);
  const int nt = (T + t2t::kTile - 1) / t2t::kTile;
  if (m->num_tiles != nt)
    return fail(T2T_EINVAL, "mask.num_tiles=%d but T=%d needs %d", m->num_tiles, T, nt);
  if (need_rows && (!m->kv_num || !m->kv_idx || !m->full_kv_num || !m->full_kv_idx ||
                    !m->row_order || !m->kv_bits_off))
    return fail(T2T_EINVAL, "mask row tables (kv_*, row_order, kv_bits_off) missing");
  if (need_cols && (!m->q_num || !m->q_idx || !m->full_q_num || !m->full_q_idx ||
                    !m->col_order || !m->q_bits_slot))
    return fail(T2T_EINVAL, "mask column tables (q_*, col_order, q_bits_slot) missing");
  if (!m->tile_bits) return fail(T2T_EINVAL, "mask.tile_bits is NULL");
  return T2T_OK;
}

t2t::MaskTables as_tables(const t2t_block_mask* m) {
  t2t::MaskTables t;
  t.Bm = m->mask_batch;
  t.nt = m->num_tiles;
  t.kv_num = m->kv_num; t.kv_idx = m->kv_idx;
  t.full_kv_num = m->full_kv_num; t.full_kv_idx = m->full_kv_idx;
  t.q_num = m->q_num; t.q_idx = m->q_idx;
  t.full_q_num = m->full_q_num; t.full_q_idx = m->full_q_idx;
  t.row_order = m->row_order; t.col_order = m->col_order;
  t.kv_bits_off = m->kv_bits_off; t.q_bits_slot = m->q_bits_slot;
  t.tile_bits = m->tile_bits;
  return t;
}

// The kernels fold the softmax scale into masked-score seeds (-inf) and the
// backward into row seeds (-LSE / scale): a positive normal scale is required
// (torch's flex_attention would also accept zero or negative scales).
int check_scale(float scale) {
  if (!(scale >= FLT_MIN && scale <= FLT_MAX))
    return fail(T2T_EINVAL, "scale=%g must be a positive finite normal number", (double)scale);
  return T2T_OK;
}

int check_dims(int B, int Hq, int Hkv, int T, int D, int dtype, bool f32_ok = false) {
  if (B < 0 || Hq < 0 || Hkv <= 0 || T < 0) return fail(T2T_EINVAL, "negative size");
  if (Hq % Hkv != 0)
    return fail(T2T_EINVAL, "Hq=%d must be a multiple of Hkv=%d (GQA)", Hq, Hkv);
  if (!(dtype == T2T_DTYPE_BF16 || (f32_ok && dtype == T2T_DTYPE_F32)))
    return fail(T2T_EUNSUPPORTED, "dtype %d not supported here", dtype);
  if (D != 64 && D != 128) return fail(T2T_EUNSUPPORTED, "head dim D=%d not in {64, 128}", D);
  return T2T_OK;
}

}  // namespace

extern "C" {

const char* t2t_version(void) { return "t2t_attn 0.1 gfx950"; }

const char* t2t_last_error(void) { return g_err; }

int t2t_token_inputs(const int32_t* spans, const int32_t* n_spans, int32_t max_spans,
                     const int32_t* grants, const int32_t* n_grants, int32_t max_grants,
                     const uint64_t* links, int32_t B, int32_t T, int32_t words, int32_t* doc,
                     uint64_t* q_bits, uint64_t* kv_bits, void* stream) {
  if (B < 0 || T < 0 || max_spans < 0 || max_grants < 0)
    return fail(T2T_EINVAL, "negative B, T, max_spans or max_grants");
  if (words < 0 || words > T2T_MAX_WORDS)
    return fail(T2T_EUNSUPPORTED, "words=%d outside [0, %d]", words, T2T_MAX_WORDS);
  if (B == 0 || T == 0) return T2T_OK;
  if (!doc || !n_spans || (max_spans > 0 && !spans))
    return fail(T2T_EINVAL, "doc, n_spans or spans is NULL");
  if ((grants == nullptr) != (n_grants == nullptr))
    return fail(T2T_EINVAL, "grants and n_grants must both be given or both be NULL");
  if (grants && max_grants == 0) return fail(T2T_EINVAL, "grants given with max_grants == 0");
  if ((grants || links) && words == 0)
    return fail(T2T_EINVAL, "grants / links need words > 0");
  if (words > 0 && (!q_bits || !kv_bits)) return fail(T2T_EINVAL, "q_bits / kv_bits is NULL");
  return hip_status(t2t::launch_token_inputs(spans, n_spans, max_spans, grants, n_grants,
                                             max_grants, links, B, T, words, doc, q_bits,
                                             kv_bits, static_cast<hipStream_t>(stream)),
                    "t2t_token_inputs launch");
}

int t2t_mask_meta(const int32_t* doc, const uint64_t* q_bits, const uint64_t* kv_bits,
                  int32_t mask_batch, int32_t T, int32_t words, int8_t* tile_class,
                  const t2t_block_mask* out, void* stream) {
  if (T < 0 || mask_batch < 0) return fail(T2T_EINVAL, "negative T or mask_batch");
  if (words < 0 || words > T2T_MAX_WORDS)
    return fail(T2T_EUNSUPPORTED, "words=%d outside [0, %d]", words, T2T_MAX_WORDS);
  if (T == 0 || mask_batch == 0) return T2T_OK;
  if (!out) return fail(T2T_EINVAL, "out is NULL");
  const int nt = (T + t2t::kTile - 1) / t2t::kTile;
  if (out->mask_batch != mask_batch || out->num_tiles != nt)
    return fail(T2T_EINVAL, "out describes Bm=%d nt=%d, expected Bm=%d nt=%d", out->mask_batch,
                out->num_tiles, mask_batch, nt);
  const int64_t need = (int64_t)mask_batch * nt * (nt + 1) / 2;
  // bitmap slots are indexed with int32 (kv_bits_off, q_bits_slot)
  if (need > 0x7fffffffLL)
    return fail(T2T_EUNSUPPORTED, "Bm=%d x %lld tiles exceed the int32 bitmap slot range",
                mask_batch, (long long)nt * (nt + 1) / 2);
  if (out->tile_bits_slots < need)
    return fail(T2T_EINVAL, "tile_bits holds %lld slots, %lld needed",
                (long long)out->tile_bits_slots, (long long)need);
  if (!doc || (words > 0 && (!q_bits || !kv_bits)) || !tile_class || !out->kv_num ||
      !out->kv_idx || !out->full_kv_num || !out->full_kv_idx || !out->q_num || !out->q_idx ||
      !out->full_q_num || !out->full_q_idx || !out->row_order || !out->col_order ||
      !out->kv_bits_off || !out->q_bits_slot || !out->tile_bits)
    return fail(T2T_EINVAL, "NULL pointer argument");
  t2t::MaskOut o;
  o.Bm = mask_batch; o.nt = nt; o.tile_class = tile_class;
  o.kv_num = out->kv_num; o.kv_idx = out->kv_idx;
  o.full_kv_num = out->full_kv_num; o.full_kv_idx = out->full_kv_idx;
  o.q_num = out->q_num; o.q_idx = out->q_idx;
  o.full_q_num = out->full_q_num; o.full_q_idx = out->full_q_idx;
  o.row_order = out->row_order; o.col_order = out->col_order;
  o.kv_bits_off = out->kv_bits_off; o.q_bits_slot = out->q_bits_slot;
  o.tile_bits = out->tile_bits;
  return hip_status(t2t::launch_mask_meta(doc, q_bits, kv_bits, T, words, o,
                                          static_cast<hipStream_t>(stream)),
                    "t2t_mask_meta launch");
}

int t2t_attn_fwd(const t2t_tensor* q, const t2t_tensor* k, const t2t_tensor* v,
                 const t2t_tensor* o, float* lse2, int32_t B, int32_t Hq, int32_t Hkv,
                 int32_t T, int32_t D, int32_t dtype, float scale, const t2t_block_mask* mask,
                 void* stream) {
  int rc = check_dims(B, Hq, Hkv, T, D, dtype, true);
  if (rc) return rc;
  rc = check_scale(scale);
  if (rc) return rc;
  if (B == 0 || Hq == 0 || T == 0) return T2T_OK;
  const int es = dtype == T2T_DTYPE_F32 ? 4 : 2;
  if (!view_ok(q, T, D, es) || !view_ok(k, T, D, es) || !view_ok(v, T, D, es) ||
      !view_ok(o, T, D, es))
    return fail(T2T_EINVAL, "q/k/v/o view invalid (NULL, misaligned, bad stride or slice >= 2 GiB)");
  if (!lse2) return fail(T2T_EINVAL, "lse2 is NULL");
  rc = check_mask(mask, B, T, true, false);
  if (rc) return rc;
  t2t::AttnDims dims{B, Hq, Hkv, T, D, scale};
  const hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == T2T_DTYPE_F32)
    return hip_status(t2t::launch_attn_fwd_f32(as_view(q), as_view(k), as_view(v), as_view(o),
                                               lse2, dims, as_tables(mask), st),
                      "t2t_attn_fwd launch");
  return hip_status(t2t::launch_attn_fwd_bf16(as_view(q), as_view(k), as_view(v), as_view(o),
                                              lse2, dims, as_tables(mask), st),
                    "t2t_attn_fwd launch");
}

int t2t_attn_bwd_preprocess(const t2t_tensor* o, const t2t_tensor* dout, float* delta,
                            int32_t B, int32_t Hq, int32_t T, int32_t D, int32_t dtype,
                            void* stream) {
  int rc = check_dims(B, Hq, Hq > 0 ? Hq : 1, T, D, dtype);
  if (rc) return rc;
  if (B == 0 || Hq == 0 || T == 0) return T2T_OK;
  if (!view_ok(o, T, D) || !view_ok(dout, T, D)) return fail(T2T_EINVAL, "o/dout view invalid");
  if (!delta) return fail(T2T_EINVAL, "delta is NULL");
  const t2t::TensorView none{nullptr, 0, 0, 0};
  t2t::AttnDims dims{B, Hq, Hq, T, D, 1.f};
  t2t::MaskTables m{};
  return hip_status(t2t::launch_attn_bwd_phase(t2t::kBwdDelta, none, none, none, as_view(o),
                                               as_view(dout), nullptr, delta, none, none, none,
                                               dims, m, static_cast<hipStream_t>(stream)),
                    "t2t_attn_bwd_preprocess launch");
}

int t2t_attn_bwd_dkdv(const t2t_tensor* q, const t2t_tensor* k, const t2t_tensor* v,
                      const t2t_tensor* dout, const float* lse2, const float* delta,
                      const t2t_tensor* dk, const t2t_tensor* dv, int32_t B, int32_t Hq,
                      int32_t Hkv, int32_t T, int32_t D, int32_t dtype, float scale,
                      const t2t_block_mask* mask, void* stream) {
  int rc = check_dims(B, Hq, Hkv, T, D, dtype);
  if (rc) return rc;
  rc = check_scale(scale);
  if (rc) return rc;
  if (B == 0 || Hq == 0 || T == 0) return T2T_OK;
  if (!view_ok(q, T, D) || !view_ok(k, T, D) || !view_ok(v, T, D) || !view_ok(dout, T, D) || !view_ok(dk, T, D) ||
      !view_ok(dv, T, D))
    return fail(T2T_EINVAL, "tensor view invalid (NULL, misaligned, bad stride or slice >= 2 GiB)");
  if (!lse2 || !delta) return fail(T2T_EINVAL, "lse2/delta is NULL");
  rc = check_mask(mask, B, T, false, true);
  if (rc) return rc;
  const t2t::TensorView none{nullptr, 0, 0, 0};
  t2t::AttnDims dims{B, Hq, Hkv, T, D, scale};
  return hip_status(t2t::launch_attn_bwd_phase(t2t::kBwdDkDv, as_view(q), as_view(k), as_view(v),
                                               none, as_view(dout), lse2,
                                               const_cast<float*>(delta), none, as_view(dk),
                                               as_view(dv), dims, as_tables(mask),
                                               static_cast<hipStream_t>(stream)),
                    "t2t_attn_bwd_dkdv launch");
}

int t2t_attn_bwd_dq(const t2t_tensor* q, const t2t_tensor* k, const t2t_tensor* v,
                    const t2t_tensor* dout, const float* lse2, const float* delta,
                    const t2t_tensor* dq, int32_t B, int32_t Hq, int32_t Hkv, int32_t T,
                    int32_t D, int32_t dtype, float scale, const t2t_block_mask* mask, void* stream) {
  int rc = check_dims(B, Hq, Hkv, T, D, dtype);
  if (rc) return rc;
  rc = check_scale(scale);
  if (rc) return rc;
  if (B == 0 || Hq == 0 || T == 0) return T2T_OK;
  if (!view_ok(q, T, D) || !view_ok(k, T, D) || !view_ok(v, T, D) || !view_ok(dout, T, D) || !view_ok(dq, T, D))
    return fail(T2T_EINVAL, "tensor view invalid (NULL, misaligned, bad stride or slice >= 2 GiB)");
  if (!lse2 || !delta) return fail(T2T_EINVAL, "lse2/delta is NULL");
  rc = check_mask(mask, B, T, true, false);
  if (rc) return rc;
  const t2t::TensorView none{nullptr, 0, 0, 0};
  t2t::AttnDims dims{B, Hq, Hkv, T, D, scale};
  return hip_status(t2t::launch_attn_bwd_phase(t2t::kBwdDq, as_view(q), as_view(k), as_view(v),
                                               none, as_view(dout), lse2,
                                               const_cast<float*>(delta), as_view(dq), none,
                                               none, dims, as_tables(mask),
                                               static_cast<hipStream_t>(stream)),
                    "t2t_attn_bwd_dq launch");
}

int t2t_attn_bwd(const t2t_tensor* q, const t2t_tensor* k, const t2t_tensor* v,
                 const t2t_tensor* o, const t2t_tensor* dout, const float* lse2,
                 float* delta, const t2t_tensor* dq, const t2t_tensor* dk,
                 const t2t_tensor* dv, int32_t B, int32_t Hq, int32_t Hkv, int32_t T,
                 int32_t D, int32_t dtype, float scale, const t2t_block_mask* mask,
                 void* stream) {
  // Validate every argument before launching anything.
  int rc = check_dims(B, Hq, Hkv, T, D, dtype, true);
  if (rc) return rc;
  rc = check_scale(scale);
  if (rc) return rc;
  if (B == 0 || Hq == 0 || T == 0) return T2T_OK;
  const int es = dtype == T2T_DTYPE_F32 ? 4 : 2;
  if (!view_ok(q, T, D, es) || !view_ok(k, T, D, es) || !view_ok(v, T, D, es) ||
      !view_ok(o, T, D, es) || !view_ok(dout, T, D, es) || !view_ok(dq, T, D, es) ||
      !view_ok(dk, T, D, es) || !view_ok(dv, T, D, es))
    return fail(T2T_EINVAL, "tensor view invalid (NULL, misaligned, bad stride or slice >= 2 GiB)");
  if (!lse2 || !delta) return fail(T2T_EINVAL, "lse2/delta is NULL");
  rc = check_mask(mask, B, T, true, true);
  if (rc) return rc;
  t2t::AttnDims dims{B, Hq, Hkv, T, D, scale};
  if (dtype == T2T_DTYPE_F32)
    return hip_status(t2t::launch_attn_bwd_f32(as_view(q), as_view(k), as_view(v), as_view(o),
                                               as_view(dout), lse2, delta, as_view(dq),
                                               as_view(dk), as_view(dv), dims, as_tables(mask),
                                               static_cast<hipStream_t>(stream)),
                      "t2t_attn_bwd launch");
  // dQ first: it computes each row's Delta = rowsum(O * dO) from the dO rows
  // it holds and writes it for dK/dV, so no separate Delta launch is needed.
  rc = hip_status(t2t::launch_attn_bwd_phase(t2t::kBwdDqDelta, as_view(q), as_view(k),
                                             as_view(v), as_view(o), as_view(dout), lse2, delta,
                                             as_view(dq), t2t::TensorView{nullptr, 0, 0, 0},
                                             t2t::TensorView{nullptr, 0, 0, 0}, dims,
                                             as_tables(mask), static_cast<hipStream_t>(stream)),
                  "t2t_attn_bwd dQ launch");
  if (rc) return rc;
  return t2t_attn_bwd_dkdv(q, k, v, dout, lse2, delta, dk, dv, B, Hq, Hkv, T, D, dtype, scale,
                           mask, stream);
}

// Delta workspace of t2t_attn_bwd_noalloc: a file-scope device array instead
// of a caller buffer.  Every GPU the library runs on holds its own copy (16
// MiB) until the process ends; in host code `scratch` only names the symbol,
// so the entry point uses the device address hipGetSymbolAddress returns for
// the current device, looked up once per device.
constexpr int64_t kScratchFloats = int64_t(4) << 20;  // B * Hq * T rows of Delta
static __device__ __align__(256) float scratch[kScratchFloats];

namespace {

constexpr int kScratchDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch_addr[kScratchDevices] = {};

// This GPU's copy of `scratch` (the current device, as for every launch).
int current_scratch(float** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_status(e, "hipGetDevice");
  if (dev < 0 || dev >= kScratchDevices)
    return fail(T2T_EUNSUPPORTED, "device %d is past the %d devices the static workspace tracks",
                dev, kScratchDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_addr[dev]) {
    void* addr = nullptr;
    e = hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_status(e, "hipGetSymbolAddress(scratch)");
    g_scratch_addr[dev] = static_cast<float*>(addr);
  }
  *out = g_scratch_addr[dev];
  return T2T_OK;
}

}  // namespace

int t2t_attn_bwd_noalloc(const t2t_tensor* q, const t2t_tensor* k, const t2t_tensor* v,
                         const t2t_tensor* o, const t2t_tensor* dout, const float* lse2,
                         const t2t_tensor* dq, const t2t_tensor* dk, const t2t_tensor* dv,
                         int32_t B, int32_t Hq, int32_t Hkv, int32_t T, int32_t D, int32_t dtype,
                         float scale, const t2t_block_mask* mask, void* stream) {
  int rc = check_dims(B, Hq, Hkv, T, D, dtype, true);
  if (rc) return rc;
  rc = check_scale(scale);
  if (rc) return rc;
  if (B == 0 || Hq == 0 || T == 0) return T2T_OK;
  const int64_t rows = (int64_t)B * Hq * T;
  if (rows > kScratchFloats)
    return fail(T2T_EINVAL,
                "B*Hq*T = %lld Delta rows exceed the static workspace of %lld rows "
                "(use t2t_attn_bwd with a caller workspace)",
                (long long)rows, (long long)kScratchFloats);
  float* delta = nullptr;
  rc = current_scratch(&delta);
  if (rc) return rc;
  // Every row of Delta is written by the dQ launch before dK/dV reads it, so
  // the workspace needs no clearing between calls.
  return t2t_attn_bwd(q, k, v, o, dout, lse2, delta, dq, dk, dv, B, Hq, Hkv, T, D, dtype, scale,
                      mask, stream);
}

namespace {

// A [B, H, T, D] view the prologue kernels address with 16-byte vector
// accesses (plain global pointers, so no 2 GiB slice limit).
bool rope_view_ok(const t2t_tensor* t) {
  return t && t->data && (reinterpret_cast<uintptr_t>(t->data) % 16) == 0 && t->stride_b >= 0 &&
         t->stride_h >= 0 && t->stride_t > 0 && (t->stride_b % 8) == 0 &&
         (t->stride_h % 8) == 0 && (t->stride_t % 8) == 0;
}

int check_rope(int B, int T, int H, int D, const float* cos, const float* sin, int table_rows,
               int pos0, const void* packed, int64_t sb, int64_t st) {
  if (B < 0 || T < 0 || H < 0 || table_rows < 0 || pos0 < 0)
    return fail(T2T_EINVAL, "negative B, T, H, table_rows or pos0");
  if (D < 16 || D > 256 || D % 16 != 0)
    return fail(T2T_EUNSUPPORTED, "head dim %d is not a multiple of 16 in [16, 256]", D);
  if (B == 0 || T == 0 || H == 0) return T2T_OK;
  if ((int64_t)pos0 + T > table_rows)
    return fail(T2T_EINVAL, "positions %d..%d exceed the %d table rows", pos0, pos0 + T - 1,
                table_rows);
  if (!cos || !sin || !packed) return fail(T2T_EINVAL, "cos, sin or the packed qkv is NULL");
  if ((reinterpret_cast<uintptr_t>(cos) | reinterpret_cast<uintptr_t>(sin) |
       reinterpret_cast<uintptr_t>(packed)) % 16)
    return fail(T2T_EINVAL, "cos, sin and the packed qkv must be 16-byte aligned");
  if (sb < 0 || st < 0 || sb % 8 || st % 8)
    return fail(T2T_EINVAL, "packed strides must be non-negative multiples of 8 elements");
  if (T > 1 && st < 3LL * H * D)
    return fail(T2T_EINVAL, "packed token stride %lld is below 3*H*D = %lld", (long long)st,
                3LL * H * D);
  return T2T_OK;
}

}  // namespace

int t2t_qkv_rope(const void* qkv, int64_t qkv_sb, int64_t qkv_st, int32_t B, int32_t T,
                 int32_t H, int32_t D, const float* cos, const float* sin, int32_t table_rows,
                 int32_t pos0, const t2t_tensor* q, const t2t_tensor* k, const t2t_tensor* v,
                 void* stream) {
  int rc = check_rope(B, T, H, D, cos, sin, table_rows, pos0, qkv, qkv_sb, qkv_st);
  if (rc || B == 0 || T == 0 || H == 0) return rc;
  if (!rope_view_ok(q) || !rope_view_ok(k) || !rope_view_ok(v))
    return fail(T2T_EINVAL, "q/k/v view invalid (NULL, misaligned or bad stride)");
  return hip_status(t2t::launch_qkv_rope(static_cast<const __bf16*>(qkv), qkv_sb, qkv_st,
                                         as_view(q), as_view(k), as_view(v), cos, sin, B, T, H,
                                         D, pos0, static_cast<hipStream_t>(stream)),
                    "t2t_qkv_rope launch");
}

int t2t_qkv_rope_backward(const t2t_tensor* dq, const t2t_tensor* dk, const t2t_tensor* dv,
                          const float* cos, const float* sin, int32_t table_rows, int32_t pos0,
                          int32_t B, int32_t T, int32_t H, int32_t D, void* dqkv,
                          int64_t dqkv_sb, int64_t dqkv_st, void* stream) {
  int rc = check_rope(B, T, H, D, cos, sin, table_rows, pos0, dqkv, dqkv_sb, dqkv_st);
  if (rc || B == 0 || T == 0 || H == 0) return rc;
  if (!rope_view_ok(dq) || !rope_view_ok(dk) || !rope_view_ok(dv))
    return fail(T2T_EINVAL, "dq/dk/dv view invalid (NULL, misaligned or bad stride)");
  return hip_status(t2t::launch_qkv_rope_bwd(as_view(dq), as_view(dk), as_view(dv), cos, sin, B,
                                             T, H, D, pos0, static_cast<__bf16*>(dqkv), dqkv_sb,
                                             dqkv_st, static_cast<hipStream_t>(stream)),
                    "t2t_qkv_rope_backward launch");
}

int64_t t2t_attn_decode_workspace(int32_t B, int32_t Hq, int32_t Tq, int32_t Tkv, int32_t D) {
  if (B < 0 || Hq < 0 || Tq < 0 || Tkv < 0 || D < 0) return 0;
  return 4 * t2t::decode_workspace_floats(B, Hq, Tq, Tkv, D);
}

int t2t_attn_decode(const t2t_tensor* q, const t2t_tensor* k, const t2t_tensor* v,
                    const t2t_tensor* o, float* lse2, const int32_t* key_doc,
                    const uint64_t* key_bits, int64_t key_stride, const int32_t* q_pos,
                    const int32_t* q_doc, const uint64_t* q_bits, int32_t mask_batch,
                    int32_t words, int32_t B, int32_t Hq, int32_t Hkv, int32_t Tq, int32_t Tkv,
                    int32_t D, int32_t dtype, float scale, void* workspace,
                    int64_t workspace_bytes, void* stream) {
  if (B < 0 || Hq < 0 || Hkv < 0 || Tq < 0 || Tkv < 0 || mask_batch < 0 || key_stride < 0)
    return fail(T2T_EINVAL, "negative size or stride");
  if (dtype != T2T_DTYPE_BF16) return fail(T2T_EUNSUPPORTED, "dtype %d is not bf16", dtype);
  if (D != 64 && D != 128) return fail(T2T_EUNSUPPORTED, "head dim %d (64 or 128)", D);
  if (words < 0 || words > T2T_MAX_WORDS)
    return fail(T2T_EUNSUPPORTED, "words=%d outside [0, %d]", words, T2T_MAX_WORDS);
  if (int rc = check_scale(scale)) return rc;
  if (B == 0 || Hq == 0 || Tq == 0) return T2T_OK;
  if (Hkv == 0 || Hq % Hkv != 0)
    return fail(T2T_EINVAL, "Hq=%d is not a multiple of Hkv=%d", Hq, Hkv);
  if ((int64_t)(Hq / Hkv) * Tq > t2t::kDecodeMaxRows)
    return fail(T2T_EUNSUPPORTED, "(Hq / Hkv) * Tq = %lld query rows per kv head exceeds %d",
                (long long)(Hq / Hkv) * Tq, t2t::kDecodeMaxRows);
  if (!(mask_batch == 1 || mask_batch == B))
    return fail(T2T_EINVAL, "mask_batch %d does not broadcast to B=%d", mask_batch, B);
  if (key_stride < Tkv) return fail(T2T_EINVAL, "key_stride %lld < Tkv %d", (long long)key_stride, Tkv);
  if (!rope_view_ok(q) || !rope_view_ok(k) || !rope_view_ok(v) || !rope_view_ok(o))
    return fail(T2T_EINVAL, "q/k/v/o view invalid (NULL, misaligned or bad stride)");
  if (!lse2 || !key_doc || !q_pos || !q_doc || (words > 0 && (!key_bits || !q_bits)))
    return fail(T2T_EINVAL, "NULL pointer argument");
  const int64_t need = t2t_attn_decode_workspace(B, Hq, Tq, Tkv, D);
  if (!workspace || workspace_bytes < need)
    return fail(T2T_EINVAL, "workspace of %lld bytes, %lld needed", (long long)workspace_bytes,
                (long long)need);
  return hip_status(t2t::launch_attn_decode(as_view(q), as_view(k), as_view(v), as_view(o), lse2,
                                            key_doc, key_bits, key_stride, q_pos, q_doc, q_bits,
                                            mask_batch, words, B, Hq, Hkv, Tq, Tkv, D, scale,
                                            static_cast<float*>(workspace),
                                            static_cast<hipStream_t>(stream)),
                    "t2t_attn_decode launch");
}

namespace {

int check_norm(int N, int C, int wdt, const void* const* ptrs, int n_ptrs,
               const int64_t* strides, int n_strides) {
  if (N < 0 || C < 0) return fail(T2T_EINVAL, "negative N or C");
  if (C % 8 != 0 || C > 4096 || C == 0)
    return fail(T2T_EUNSUPPORTED, "row length %d is not a multiple of 8 in [8, 4096]", C);
  if (wdt != 0 && wdt != 1) return fail(T2T_EUNSUPPORTED, "weight dtype %d (0 bf16, 1 f32)", wdt);
  for (int i = 0; i < n_ptrs; ++i) {
    if (!ptrs[i]) return fail(T2T_EINVAL, "NULL pointer argument");
    if (reinterpret_cast<uintptr_t>(ptrs[i]) % 16)
      return fail(T2T_EINVAL, "row, weight and gradient pointers must be 16-byte aligned");
  }
  for (int i = 0; i < n_strides; ++i)
    if (strides[i] < C || strides[i] % 8)
      return fail(T2T_EINVAL, "row stride %lld is below C or not a multiple of 8",
                  (long long)strides[i]);
  return T2T_OK;
}

}  // namespace

int t2t_rms_norm(const void* x, int64_t x_stride, const void* weight, int32_t weight_dtype,
                 void* y, int64_t y_stride, float* rstd, int32_t N, int32_t C, float eps,
                 void* stream) {
  if (N == 0 && C >= 0) return T2T_OK;
  const void* ptrs[] = {x, weight, y};
  const int64_t strides[] = {x_stride, y_stride};
  int rc = check_norm(N, C, weight_dtype, ptrs, 3, strides, 2);
  if (rc) return rc;
  if (!rstd) return fail(T2T_EINVAL, "rstd is NULL");
  return hip_status(t2t::launch_rmsnorm_fwd(static_cast<const __bf16*>(x), x_stride, weight,
                                            weight_dtype == 1, static_cast<__bf16*>(y), y_stride,
                                            rstd, N, C, eps, static_cast<hipStream_t>(stream)),
                    "t2t_rms_norm launch");
}

int64_t t2t_wgrad_workspace(int32_t M, int32_t N, int32_t K) {
  if (M <= 0 || N <= 0 || K <= 0 || M % 128 || N % 128 || K % 64) return 0;
  return (int64_t)t2t::wgrad_splits(M, N, K) * M * N * 4;
}

int t2t_wgrad(const void* a, int64_t lda, const void* b, int64_t ldb, void* out,
              int32_t out_dtype, int32_t M, int32_t N, int32_t K, void* workspace,
              int64_t workspace_bytes, void* stream) {
  if (M <= 0 || N <= 0 || K <= 0) return fail(T2T_EINVAL, "M=%d N=%d K=%d", M, N, K);
  if (M % 128 || N % 128 || K % 64)
    return fail(T2T_EUNSUPPORTED, "M=%d N=%d K=%d: need M, N multiples of 128 and K of 64", M,
                N, K);
  if (out_dtype != T2T_DTYPE_BF16 && out_dtype != T2T_DTYPE_F32)
    return fail(T2T_EINVAL, "out_dtype=%d", out_dtype);
  if (!a || !b || !out || !workspace) return fail(T2T_EINVAL, "a / b / out / workspace is NULL");
  if ((reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(b) |
       reinterpret_cast<uintptr_t>(out) | reinterpret_cast<uintptr_t>(workspace)) & 15)
    return fail(T2T_EINVAL, "buffers must be 16-byte aligned");
  if (lda % 8 || ldb % 8 || lda < M || ldb < N)
    return fail(T2T_EINVAL, "lda=%lld ldb=%lld: need multiples of 8, >= M / N", (long long)lda,
                (long long)ldb);
  const int64_t need = t2t_wgrad_workspace(M, N, K);
  if (workspace_bytes < need)
    return fail(T2T_EINVAL, "workspace of %lld bytes, %lld needed", (long long)workspace_bytes,
                (long long)need);
  return hip_status(t2t::launch_wgrad(static_cast<const __bf16*>(a), lda,
                                      static_cast<const __bf16*>(b), ldb,
                                      static_cast<float*>(workspace), out,
                                      out_dtype == T2T_DTYPE_F32, M, N, K,
                                      static_cast<hipStream_t>(stream)),
                    "t2t_wgrad launch");
}

namespace {

int check_swiglu(int32_t N, int32_t H, const void* const* ptrs, int np, const int64_t* strides,
                 int ns, const int64_t* min_strides) {
  if (N < 0 || H <= 0 || H % 8 != 0)
    return fail(T2T_EINVAL, "N=%d H=%d: need H > 0, H %% 8 == 0", N, H);
  for (int i = 0; i < np; ++i) {
    if (!ptrs[i]) return fail(T2T_EINVAL, "NULL buffer");
    if (reinterpret_cast<uintptr_t>(ptrs[i]) & 15)
      return fail(T2T_EINVAL, "buffers must be 16-byte aligned");
  }
  for (int i = 0; i < ns; ++i)
    if (strides[i] % 8 != 0 || strides[i] < min_strides[i])
      return fail(T2T_EINVAL, "row stride %lld (need a multiple of 8, >= %lld)",
                  (long long)strides[i], (long long)min_strides[i]);
  return T2T_OK;
}

}  // namespace

int t2t_swiglu(const void* gu, int64_t gu_stride, void* h, int64_t h_stride, int32_t N, int32_t H,
               void* stream) {
  const void* ptrs[] = {gu, h};
  const int64_t strides[] = {gu_stride, h_stride};
  const int64_t mins[] = {2 * (int64_t)H, H};
  const int rc = check_swiglu(N, H, ptrs, 2, strides, 2, mins);
  if (rc) return rc;
  return hip_status(t2t::launch_swiglu_fwd(static_cast<const __bf16*>(gu), gu_stride,
                                           static_cast<__bf16*>(h), h_stride, N, H,
                                           static_cast<hipStream_t>(stream)),
                    "t2t_swiglu launch");
}

int t2t_swiglu_backward(const void* gu, int64_t gu_stride, const void* dh, int64_t dh_stride,
                        void* dgu, int64_t dgu_stride, int32_t N, int32_t H, void* stream) {
  const void* ptrs[] = {gu, dh, dgu};
  const int64_t strides[] = {gu_stride, dh_stride, dgu_stride};
  const int64_t mins[] = {2 * (int64_t)H, H, 2 * (int64_t)H};
  const int rc = check_swiglu(N, H, ptrs, 3, strides, 3, mins);
  if (rc) return rc;
  return hip_status(t2t::launch_swiglu_bwd(static_cast<const __bf16*>(gu), gu_stride,
                                           static_cast<const __bf16*>(dh), dh_stride,
                                           static_cast<__bf16*>(dgu), dgu_stride, N, H,
                                           static_cast<hipStream_t>(stream)),
                    "t2t_swiglu_backward launch");
}

int t2t_ce_rows(const void* logits, void* grad, int64_t rows, int32_t V, int64_t ld,
                const int64_t* target, int64_t ignore_index, const float* scale, float* row_loss,
                void* stream) {
  if (rows < 0 || rows > 0x7fffffffLL) return fail(T2T_EINVAL, "rows=%lld", (long long)rows);
  if (V < 1 || ld < V || ld % 8 != 0)
    return fail(T2T_EINVAL, "V=%d ld=%lld: need 1 <= V <= ld and ld %% 8 == 0", V, (long long)ld);
  if (rows == 0) return T2T_OK;
  if (!logits || !grad || !target || !scale || !row_loss)
    return fail(T2T_EINVAL, "logits / grad / target / scale / row_loss is NULL");
  if ((reinterpret_cast<uintptr_t>(logits) | reinterpret_cast<uintptr_t>(grad)) & 15)
    return fail(T2T_EINVAL, "logits and grad must be 16-byte aligned");
  return hip_status(t2t::launch_ce_rows(static_cast<const uint16_t*>(logits),
                                        static_cast<uint16_t*>(grad), rows, V, ld, target,
                                        ignore_index, scale, row_loss,
                                        static_cast<hipStream_t>(stream)),
                    "t2t_ce_rows launch");
}

int64_t t2t_rms_norm_backward_workspace(int32_t N, int32_t C) {
  if (N <= 0 || C <= 0) return 0;
  return (int64_t)t2t::rmsnorm_bwd_groups(N, C) * C * 4;
}

int t2t_rms_norm_backward(const void* dy, int64_t dy_stride, const void* x, int64_t x_stride,
                          const void* weight, int32_t weight_dtype, const float* rstd, void* dx,
                          int64_t dx_stride, void* dweight, void* workspace,
                          int64_t workspace_bytes, int32_t N, int32_t C, void* stream) {
  if (N == 0 && C >= 0) return T2T_OK;
  const void* ptrs[] = {dy, x, weight, dx, dweight};
  const int64_t strides[] = {dy_stride, x_stride, dx_stride};
  int rc = check_norm(N, C, weight_dtype, ptrs, 5, strides, 3);
  if (rc) return rc;
  if (!rstd) return fail(T2T_EINVAL, "rstd is NULL");
  const int64_t need = t2t_rms_norm_backward_workspace(N, C);
  if (!workspace || workspace_bytes < need)
    return fail(T2T_EINVAL, "workspace of %lld bytes, %lld needed", (long long)workspace_bytes,
                (long long)need);
  return hip_status(
      t2t::launch_rmsnorm_bwd(static_cast<const __bf16*>(dy), dy_stride,
                              static_cast<const __bf16*>(x), x_stride, weight, weight_dtype == 1,
                              rstd, static_cast<__bf16*>(dx), dx_stride, dweight,
                              static_cast<float*>(workspace), N, C,
                              static_cast<hipStream_t>(stream)),
      "t2t_rms_norm_backward launch");
}

}  // extern "C"

namespace {

int check_rows(int M, int K, int N, const void* x, int64_t x_stride, const void* weight,
               const void* norm_weight, int norm_dtype) {
  if (M < 0 || M > t2t::kRowsMaxRows)
    return fail(T2T_EUNSUPPORTED, "M = %d rows; 0 to %d supported", M, t2t::kRowsMaxRows);
  if (K < 1 || K > 4096) return fail(T2T_EUNSUPPORTED, "K = %d outside [1, 4096]", K);
  if (N < 1) return fail(T2T_EINVAL, "N = %d", N);
  if (!x || !weight) return fail(T2T_EINVAL, "x or weight is NULL");
  if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(weight)) % 2)
    return fail(T2T_EINVAL, "x and weight must be 2-byte aligned");
  if (x_stride < K) return fail(T2T_EINVAL, "x row stride %lld is below K", (long long)x_stride);
  if (norm_weight) {
    if (norm_dtype != 0 && norm_dtype != 1)
      return fail(T2T_EUNSUPPORTED, "norm weight dtype %d (0 bf16, 1 f32)", norm_dtype);
    if (reinterpret_cast<uintptr_t>(norm_weight) % (norm_dtype ? 4 : 2))
      return fail(T2T_EINVAL, "norm weight misaligned for its dtype");
  }
  return T2T_OK;
}

}  // namespace

extern "C" {

int t2t_rows_linear(const void* x, int64_t x_stride, int32_t M, int32_t K, const void* weight,
                    int32_t N, const void* norm_weight, int32_t norm_dtype, float eps,
                    int32_t epilogue, const void* res, int64_t res_stride, const void* skip,
                    int64_t skip_stride, const void* skip_weight, int32_t skip_weight_dtype,
                    void* y, int64_t y_stride, void* stream) {
  int rc = check_rows(M, K, N, x, x_stride, weight, norm_weight, norm_dtype);
  if (rc) return rc;
  if (epilogue != T2T_ROWS_STORE && epilogue != T2T_ROWS_ADD && epilogue != T2T_ROWS_SWIGLU)
    return fail(T2T_EUNSUPPORTED, "epilogue %d (0 store, 1 add, 2 swiglu)", epilogue);
  if (!y) return fail(T2T_EINVAL, "y is NULL");
  if (y_stride < N) return fail(T2T_EINVAL, "y row stride %lld is below N", (long long)y_stride);
  if (epilogue == T2T_ROWS_ADD && (!res || res_stride < N))
    return fail(T2T_EINVAL, "the add epilogue needs res with a row stride of at least N");
  if (skip_weight) {
    if (epilogue != T2T_ROWS_ADD)
      return fail(T2T_EINVAL, "a skip residual is only taken by the add epilogue");
    if (skip_weight_dtype != 0 && skip_weight_dtype != 1)
      return fail(T2T_EUNSUPPORTED, "skip weight dtype %d (0 bf16, 1 f32)", skip_weight_dtype);
    if (skip && skip_stride < N)
      return fail(T2T_EINVAL, "skip row stride %lld is below N", (long long)skip_stride);
  } else if (skip) {
    return fail(T2T_EINVAL, "skip rows given without a skip weight");
  }
  if (M == 0) return T2T_OK;
  return hip_status(
      t2t::launch_rows_linear(epilogue, static_cast<const __bf16*>(x), x_stride, M, K,
                              static_cast<const __bf16*>(weight), N, norm_weight, norm_dtype == 1,
                              eps, static_cast<const __bf16*>(res), res_stride,
                              static_cast<const __bf16*>(skip), skip_stride, skip_weight,
                              skip_weight_dtype == 1, static_cast<__bf16*>(y), y_stride,
                              static_cast<hipStream_t>(stream)),
      "t2t_rows_linear launch");
}

int t2t_rows_qkv_rope(const void* x, int64_t x_stride, int32_t M, int32_t K, const void* weight,
                      const void* norm_weight, int32_t norm_dtype, float eps, int32_t H,
                      int32_t D, const float* cos, const float* sin, int32_t table_rows,
                      const int64_t* pos, int32_t pos0, const t2t_tensor* q,
                      const t2t_tensor* k_cache, const t2t_tensor* v_cache, int32_t cache_rows,
                      void* stream) {
  if (H < 1 || D < 2 || D % 2 || (int64_t)H * D > (1 << 20))
    return fail(T2T_EUNSUPPORTED, "H = %d, D = %d (H >= 1, even D)", H, D);
  int rc = check_rows(M, K, H * D, x, x_stride, weight, norm_weight, norm_dtype);
  if (rc) return rc;
  if (!cos || !sin) return fail(T2T_EINVAL, "cos or sin is NULL");
  if (table_rows < 0 || cache_rows < 0 || pos0 < 0)
    return fail(T2T_EINVAL, "negative table_rows, cache_rows or pos0");
  if (!pos && (int64_t)pos0 + M > std::min(table_rows, cache_rows))
    return fail(T2T_EINVAL, "positions %d..%d exceed the %d table rows or %d cache rows", pos0,
                pos0 + M - 1, table_rows, cache_rows);
  for (const t2t_tensor* t : {q, k_cache, v_cache})
    if (!t || !t->data || t->stride_h < 0 || t->stride_t <= 0)
      return fail(T2T_EINVAL, "q / k_cache / v_cache view invalid (NULL or bad stride)");
  if (M == 0) return T2T_OK;
  return hip_status(
      t2t::launch_rows_qkv_rope(static_cast<const __bf16*>(x), x_stride, M, K,
                                static_cast<const __bf16*>(weight), norm_weight, norm_dtype == 1,
                                eps, H, D, cos, sin, pos, pos0, std::min(table_rows, cache_rows),
                                as_view(q), as_view(k_cache), as_view(v_cache),
                                static_cast<hipStream_t>(stream)),
      "t2t_rows_qkv_rope launch");
}

int t2t_first_input_diff(const int64_t* tokens_a, const int64_t* tokens_b, const int32_t* doc_a,
                         const int32_t* doc_b, const uint64_t* q_bits_a, const uint64_t* q_bits_b,
                         const uint64_t* kv_bits_a, const uint64_t* kv_bits_b,
                         int64_t bits_stride_a, int64_t bits_stride_b, int32_t words, int32_t n,
                         int32_t* out, void* stream) {
  if (n < 0 || words < 0 || words > T2T_MAX_WORDS)
    return fail(T2T_EINVAL, "n = %d, words = %d (0 to %d)", n, words, T2T_MAX_WORDS);
  if (!out) return fail(T2T_EINVAL, "out is NULL");
  if (n > 0 && (!tokens_a || !tokens_b || !doc_a || !doc_b))
    return fail(T2T_EINVAL, "token or doc array is NULL");
  if (n > 0 && words > 0) {
    if (!q_bits_a || !q_bits_b || !kv_bits_a || !kv_bits_b)
      return fail(T2T_EINVAL, "a grant-word array is NULL");
    if (bits_stride_a < n || bits_stride_b < n)
      return fail(T2T_EINVAL, "grant-word stride below n");
  }
  return hip_status(t2t::launch_first_input_diff(tokens_a, tokens_b, doc_a, doc_b, q_bits_a,
                                                 q_bits_b, kv_bits_a, kv_bits_b, bits_stride_a,
                                                 bits_stride_b, words, n, out,
                                                 static_cast<hipStream_t>(stream)),
                    "t2t_first_input_diff launch");
}

int t2t_clock_probe(uint64_t* out, int32_t iters, int32_t* wall_khz, void* stream) {
  if (!out || !wall_khz) return fail(T2T_EINVAL, "out or wall_khz is NULL");
  if (iters < 1 || iters > 10000000) return fail(T2T_EINVAL, "iters=%d outside [1, 1e7]", iters);
  int khz = 0;
  hipError_t e = t2t::wall_clock_khz(&khz);
  if (e != hipSuccess) return hip_status(e, "wall-clock rate query");
  *wall_khz = khz;
  return hip_status(t2t::launch_clock_probe(out, iters, static_cast<hipStream_t>(stream)),
                    "t2t_clock_probe launch");
}

}  // extern "C"
