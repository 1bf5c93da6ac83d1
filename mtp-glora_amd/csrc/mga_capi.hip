// C ABI entry points (declared in include/mtp_glora_amd.h): argument checks,
// then kernel launches on the caller's stream. No device allocation happens here.
#include <math.h>
#include <stdarg.h>
#include <stdio.h>

#include <algorithm>
#include <mutex>

#include "../../include/mtp_glora_amd.h"
#include "mga_common.hpp"
#include "mga_internal.hpp"

static_assert(MGA_BWD_DQ == mga::kBwdDq && MGA_BWD_DKDV == mga::kBwdDkDv, "pass flags");
static_assert(MGA_DTYPE_BF16 == mga::kDtBf16 && MGA_DTYPE_F32 == mga::kDtF32 && MGA_DTYPE_F16 == mga::kDtF16,
              "dtype codes");

namespace mga {

int device_cu_count() {
  static int counts[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (counts[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    counts[dev] = n;
  }
  return counts[dev];
}

}  // namespace mga

namespace {

thread_local char g_err[1024] = {0};

int fail(int code, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char *what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(MGA_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
  g_err[0] = 0;
  return MGA_OK;
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

int elem_bytes(int dtype) {
  return (dtype == MGA_DTYPE_BF16 || dtype == MGA_DTYPE_F16) ? 2 : (dtype == MGA_DTYPE_F32 ? 4 : 0);
}

// A [heads, rows, head_dim] operand addressed with element strides: every row
// start must be 16-byte aligned for the vector loads.
int check_operand(const char *name, const void *p, int64_t sh, int64_t ss, int eb) {
  if (!p) return fail(MGA_ERR_INVALID, "%s: null pointer", name);
  if (!aligned16(p)) return fail(MGA_ERR_INVALID, "%s: base pointer not 16-byte aligned", name);
  if (sh < 0 || ss <= 0) return fail(MGA_ERR_INVALID, "%s: invalid strides (%lld, %lld)", name,
                                      (long long)sh, (long long)ss);
  // tile loads address up to 128 rows with 32-bit per-lane offsets
  if (ss >= (int64_t(1) << 23))
    return fail(MGA_ERR_INVALID, "%s: row stride %lld elements is too large (limit 2^23)", name, (long long)ss);
  if (((sh * eb) & 15) || ((ss * eb) & 15))
    return fail(MGA_ERR_INVALID, "%s: strides (%lld, %lld) elements are not multiples of 16 bytes",
                name, (long long)sh, (long long)ss);
  return MGA_OK;
}

int check_attn_common(int32_t S, int32_t L, int32_t P, int32_t Hq, int32_t Hkv, int32_t hd,
                      int32_t dtype, float scale) {
  if (S <= 0) return fail(MGA_ERR_INVALID, "S must be positive (got %d)", S);
  // the kernels mask a score to -inf before it is scaled
  if (!(scale > 0.f) || !(scale < __builtin_huge_valf()))
    return fail(MGA_ERR_INVALID, "scale must be positive and finite (got %g)", (double)scale);
  if (P < 0 || L != P + S) return fail(MGA_ERR_INVALID, "need L == P + S (L=%d P=%d S=%d)", L, P, S);
  if (Hq <= 0 || Hkv <= 0 || Hq % Hkv) return fail(MGA_ERR_INVALID, "Hq (%d) must be a positive multiple of Hkv (%d)", Hq, Hkv);
  if (hd != 64 && hd != 128) return fail(MGA_ERR_INVALID, "head_dim must be 64 or 128 (got %d)", hd);
  if (!elem_bytes(dtype)) return fail(MGA_ERR_INVALID, "unknown dtype code %d", dtype);
  return MGA_OK;
}

// Workspace of mga_attn_bwd_noalloc (the backward's row data: three words per
// query head and row): a device array of 3 * kNoAllocRows floats, one copy on
// every GPU the library runs on, held until the process ends. Host code
// reaches it only through the address hipGetSymbolAddress returns for the
// current device.
constexpr int64_t kNoAllocRows = int64_t(1) << 21;   // Hq * S <= 2 097 152 (24 MiB)
static __device__ __align__(256) float scratch[MGA_BWD_WS_WORDS_PER_ROW * kNoAllocRows];

std::mutex g_scratch_mu;
constexpr int kMaxDevices = 256;
float *g_scratch_ptr[kMaxDevices] = {};

// The current device's copy of scratch, looked up once per device.
int scratch_for_current_device(float **out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(MGA_ERR_HIP, "mga_attn_bwd_noalloc: hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return fail(MGA_ERR_INVALID, "mga_attn_bwd_noalloc: device id %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    float *ptr = nullptr;
    e = hipGetSymbolAddress((void **)&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr)
      return fail(MGA_ERR_HIP, "mga_attn_bwd_noalloc: hipGetSymbolAddress(scratch) on device %d: %s", dev,
                  hipGetErrorString(e));
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return MGA_OK;
}

}  // namespace

extern "C" {

int mga_version(void) { return 100; }

const char *mga_last_error(void) { return g_err; }

int mga_kv_append(const void *src_k, const void *src_v, int64_t src_stride_h, int64_t src_stride_s,
                  int64_t src_rows, const int32_t *idx, int32_t n_rows, void *dst_k, void *dst_v,
                  int64_t dst_stride_h, int64_t dst_stride_s, int64_t dst_offset,
                  int64_t dst_capacity, int32_t n_heads, int32_t head_dim, int32_t dtype,
                  void *stream) {
  const int eb = elem_bytes(dtype);
  if (!eb) return fail(MGA_ERR_INVALID, "mga_kv_append: unknown dtype code %d", dtype);
  if (n_rows < 0 || n_heads <= 0 || head_dim <= 0)
    return fail(MGA_ERR_INVALID, "mga_kv_append: bad sizes (rows=%d heads=%d head_dim=%d)", n_rows,
                n_heads, head_dim);
  const int row_bytes = head_dim * eb;
  if (row_bytes < 16 || (row_bytes & (row_bytes - 1)))
    return fail(MGA_ERR_INVALID, "mga_kv_append: head_dim*elem (%d bytes) must be a power of two >= 16",
                row_bytes);
  if (src_rows < 0 || (!idx && n_rows > src_rows))
    return fail(MGA_ERR_INVALID, "mga_kv_append: %d rows requested from a %lld-row source", n_rows,
                (long long)src_rows);
  if (dst_offset < 0 || dst_offset + n_rows > dst_capacity)
    return fail(MGA_ERR_CAPACITY, "mga_kv_append: rows [%lld, %lld) exceed the cache capacity %lld",
                (long long)dst_offset, (long long)(dst_offset + n_rows), (long long)dst_capacity);
  int rc;
  if ((rc = check_operand("src_k", src_k, src_stride_h, src_stride_s, eb))) return rc;
  if ((rc = check_operand("src_v", src_v, src_stride_h, src_stride_s, eb))) return rc;
  if ((rc = check_operand("dst_k", dst_k, dst_stride_h, dst_stride_s, eb))) return rc;
  if ((rc = check_operand("dst_v", dst_v, dst_stride_h, dst_stride_s, eb))) return rc;
  if ((int64_t)n_rows * (row_bytes / 16) > 0x7fffffffLL)
    return fail(MGA_ERR_INVALID, "mga_kv_append: too many rows per head (%d)", n_rows);
  if (n_rows == 0) { g_err[0] = 0; return MGA_OK; }
  mga::launch_kv_copy_rows(src_k, src_v, src_stride_h * eb, src_stride_s * eb, src_rows, idx, n_rows, dst_k,
                           dst_v, dst_stride_h * eb, dst_stride_s * eb, dst_offset, n_heads,
                           row_bytes, (hipStream_t)stream);
  return check_launch("mga_kv_append");
}

int mga_regular_index(const int64_t *regular_mask, int64_t stride, int32_t n, int32_t *idx,
                      int32_t *count, void *stream) {
  if (!regular_mask || !idx || !count) return fail(MGA_ERR_INVALID, "mga_regular_index: null pointer");
  if (n <= 0 || stride <= 0) return fail(MGA_ERR_INVALID, "mga_regular_index: bad size/stride (%d, %lld)", n, (long long)stride);
  mga::launch_regular_index(regular_mask, stride, n, idx, count, (hipStream_t)stream);
  return check_launch("mga_regular_index");
}

int mga_mtp_block_mask(const int64_t *gate, int64_t gate_stride, int32_t S, int64_t P,
                       int32_t *code, int8_t *tile_class, int32_t *kv_num, int32_t *kv_idx,
                       int32_t *full_kv_num, int32_t *full_kv_idx, int32_t *q_num, int32_t *q_idx,
                       int32_t *full_q_num, int32_t *full_q_idx, void *stream) {
  if (!gate || !code || !tile_class || !kv_num || !kv_idx || !full_kv_num || !full_kv_idx ||
      !q_num || !q_idx || !full_q_num || !full_q_idx)
    return fail(MGA_ERR_INVALID, "mga_mtp_block_mask: null pointer");
  if (S <= 0 || P < 0 || gate_stride <= 0 || P + S > 0x7fffffffLL)
    return fail(MGA_ERR_INVALID, "mga_mtp_block_mask: bad sizes (S=%d P=%lld stride=%lld)", S,
                (long long)P, (long long)gate_stride);
  mga::launch_mtp_block_mask(gate, gate_stride, S, P, code, tile_class, kv_num, kv_idx, full_kv_num,
                             full_kv_idx, q_num, q_idx, full_q_num, full_q_idx, (hipStream_t)stream);
  return check_launch("mga_mtp_block_mask");
}

int mga_attn_fwd(const void *q, int64_t q_sh, int64_t q_ss, const void *k, int64_t k_sh,
                 int64_t k_ss, const void *v, int64_t v_sh, int64_t v_ss, void *o, int64_t o_sh,
                 int64_t o_ss, float *lse, const int32_t *code, const int32_t *kv_num,
                 const int32_t *kv_idx, const int32_t *full_kv_num, const int32_t *full_kv_idx,
                 int32_t S, int32_t L, int32_t P, int32_t Hq, int32_t Hkv, int32_t head_dim,
                 int32_t dtype, float scale, void *stream) {
  int rc;
  if ((rc = check_attn_common(S, L, P, Hq, Hkv, head_dim, dtype, scale))) return rc;
  const int eb = elem_bytes(dtype);
  if ((rc = check_operand("q", q, q_sh, q_ss, eb))) return rc;
  if ((rc = check_operand("k", k, k_sh, k_ss, eb))) return rc;
  if ((rc = check_operand("v", v, v_sh, v_ss, eb))) return rc;
  if ((rc = check_operand("o", o, o_sh, o_ss, eb))) return rc;
  if (!lse || !code || !kv_num || !kv_idx || !full_kv_num || !full_kv_idx)
    return fail(MGA_ERR_INVALID, "mga_attn_fwd: null lse/code/block-mask pointer");
  mga::AttnArgs a = {};
  a.q = q; a.q_sh = q_sh; a.q_ss = q_ss;
  a.k = k; a.k_sh = k_sh; a.k_ss = k_ss;
  a.v = v; a.v_sh = v_sh; a.v_ss = v_ss;
  a.o = o; a.o_sh = o_sh; a.o_ss = o_ss;
  a.lse = lse; a.code = code;
  a.kv_num = kv_num; a.kv_idx = kv_idx; a.fkv_num = full_kv_num; a.fkv_idx = full_kv_idx;
  a.S = S; a.L = L; a.P = P; a.Hq = Hq; a.Hkv = Hkv;
  a.nQ = (S + MGA_BLOCK - 1) / MGA_BLOCK;
  a.nKV = (L + MGA_BLOCK - 1) / MGA_BLOCK;
  a.scale = scale;
  a.scale_log2 = scale * mga::kLog2e;
  mga::launch_attn_fwd(a, head_dim, dtype, (hipStream_t)stream);
  return check_launch("mga_attn_fwd");
}

int mga_attn_bwd(const void *q, int64_t q_sh, int64_t q_ss, const void *k, int64_t k_sh,
                 int64_t k_ss, const void *v, int64_t v_sh, int64_t v_ss, const void *o,
                 int64_t o_sh, int64_t o_ss, const void *dout, int64_t do_sh, int64_t do_ss,
                 const float *lse, float *delta, void *dq, int64_t dq_sh, int64_t dq_ss, void *dk,
                 int64_t dk_sh, int64_t dk_ss, void *dv, int64_t dv_sh, int64_t dv_ss,
                 int32_t grad_start, const int32_t *code, const int32_t *kv_num,
                 const int32_t *kv_idx, const int32_t *full_kv_num, const int32_t *full_kv_idx,
                 const int32_t *q_num, const int32_t *q_idx, const int32_t *full_q_num,
                 const int32_t *full_q_idx, int32_t S, int32_t L, int32_t P, int32_t Hq,
                 int32_t Hkv, int32_t head_dim, int32_t dtype, float scale, int32_t passes,
                 void *stream) {
  int rc;
  if ((rc = check_attn_common(S, L, P, Hq, Hkv, head_dim, dtype, scale))) return rc;
  if (passes <= 0 || (passes & ~(MGA_BWD_DQ | MGA_BWD_DKDV)))
    return fail(MGA_ERR_INVALID, "mga_attn_bwd: passes must be a non-empty set of MGA_BWD_DQ | MGA_BWD_DKDV (got %d)", passes);
  const int eb = elem_bytes(dtype);
  if ((rc = check_operand("q", q, q_sh, q_ss, eb))) return rc;
  if ((rc = check_operand("k", k, k_sh, k_ss, eb))) return rc;
  if ((rc = check_operand("v", v, v_sh, v_ss, eb))) return rc;
  if ((rc = check_operand("o", o, o_sh, o_ss, eb))) return rc;
  if ((rc = check_operand("dout", dout, do_sh, do_ss, eb))) return rc;
  if ((passes & MGA_BWD_DQ) && (rc = check_operand("dq", dq, dq_sh, dq_ss, eb))) return rc;
  if (grad_start < 0 || grad_start > L)
    return fail(MGA_ERR_INVALID, "mga_attn_bwd: grad_start %d outside [0, L=%d]", grad_start, L);
  if ((passes & MGA_BWD_DKDV) && grad_start < L) {
    if ((rc = check_operand("dk", dk, dk_sh, dk_ss, eb))) return rc;
    if ((rc = check_operand("dv", dv, dv_sh, dv_ss, eb))) return rc;
  }
  if (!lse || !delta || !code || !kv_num || !kv_idx || !full_kv_num || !full_kv_idx || !q_num ||
      !q_idx || !full_q_num || !full_q_idx)
    return fail(MGA_ERR_INVALID, "mga_attn_bwd: null lse/delta/code/block-mask pointer");
  // the dK/dV pass addresses the workspace with 32-bit byte offsets
  if ((int64_t)Hq * S * MGA_BWD_WS_WORDS_PER_ROW * 4 >= (int64_t(1) << 32) - 16)
    return fail(MGA_ERR_INVALID, "mga_attn_bwd: Hq * S = %lld too large for the delta workspace",
                (long long)Hq * S);
  if (!aligned16(delta)) return fail(MGA_ERR_INVALID, "mga_attn_bwd: delta workspace not 16-byte aligned");
  mga::AttnArgs a = {};
  a.q = q; a.q_sh = q_sh; a.q_ss = q_ss;
  a.k = k; a.k_sh = k_sh; a.k_ss = k_ss;
  a.v = v; a.v_sh = v_sh; a.v_ss = v_ss;
  a.o = o; a.o_sh = o_sh; a.o_ss = o_ss;
  a.dout = dout; a.do_sh = do_sh; a.do_ss = do_ss;
  a.lse = const_cast<float *>(lse); a.delta = delta;
  a.dq = dq; a.dq_sh = dq_sh; a.dq_ss = dq_ss;
  a.dk = dk; a.dk_sh = dk_sh; a.dk_ss = dk_ss;
  a.dv = dv; a.dv_sh = dv_sh; a.dv_ss = dv_ss;
  a.grad_start = grad_start; a.code = code;
  a.kv_num = kv_num; a.kv_idx = kv_idx; a.fkv_num = full_kv_num; a.fkv_idx = full_kv_idx;
  a.q_num = q_num; a.q_idx = q_idx; a.fq_num = full_q_num; a.fq_idx = full_q_idx;
  a.S = S; a.L = L; a.P = P; a.Hq = Hq; a.Hkv = Hkv;
  a.nQ = (S + MGA_BLOCK - 1) / MGA_BLOCK;
  a.nKV = (L + MGA_BLOCK - 1) / MGA_BLOCK;
  a.scale = scale;
  a.scale_log2 = scale * mga::kLog2e;
  mga::launch_attn_bwd(a, head_dim, dtype, passes, (hipStream_t)stream);
  return check_launch("mga_attn_bwd");
}

int mga_attn_bwd_noalloc(const void *q, int64_t q_sh, int64_t q_ss, const void *k, int64_t k_sh,
                         int64_t k_ss, const void *v, int64_t v_sh, int64_t v_ss, const void *o,
                         int64_t o_sh, int64_t o_ss, const void *dout, int64_t do_sh, int64_t do_ss,
                         const float *lse, void *dq, int64_t dq_sh, int64_t dq_ss, void *dk,
                         int64_t dk_sh, int64_t dk_ss, void *dv, int64_t dv_sh, int64_t dv_ss,
                         int32_t grad_start, const int32_t *code, const int32_t *kv_num,
                         const int32_t *kv_idx, const int32_t *full_kv_num, const int32_t *full_kv_idx,
                         const int32_t *q_num, const int32_t *q_idx, const int32_t *full_q_num,
                         const int32_t *full_q_idx, int32_t S, int32_t L, int32_t P, int32_t Hq,
                         int32_t Hkv, int32_t head_dim, int32_t dtype, float scale, int32_t passes,
                         void *stream) {
  if (Hq <= 0 || S <= 0) return fail(MGA_ERR_INVALID, "mga_attn_bwd_noalloc: Hq (%d) and S (%d) must be positive", Hq, S);
  if ((int64_t)Hq * S > kNoAllocRows)
    return fail(MGA_ERR_INVALID,
                "mga_attn_bwd_noalloc: Hq * S = %lld exceeds its fixed workspace of %lld (query head, row) "
                "pairs; use mga_attn_bwd with a caller-allocated delta",
                (long long)Hq * S, (long long)kNoAllocRows);
  float *delta = nullptr;
  int rc = scratch_for_current_device(&delta);
  if (rc != MGA_OK) return rc;
  return mga_attn_bwd(q, q_sh, q_ss, k, k_sh, k_ss, v, v_sh, v_ss, o, o_sh, o_ss, dout, do_sh, do_ss, lse,
                      delta, dq, dq_sh, dq_ss, dk, dk_sh, dk_ss, dv, dv_sh, dv_ss, grad_start, code, kv_num,
                      kv_idx, full_kv_num, full_kv_idx, q_num, q_idx, full_q_num, full_q_idx, S, L, P, Hq,
                      Hkv, head_dim, dtype, scale, passes, stream);
}

namespace {

int check_qk_rope(const char *fn, const void *q, const void *k, const void *qw, const void *kw, const void *c,
                  const void *sn, const float *rstd, int32_t S, int32_t Hq, int32_t Hkv, int32_t D, int32_t dtype) {
  if (!elem_bytes(dtype)) return fail(MGA_ERR_INVALID, "%s: unknown dtype code %d", fn, dtype);
  if (S <= 0 || Hq <= 0 || Hkv <= 0) return fail(MGA_ERR_INVALID, "%s: bad sizes (S=%d Hq=%d Hkv=%d)", fn, S, Hq, Hkv);
  if (D <= 0 || D > 128 || (D & 1)) return fail(MGA_ERR_INVALID, "%s: head_dim must be even and <= 128 (got %d)", fn, D);
  if (!q || !k || !qw || !kw || !c || !sn || !rstd) return fail(MGA_ERR_INVALID, "%s: null pointer argument", fn);
  return MGA_OK;
}

}  // namespace

namespace {

int qk_rope_fwd(const char *fn, const void *q, int64_t q_ss, int64_t q_hs, const void *k, int64_t k_ss,
                int64_t k_hs, const void *v, int64_t v_ss, int64_t v_hs, const void *q_weight, const void *k_weight,
                const void *cos, const void *sin, int64_t cs_ss, float eps, const int32_t *rows, int32_t src_rows,
                int32_t S, int32_t Hq, int32_t Hkv, int32_t head_dim, int32_t dtype, void *q_out, int64_t qo_ss,
                int64_t qo_hs, void *k_out, int64_t ko_ss, int64_t ko_hs, void *v_out, int64_t vo_ss,
                int64_t vo_hs, float *rstd, void *stream) {
  if (!elem_bytes(dtype)) return fail(MGA_ERR_INVALID, "%s: unknown dtype code %d", fn, dtype);
  if (S <= 0 || Hkv <= 0 || (q && Hq <= 0)) return fail(MGA_ERR_INVALID, "%s: bad sizes (S=%d Hq=%d Hkv=%d)", fn, S, Hq, Hkv);
  if (head_dim <= 0 || head_dim > 128 || (head_dim & 1))
    return fail(MGA_ERR_INVALID, "%s: head_dim must be even and <= 128 (got %d)", fn, head_dim);
  if (!k || !k_weight || !cos || !sin || !k_out) return fail(MGA_ERR_INVALID, "%s: null pointer argument", fn);
  if (q && (!q_weight || !q_out)) return fail(MGA_ERR_INVALID, "%s: query without its weight or output", fn);
  if (!q && (q_out || rstd)) return fail(MGA_ERR_INVALID, "%s: query output or rstd without a query", fn);
  if ((v == nullptr) != (v_out == nullptr)) return fail(MGA_ERR_INVALID, "%s: value operand without its output", fn);
  if (rows && src_rows <= 0) return fail(MGA_ERR_INVALID, "%s: row gather needs src_rows > 0 (got %d)", fn, src_rows);
  mga::QkRopeArgs a = {};
  a.q = q; a.q_ss = q_ss; a.q_hs = q_hs;
  a.k = k; a.k_ss = k_ss; a.k_hs = k_hs;
  a.v = v; a.v_ss = v_ss; a.v_hs = v_hs;
  a.qw = q_weight; a.kw = k_weight; a.cos = cos; a.sin = sin; a.cs_ss = cs_ss;
  a.qo = q_out; a.qo_ss = qo_ss; a.qo_hs = qo_hs;
  a.ko = k_out; a.ko_ss = ko_ss; a.ko_hs = ko_hs;
  a.vo = v_out; a.vo_ss = vo_ss; a.vo_hs = vo_hs;
  a.rows = rows; a.src_rows = src_rows;
  a.rstd = rstd; a.eps = eps; a.S = S; a.Hq = q ? Hq : 0; a.Hkv = Hkv; a.D = head_dim;
  mga::launch_qk_norm_rope(a, dtype, false, (hipStream_t)stream);
  return check_launch(fn);
}

}  // namespace

int mga_qk_norm_rope_fwd(const void *q, int64_t q_ss, int64_t q_hs, const void *k, int64_t k_ss, int64_t k_hs,
                         const void *q_weight, const void *k_weight, const void *cos, const void *sin,
                         int64_t cs_ss, float eps, int32_t S, int32_t Hq, int32_t Hkv, int32_t head_dim,
                         int32_t dtype, void *q_out, int64_t qo_ss, int64_t qo_hs, void *k_out, int64_t ko_ss,
                         int64_t ko_hs, float *rstd, void *stream) {
  int rc = check_qk_rope("mga_qk_norm_rope_fwd", q, k, q_weight, k_weight, cos, sin, rstd, S, Hq, Hkv, head_dim, dtype);
  if (rc != MGA_OK) return rc;
  return qk_rope_fwd("mga_qk_norm_rope_fwd", q, q_ss, q_hs, k, k_ss, k_hs, nullptr, 0, 0, q_weight, k_weight, cos,
                     sin, cs_ss, eps, nullptr, 0, S, Hq, Hkv, head_dim, dtype, q_out, qo_ss, qo_hs, k_out, ko_ss,
                     ko_hs, nullptr, 0, 0, rstd, stream);
}

int mga_qk_norm_rope_stage_fwd(const void *q, int64_t q_ss, int64_t q_hs, const void *k, int64_t k_ss,
                               int64_t k_hs, const void *v, int64_t v_ss, int64_t v_hs, const void *q_weight,
                               const void *k_weight, const void *cos, const void *sin, int64_t cs_ss, float eps,
                               const int32_t *rows, int32_t src_rows, int32_t S, int32_t Hq, int32_t Hkv,
                               int32_t head_dim, int32_t dtype, void *q_out, int64_t qo_ss, int64_t qo_hs,
                               void *k_out, int64_t ko_ss, int64_t ko_hs, void *v_out, int64_t vo_ss,
                               int64_t vo_hs, float *rstd, void *stream) {
  if (!v || !v_out) return fail(MGA_ERR_INVALID, "mga_qk_norm_rope_stage_fwd: null value operand");
  return qk_rope_fwd("mga_qk_norm_rope_stage_fwd", q, q_ss, q_hs, k, k_ss, k_hs, v, v_ss, v_hs, q_weight, k_weight,
                     cos, sin, cs_ss, eps, rows, src_rows, S, Hq, Hkv, head_dim, dtype, q_out, qo_ss, qo_hs, k_out,
                     ko_ss, ko_hs, v_out, vo_ss, vo_hs, rstd, stream);
}

int mga_qk_norm_rope_bwd(const void *q, int64_t q_ss, int64_t q_hs, const void *k, int64_t k_ss, int64_t k_hs,
                         const void *q_weight, const void *k_weight, const void *cos, const void *sin,
                         int64_t cs_ss, const float *rstd, int32_t S, int32_t Hq, int32_t Hkv, int32_t head_dim,
                         int32_t dtype, const void *dq_out, int64_t dqo_ss, int64_t dqo_hs, const void *dk_out,
                         int64_t dko_ss, int64_t dko_hs, void *dq, int64_t dq_ss, int64_t dq_hs, void *dk,
                         int64_t dk_ss, int64_t dk_hs, void *stream) {
  int rc = check_qk_rope("mga_qk_norm_rope_bwd", q, k, q_weight, k_weight, cos, sin, rstd, S, Hq, Hkv, head_dim, dtype);
  if (rc != MGA_OK) return rc;
  if (!dq_out || !dk_out || !dq || !dk) return fail(MGA_ERR_INVALID, "mga_qk_norm_rope_bwd: null gradient pointer");
  mga::QkRopeArgs a = {};
  a.q = q; a.q_ss = q_ss; a.q_hs = q_hs;
  a.k = k; a.k_ss = k_ss; a.k_hs = k_hs;
  a.qw = q_weight; a.kw = k_weight; a.cos = cos; a.sin = sin; a.cs_ss = cs_ss;
  a.dqo = dq_out; a.dqo_ss = dqo_ss; a.dqo_hs = dqo_hs;
  a.dko = dk_out; a.dko_ss = dko_ss; a.dko_hs = dko_hs;
  a.dq = dq; a.dq_ss = dq_ss; a.dq_hs = dq_hs;
  a.dk = dk; a.dk_ss = dk_ss; a.dk_hs = dk_hs;
  a.rstd = const_cast<float *>(rstd); a.S = S; a.Hq = Hq; a.Hkv = Hkv; a.D = head_dim;
  mga::launch_qk_norm_rope(a, dtype, true, (hipStream_t)stream);
  return check_launch("mga_qk_norm_rope_bwd");
}

namespace {

constexpr int64_t kBlasWorkspace = int64_t(32) << 20;   // hipBLASLt workspace per call

int64_t align256(int64_t b) { return (b + 255) & ~int64_t(255); }
int64_t lora_rpad(int32_t rank) { return (rank + 31) / 32 * 32; }

struct LoraWs {
  void *blas, *u, *da, *at;
  float *part;
  void *packed;
  float *dapart;
  float *skpart;
};

// [hipBLASLt workspace | u = dY B : S x rpad | d_a : S x rpad | A^T : K x rpad
//  (bf16) | split-K partial sums of the down-projection: 8 x S x 96 fp32 |
//  lora_A in MFMA-operand order, up to 96 ranks at a time: K / 16 x 3 KB |
//  split partial sums of grad_A: 16 x rpad x K fp32 | split partial sums of
//  lora_B's backward products: 8 x max(S, N) x rpad fp32]
int64_t lora_ws_bytes(int32_t S, int32_t K, int32_t N, int32_t rank) {
  const int64_t rp = lora_rpad(rank);
  return kBlasWorkspace + 2 * align256((int64_t)S * rp * 4) + align256((int64_t)K * rp * 2) +
         align256((int64_t)8 * S * 96 * 4) + align256((int64_t)K / 16 * 3 * 1024) +
         align256((int64_t)mga::kDaMaxSplit * rp * K * 4) +
         align256((int64_t)mga::kSkinnyMaxSplit * std::max(S, N) * rp * 4);
}

LoraWs lora_ws(void *ws, int32_t S, int32_t K, int32_t rank) {
  const int64_t rp = lora_rpad(rank);
  char *p = static_cast<char *>(ws);
  LoraWs w;
  w.blas = p;
  w.u = p + kBlasWorkspace;
  w.da = static_cast<char *>(w.u) + align256((int64_t)S * rp * 4);
  w.at = static_cast<char *>(w.da) + align256((int64_t)S * rp * 4);
  w.part = reinterpret_cast<float *>(static_cast<char *>(w.at) + align256((int64_t)K * rp * 2));
  w.packed = reinterpret_cast<char *>(w.part) + align256((int64_t)8 * S * 96 * 4);
  w.dapart = reinterpret_cast<float *>(static_cast<char *>(w.packed) + align256((int64_t)K / 16 * 3 * 1024));
  w.skpart = reinterpret_cast<float *>(reinterpret_cast<char *>(w.dapart) +
                                       align256((int64_t)mga::kDaMaxSplit * rp * K * 4));
  return w;
}

int check_lora_sizes(const char *fn, int32_t S, int32_t K, int32_t N, int32_t rank, double p) {
  if (S <= 0 || N <= 0 || K <= 0) return fail(MGA_ERR_INVALID, "%s: bad sizes (S=%d K=%d N=%d)", fn, S, K, N);
  if (K % 16) return fail(MGA_ERR_INVALID, "%s: in_features must be a multiple of 16 (got %d)", fn, K);
  if (rank < 1) return fail(MGA_ERR_INVALID, "%s: rank must be positive (got %d)", fn, rank);
  if (!(p >= 0.0 && p < 1.0)) return fail(MGA_ERR_INVALID, "%s: dropout probability %g not in [0, 1)", fn, p);
  return MGA_OK;
}

// A bf16 matrix read with 16-byte vectors along its rows.
int check_vec_rows(const char *fn, const char *name, const void *ptr, int64_t rs, int64_t cols) {
  if (!ptr) return fail(MGA_ERR_INVALID, "%s: %s is null", fn, name);
  if (!aligned16(ptr)) return fail(MGA_ERR_INVALID, "%s: %s is not 16-byte aligned", fn, name);
  if (rs < cols || rs % 8) return fail(MGA_ERR_INVALID, "%s: %s row stride %lld must be >= %lld and a multiple of 8",
                                       fn, name, (long long)rs, (long long)cols);
  return MGA_OK;
}

int check_rows_ld(const char *fn, const char *name, const void *ptr, int64_t rs, int64_t cols) {
  if (!ptr) return fail(MGA_ERR_INVALID, "%s: %s is null", fn, name);
  if (rs < cols) return fail(MGA_ERR_INVALID, "%s: %s row stride %lld < %lld", fn, name, (long long)rs,
                             (long long)cols);
  return MGA_OK;
}

uint32_t drop_threshold(double p) { return (uint32_t)llround(p * 65536.0); }
float keep_scale(double p) { return (float)(1.0 / (1.0 - p)); }

int blas(const char *fn, bool ta, bool tb, int64_t M, int64_t N, int64_t K, const void *A, int64_t lda, const void *B,
         int64_t ldb, bool acc, void *D, int64_t ldd, const LoraWs &w, hipStream_t st, int dtype = MGA_DTYPE_BF16) {
  const char *err = nullptr;
  if (mga::gemm(dtype, ta, tb, M, N, K, A, lda, B, ldb, acc, D, ldd, w.blas, (size_t)kBlasWorkspace, st, &err))
    return fail(MGA_ERR_HIP, "%s: hipBLASLt GEMM (%lld x %lld x %lld): %s", fn, (long long)M, (long long)N,
                (long long)K, err ? err : "error");
  return MGA_OK;
}

// fp16 / fp32 operands: hipBLASLt GEMMs in the operand type and the
// elementwise kernels of the general path; the dropout output h is always
// written (the backward's grad_A reads it).
int gated_lora_fwd_general(const char *fn, int dtype, const void *x, int64_t x_rs, const void *weight, int64_t w_rs,
                           const void *lora_a, int64_t a_rs, const void *lora_b, int64_t b_rs, const float *gate,
                           float scaling, double dropout_p, uint64_t seed, int32_t S, int32_t K, int32_t N,
                           int32_t rank, void *y, int64_t y_rs, void *t, int64_t t_rs, void *h, int64_t h_rs,
                           const LoraWs &w, hipStream_t st) {
  int rc;
  const uint32_t thr = drop_threshold(dropout_p);
  if (thr && (rc = check_rows_ld(fn, "dropout output h", h, h_rs, K))) return rc;
  const void *src = x;
  int64_t src_rs = x_rs;
  if (thr) {   // h = dropout(x)
    mga::launch_lora_gen_dropout(dtype, x, x_rs, S, K, thr, keep_scale(dropout_p), seed, h, h_rs, st);
    if ((rc = check_launch(fn)) != MGA_OK) return rc;
    src = h;
    src_rs = h_rs;
  }
  // t = T(T(s T(h A^T)) gate)
  if ((rc = blas(fn, false, true, S, rank, K, src, src_rs, lora_a, a_rs, false, t, t_rs, w, st, dtype))) return rc;
  mga::launch_lora_gen_scale_rows(dtype, t, t_rs, gate, scaling, false, S, rank, (int32_t)lora_rpad(rank), t, t_rs,
                                  st);
  if ((rc = check_launch(fn)) != MGA_OK) return rc;
  // y = T(x W^T + T(t B^T))
  if ((rc = blas(fn, false, true, S, N, rank, t, t_rs, lora_b, b_rs, false, y, y_rs, w, st, dtype))) return rc;
  return blas(fn, false, true, S, N, K, x, x_rs, weight, w_rs, true, y, y_rs, w, st, dtype);
}

int gated_lora_bwd_general(const char *fn, int dtype, const void *grad_y, int64_t gy_rs, const void *x, int64_t x_rs,
                           const void *h, int64_t h_rs, const void *weight, int64_t w_rs, const void *lora_a,
                           int64_t a_rs, const void *lora_b, int64_t b_rs, const void *t, int64_t t_rs,
                           const float *gate, float scaling, double dropout_p, uint64_t seed, int32_t S, int32_t K,
                           int32_t N, int32_t rank, void *grad_x, int64_t gx_rs, void *grad_a, int64_t ga_rs,
                           void *grad_b, int64_t gb_rs, const LoraWs &w, hipStream_t st) {
  int rc;
  const uint32_t thr = drop_threshold(dropout_p);
  const int64_t rp = lora_rpad(rank);
  if (grad_a && thr && !h)
    return fail(MGA_ERR_INVALID, "%s: the dropout output h of the forward is needed for grad_A with fp16 / fp32", fn);
  // d_a = T(T(T(dY B) gate) s)
  if ((rc = blas(fn, false, false, S, rank, N, grad_y, gy_rs, lora_b, b_rs, false, w.u, rp, w, st, dtype))) return rc;
  mga::launch_lora_gen_scale_rows(dtype, w.u, rp, gate, scaling, true, S, rank, (int32_t)rp, w.da, rp, st);
  if ((rc = check_launch(fn)) != MGA_OK) return rc;
  // dB = dY^T t
  if (grad_b && (rc = blas(fn, true, false, N, rank, S, grad_y, gy_rs, t, t_rs, false, grad_b, gb_rs, w, st, dtype)))
    return rc;
  if (grad_x) {
    // dX = T(dY W + T(mask T(d_a A) / (1 - p)))
    if ((rc = blas(fn, false, false, S, K, rank, w.da, rp, lora_a, a_rs, false, grad_x, gx_rs, w, st, dtype)))
      return rc;
    if (thr) {
      mga::launch_lora_gen_dx_mask(dtype, grad_x, gx_rs, S, K, thr, keep_scale(dropout_p), seed, st);
      if ((rc = check_launch(fn)) != MGA_OK) return rc;
    }
    if ((rc = blas(fn, false, false, S, K, N, grad_y, gy_rs, weight, w_rs, true, grad_x, gx_rs, w, st, dtype)))
      return rc;
  }
  // dA = d_a^T dropout(x)
  if (grad_a && (rc = blas(fn, true, false, rank, K, S, w.da, rp, thr ? h : x, thr ? h_rs : x_rs, false, grad_a,
                           ga_rs, w, st, dtype)))
    return rc;
  return MGA_OK;
}

}  // namespace

int64_t mga_gated_lora_workspace_bytes(int32_t S, int32_t K, int32_t N, int32_t rank) {
  (void)N;
  if (S <= 0 || K <= 0 || rank <= 0) return 0;
  return lora_ws_bytes(S, K, N, rank);
}

int mga_gated_lora_fwd(const void *x, int64_t x_rs, const void *weight, int64_t w_rs, const void *lora_a,
                       int64_t a_rs, const void *lora_b, int64_t b_rs, const float *gate, float scaling,
                       double dropout_p, uint64_t seed, int32_t S, int32_t K, int32_t N, int32_t rank, void *y,
                       int64_t y_rs, void *t, int64_t t_rs, void *h, int64_t h_rs, void *workspace,
                       int64_t workspace_bytes, int32_t dtype, void *stream) {
  const char *fn = "mga_gated_lora_fwd";
  int rc;
  if ((rc = check_lora_sizes(fn, S, K, N, rank, dropout_p)) != MGA_OK) return rc;
  if (!elem_bytes(dtype)) return fail(MGA_ERR_INVALID, "%s: unknown dtype code %d", fn, dtype);
  if (dtype != MGA_DTYPE_BF16) {
    const int64_t rp = lora_rpad(rank);
    if ((rc = check_rows_ld(fn, "x", x, x_rs, K)) || (rc = check_rows_ld(fn, "weight", weight, w_rs, K)) ||
        (rc = check_rows_ld(fn, "lora_A", lora_a, a_rs, K)) || (rc = check_rows_ld(fn, "lora_B", lora_b, b_rs, rank)) ||
        (rc = check_rows_ld(fn, "output", y, y_rs, N)) || (rc = check_rows_ld(fn, "t", t, t_rs, rp)))
      return rc;
    if (!workspace || workspace_bytes < lora_ws_bytes(S, K, N, rank))
      return fail(MGA_ERR_INVALID, "%s: workspace of %lld bytes needed", fn, (long long)lora_ws_bytes(S, K, N, rank));
    return gated_lora_fwd_general(fn, dtype, x, x_rs, weight, w_rs, lora_a, a_rs, lora_b, b_rs, gate, scaling,
                                  dropout_p, seed, S, K, N, rank, y, y_rs, t, t_rs, h, h_rs,
                                  lora_ws(workspace, S, K, rank), (hipStream_t)stream);
  }
  const uint32_t thr = drop_threshold(dropout_p);
  const int64_t rp = lora_rpad(rank);
  if ((rc = check_vec_rows(fn, "x", x, x_rs, K)) != MGA_OK || (rc = check_rows_ld(fn, "weight", weight, w_rs, K)) ||
      (rc = check_vec_rows(fn, "lora_A", lora_a, a_rs, K)) || (rc = check_rows_ld(fn, "lora_B", lora_b, b_rs, rank)) ||
      (rc = check_rows_ld(fn, "output", y, y_rs, N)) || (rc = check_rows_ld(fn, "t", t, t_rs, rp)))
    return rc;
  if (thr > 0 && h && (rc = check_vec_rows(fn, "dropout output h", h, h_rs, K)) != MGA_OK) return rc;
  if (!workspace || workspace_bytes < lora_ws_bytes(S, K, N, rank))
    return fail(MGA_ERR_INVALID, "%s: workspace of %lld bytes needed", fn, (long long)lora_ws_bytes(S, K, N, rank));
  const LoraWs w = lora_ws(workspace, S, K, rank);
  hipStream_t st = (hipStream_t)stream;
  // t = T(T(s T(dropout(x) A^T)) gate)
  mga::LoraDownArgs a = {};
  a.x = x; a.x_rs = x_rs; a.A = lora_a; a.a_rs = a_rs; a.gate = gate; a.scaling = scaling;
  a.keep_scale = keep_scale(dropout_p); a.thr = thr; a.seed = seed; a.h = thr && h ? h : nullptr; a.h_rs = h_rs;
  a.t = t; a.t_rs = t_rs; a.part = w.part; a.packed = w.packed; a.S = S; a.K = K; a.rank = rank;
  mga::launch_lora_down(a, st);
  if ((rc = check_launch(fn)) != MGA_OK) return rc;
  // y = T(t B^T), then y = T(x W^T + y): the base GEMM reads the LoRA term in
  // its epilogue (free in a compute-bound GEMM) instead of a second pass over y
  if ((rc = blas(fn, false, true, S, N, rank, t, t_rs, lora_b, b_rs, false, y, y_rs, w, st)) != MGA_OK) return rc;
  if ((rc = blas(fn, false, true, S, N, K, x, x_rs, weight, w_rs, true, y, y_rs, w, st)) != MGA_OK) return rc;
  return MGA_OK;
}

int mga_gated_lora_bwd(const void *grad_y, int64_t gy_rs, const void *x, int64_t x_rs, const void *h, int64_t h_rs,
                       const void *weight, int64_t w_rs, const void *lora_a, int64_t a_rs, const void *lora_b,
                       int64_t b_rs, const void *t, int64_t t_rs, const float *gate, float scaling, double dropout_p,
                       uint64_t seed, int32_t S, int32_t K, int32_t N, int32_t rank, void *grad_x, int64_t gx_rs,
                       void *grad_a, int64_t ga_rs, void *grad_b, int64_t gb_rs, void *workspace,
                       int64_t workspace_bytes, int32_t dtype, void *stream) {
  const char *fn = "mga_gated_lora_bwd";
  int rc;
  if ((rc = check_lora_sizes(fn, S, K, N, rank, dropout_p)) != MGA_OK) return rc;
  if (!elem_bytes(dtype)) return fail(MGA_ERR_INVALID, "%s: unknown dtype code %d", fn, dtype);
  if (dtype != MGA_DTYPE_BF16) {
    const int64_t rp = lora_rpad(rank);
    const bool thr = drop_threshold(dropout_p) != 0;
    if ((rc = check_rows_ld(fn, "grad_output", grad_y, gy_rs, N)) ||
        (rc = check_rows_ld(fn, "lora_B", lora_b, b_rs, rank)) || (rc = check_rows_ld(fn, "t", t, t_rs, rp)))
      return rc;
    if (grad_x && ((rc = check_rows_ld(fn, "weight", weight, w_rs, K)) ||
                   (rc = check_rows_ld(fn, "lora_A", lora_a, a_rs, K)) ||
                   (rc = check_rows_ld(fn, "grad_x", grad_x, gx_rs, K))))
      return rc;
    if (grad_a && ((rc = check_rows_ld(fn, "grad_A", grad_a, ga_rs, K)) ||
                   (!thr && (rc = check_rows_ld(fn, "x", x, x_rs, K)))))
      return rc;
    if (grad_b && (rc = check_rows_ld(fn, "grad_B", grad_b, gb_rs, rank))) return rc;
    if (!workspace || workspace_bytes < lora_ws_bytes(S, K, N, rank))
      return fail(MGA_ERR_INVALID, "%s: workspace of %lld bytes needed", fn, (long long)lora_ws_bytes(S, K, N, rank));
    return gated_lora_bwd_general(fn, dtype, grad_y, gy_rs, x, x_rs, h, h_rs, weight, w_rs, lora_a, a_rs, lora_b, b_rs,
                                  t, t_rs, gate, scaling, dropout_p, seed, S, K, N, rank, grad_x, gx_rs, grad_a,
                                  ga_rs, grad_b, gb_rs, lora_ws(workspace, S, K, rank), (hipStream_t)stream);
  }
  const uint32_t thr = drop_threshold(dropout_p);
  const int64_t rp = lora_rpad(rank);
  if ((rc = check_rows_ld(fn, "grad_output", grad_y, gy_rs, N)) ||
      (rc = check_rows_ld(fn, "lora_B", lora_b, b_rs, rank)) || (rc = check_rows_ld(fn, "t", t, t_rs, rp)))
    return rc;
  if (grad_x && ((rc = check_rows_ld(fn, "weight", weight, w_rs, K)) ||
                 (rc = check_rows_ld(fn, "lora_A", lora_a, a_rs, K)) ||
                 (rc = check_rows_ld(fn, "grad_x", grad_x, gx_rs, K))))
    return rc;
  if (grad_x && thr && (!aligned16(grad_x) || gx_rs % 4))
    return fail(MGA_ERR_INVALID, "%s: grad_x must be 16-byte aligned with a row stride multiple of 4", fn);
  // with dropout and no saved dropout output, grad_A draws the mask again from x
  const bool da_from_x = grad_a && thr && !h;
  if (grad_a && (rc = check_rows_ld(fn, "grad_A", grad_a, ga_rs, K))) return rc;
  if (da_from_x) {
    if (K % 128)
      return fail(MGA_ERR_INVALID, "%s: the dropout output h is needed when in_features (%d) is not a multiple of 128",
                  fn, K);
    if ((rc = check_vec_rows(fn, "x", x, x_rs, K))) return rc;
  } else if (grad_a && (rc = check_rows_ld(fn, thr ? "dropout output h" : "x", thr ? h : x, thr ? h_rs : x_rs, K))) {
    return rc;
  }
  if (grad_b && (rc = check_rows_ld(fn, "grad_B", grad_b, gb_rs, rank))) return rc;
  if (!workspace || workspace_bytes < lora_ws_bytes(S, K, N, rank))
    return fail(MGA_ERR_INVALID, "%s: workspace of %lld bytes needed", fn, (long long)lora_ws_bytes(S, K, N, rank));
  const LoraWs w = lora_ws(workspace, S, K, rank);
  hipStream_t st = (hipStream_t)stream;
  // u = dY B, d_a = T(T(T(u) gate) s) (the gradient at lora_A's output), and
  // dB = dY^T t: one streaming pass over dY each (ranks up to 128, 16-byte
  // rows), else hipBLASLt
  const bool skinny = rank <= 128 && N % 8 == 0 && aligned16(grad_y) && gy_rs % 8 == 0 && aligned16(lora_b) &&
                      b_rs % 8 == 0 && aligned16(t) && t_rs % 8 == 0;
  mga::LoraSkinnyArgs sk = {};
  sk.dy = grad_y; sk.dy_rs = gy_rs; sk.part = w.skpart; sk.S = S; sk.N = N; sk.rank = rank; sk.rp = (int32_t)rp;
  if (skinny) {
    sk.sm = lora_b; sk.sm_rs = b_rs;
    mga::launch_lora_grad_u(sk, gate, scaling, w.da, rp, st);
    if ((rc = check_launch(fn)) != MGA_OK) return rc;
  } else {
    if ((rc = blas(fn, false, false, S, rank, N, grad_y, gy_rs, lora_b, b_rs, false, w.u, rp, w, st)) != MGA_OK)
      return rc;
    mga::launch_lora_scale_rows(w.u, rp, gate, scaling, S, rank, (int32_t)rp, w.da, rp, st);
    if ((rc = check_launch(fn)) != MGA_OK) return rc;
  }
  if (grad_b && skinny) {
    sk.sm = t; sk.sm_rs = t_rs;
    mga::launch_lora_grad_b(sk, grad_b, gb_rs, st);
    if ((rc = check_launch(fn)) != MGA_OK) return rc;
  } else if (grad_b && (rc = blas(fn, true, false, N, rank, S, grad_y, gy_rs, t, t_rs, false, grad_b, gb_rs, w, st))) {
    return rc;
  }
  if (grad_x) {
    // the LoRA path's gradient first (through dropout when it is on), then
    // dX = T(dY W + that): the base GEMM accumulates onto it in its epilogue
    if (thr) {
      mga::launch_lora_transpose(lora_a, a_rs, rank, K, (int32_t)rp, w.at, rp, st);
      mga::LoraDxArgs d = {};
      d.da = w.da; d.da_rs = rp; d.At = w.at; d.at_rs = rp; d.dx = grad_x; d.dx_rs = gx_rs;
      d.keep_scale = keep_scale(dropout_p); d.thr = thr; d.seed = seed; d.S = S; d.K = K; d.rank = rank;
      mga::launch_lora_dx(d, st);
      if ((rc = check_launch(fn)) != MGA_OK) return rc;
    } else if ((rc = blas(fn, false, false, S, K, rank, w.da, rp, lora_a, a_rs, false, grad_x, gx_rs, w, st))) {
      return rc;
    }
    if ((rc = blas(fn, false, false, S, K, N, grad_y, gy_rs, weight, w_rs, true, grad_x, gx_rs, w, st)) != MGA_OK)
      return rc;
  }
  // dA = d_a^T dropout(x)
  if (da_from_x) {
    mga::LoraDaArgs d = {};
    d.x = x; d.x_rs = x_rs; d.da = w.da; d.da_rs = rp; d.dA = grad_a; d.dA_rs = ga_rs; d.part = w.dapart;
    d.keep_scale = keep_scale(dropout_p); d.thr = thr; d.seed = seed; d.S = S; d.K = K; d.rank = rank;
    mga::launch_lora_da(d, st);
    if ((rc = check_launch(fn)) != MGA_OK) return rc;
  } else if (grad_a && (rc = blas(fn, true, false, rank, K, S, w.da, rp, thr ? h : x, thr ? h_rs : x_rs, false,
                                  grad_a, ga_rs, w, st))) {
    return rc;
  }
  return MGA_OK;
}

int64_t mga_soft_ce_workspace_floats(int32_t n_rows, int32_t n_cols) {
  if (n_rows <= 0 || n_cols <= 0) return 0;
  return mga::soft_ce_workspace_floats(n_rows, n_cols);
}

namespace {

// rows of a [n_rows, n_cols] operand; true in *vec when 16-byte vector loads apply
int check_rows(const char *fn, const char *name, const void *p, int64_t rs, int32_t n_cols, int eb, bool *vec) {
  if (!p) return fail(MGA_ERR_INVALID, "%s: %s is null", fn, name);
  if (rs < n_cols) return fail(MGA_ERR_INVALID, "%s: %s row stride %lld < n_cols %d", fn, name, (long long)rs, n_cols);
  *vec = *vec && aligned16(p) && ((rs * eb) & 15) == 0;
  return MGA_OK;
}

int check_soft_ce(const char *fn, const void *x, int64_t xs, const void *t, int64_t ts, int32_t n_rows,
                  int32_t n_cols, int32_t dtype, bool *vec) {
  const int eb = elem_bytes(dtype);
  if (!eb) return fail(MGA_ERR_INVALID, "%s: unknown dtype code %d", fn, dtype);
  if (n_rows <= 0 || n_cols <= 0) return fail(MGA_ERR_INVALID, "%s: bad sizes (rows=%d cols=%d)", fn, n_rows, n_cols);
  int rc = check_rows(fn, "student", x, xs, n_cols, eb, vec);
  if (rc == MGA_OK) rc = check_rows(fn, "teacher", t, ts, n_cols, eb, vec);
  return rc;
}

}  // namespace

int mga_soft_ce_fwd(const void *student, int64_t student_row_stride, const void *teacher,
                    int64_t teacher_row_stride, int32_t n_rows, int32_t n_cols, int32_t dtype, float *row_loss,
                    float *stats, float *workspace, void *stream) {
  bool vec = true;
  int rc = check_soft_ce("mga_soft_ce_fwd", student, student_row_stride, teacher, teacher_row_stride, n_rows, n_cols,
                         dtype, &vec);
  if (rc != MGA_OK) return rc;
  if (!row_loss || !stats || !workspace) return fail(MGA_ERR_INVALID, "mga_soft_ce_fwd: null output or workspace");
  mga::launch_soft_ce_fwd(student, student_row_stride, teacher, teacher_row_stride, n_rows, n_cols,
                          dtype, vec, row_loss, stats, workspace, (hipStream_t)stream);
  return check_launch("mga_soft_ce_fwd");
}

int mga_soft_ce_bwd(const void *student, int64_t student_row_stride, const void *teacher,
                    int64_t teacher_row_stride, int32_t n_rows, int32_t n_cols, int32_t dtype,
                    const float *grad_output, const float *stats, void *grad, int64_t grad_row_stride, void *stream) {
  bool vec = true;
  int rc = check_soft_ce("mga_soft_ce_bwd", student, student_row_stride, teacher, teacher_row_stride, n_rows, n_cols,
                         dtype, &vec);
  if (rc == MGA_OK) rc = check_rows("mga_soft_ce_bwd", "grad", grad, grad_row_stride, n_cols, elem_bytes(dtype), &vec);
  if (rc != MGA_OK) return rc;
  if (!grad_output || !stats) return fail(MGA_ERR_INVALID, "mga_soft_ce_bwd: null grad_output or stats");
  mga::launch_soft_ce_bwd(student, student_row_stride, teacher, teacher_row_stride, n_rows, n_cols,
                          dtype, vec, grad_output, stats, grad, grad_row_stride, (hipStream_t)stream);
  return check_launch("mga_soft_ce_bwd");
}

}  // extern "C"
