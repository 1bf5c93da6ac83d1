// Host-side launchers shared between the kernel files and the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mga {

struct AttnArgs {
  const void *q; int64_t q_sh, q_ss;
  const void *k; int64_t k_sh, k_ss;
  const void *v; int64_t v_sh, v_ss;
  const void *o; int64_t o_sh, o_ss;      // fwd: output; bwd: saved output
  const void *dout; int64_t do_sh, do_ss;
  float *lse;                               // [Hq, S] natural log
  float *delta;                             // [Hq, S] workspace (bwd)
  void *dq; int64_t dq_sh, dq_ss;
  void *dk; int64_t dk_sh, dk_ss;
  void *dv; int64_t dv_sh, dv_ss;
  int32_t grad_start;
  const int32_t *code;
  const int32_t *kv_num, *kv_idx, *fkv_num, *fkv_idx;
  const int32_t *q_num, *q_idx, *fq_num, *fq_idx;
  int32_t S, L, P, Hq, Hkv, nQ, nKV;
  float scale, scale_log2;
};

void launch_kv_copy_rows(const void *src_k, const void *src_v, int64_t src_sh_b, int64_t src_ss_b,
                         int64_t src_rows, const int32_t *idx, int32_t n_rows, void *dst_k, void *dst_v,
                         int64_t dst_sh_b, int64_t dst_ss_b, int64_t dst_off, int32_t n_heads,
                         int32_t row_bytes, hipStream_t stream);

void launch_regular_index(const int64_t *mask, int64_t stride, int32_t n, int32_t *idx,
                          int32_t *count, hipStream_t stream);

void launch_mtp_block_mask(const int64_t *gate, int64_t gate_stride, int32_t S, int64_t P,
                           int32_t *code, int8_t *cls, int32_t *kv_num, int32_t *kv_idx,
                           int32_t *full_kv_num, int32_t *full_kv_idx, int32_t *q_num,
                           int32_t *q_idx, int32_t *full_q_num, int32_t *full_q_idx,
                           hipStream_t stream);

// Element types of the operands (the C ABI's MGA_DTYPE_* codes).
constexpr int kDtBf16 = 0;
constexpr int kDtF32 = 1;
constexpr int kDtF16 = 2;

// head_dim in {64, 128}; dtype one of kDt*.
void launch_attn_fwd(const AttnArgs &a, int head_dim, int dtype, hipStream_t stream);
// passes: kBwdDq (delta + dQ) and/or kBwdDkDv (dK/dV; reads the delta the dQ pass wrote).
constexpr int kBwdDq = 1;
constexpr int kBwdDkDv = 2;
void launch_attn_bwd(const AttnArgs &a, int head_dim, int dtype, int passes, hipStream_t stream);
// fp32 operands (mga_attn_f32.hip): fp32 MFMAs throughout; same contract.
void launch_attn_fwd_f32(const AttnArgs &a, int head_dim, hipStream_t stream);
void launch_attn_bwd_f32(const AttnArgs &a, int head_dim, int passes, hipStream_t stream);

// Fused Qwen3 q/k RMSNorm + rotary embedding (mga_qk_rope.hip). Operands are
// [S, heads, D] addressed with (token stride, head stride) in elements; cos
// and sin [S, D] with token stride cs_ss; rstd [S, Hq + Hkv] (token-major).
struct QkRopeArgs {
  const void *q; int64_t q_ss, q_hs;
  const void *k; int64_t k_ss, k_hs;
  const void *qw, *kw, *cos, *sin; int64_t cs_ss;
  void *qo; int64_t qo_ss, qo_hs;     // forward outputs
  void *ko; int64_t ko_ss, ko_hs;
  const void *v; int64_t v_ss, v_hs;  // forward, optional: value rows copied to vo unchanged
  void *vo; int64_t vo_ss, vo_hs;
  const int32_t *rows;                // forward, optional: output row s reads input row rows[s]
  int32_t src_rows;                   //   (and cos / sin row rows[s]); rows outside [0, src_rows) are skipped
  const void *dqo; int64_t dqo_ss, dqo_hs;   // backward: gradients of the outputs
  const void *dko; int64_t dko_ss, dko_hs;
  void *dq; int64_t dq_ss, dq_hs;     // backward outputs
  void *dk; int64_t dk_ss, dk_hs;
  float *rstd;                        // forward: may be null (nothing saved)
  float eps;
  int32_t S, Hq, Hkv, D;              // forward with q null: key (and value) rows only
};
void launch_qk_norm_rope(const QkRopeArgs &a, int dtype, bool backward, hipStream_t stream);

// Plain GEMM through hipBLASLt, row-major (mga_blas.hip), operands and
// output of one element type (kDt*), fp32 compute:
// D[M, N] = op(A)[M, K] op(B)[K, N] (+ D), op(A) = A^T when ta (A stored
// [K, M]), op(B) = B^T when tb (B stored [N, K]). Returns 0, or -1 with *err set.
int gemm(int dtype, bool ta, bool tb, int64_t M, int64_t N, int64_t K, const void *A, int64_t lda, const void *B,
         int64_t ldb, bool accumulate, void *D, int64_t ldd, void *workspace, size_t ws_bytes, hipStream_t stream,
         const char **err);
int gemm_bf16(bool ta, bool tb, int64_t M, int64_t N, int64_t K, const void *A, int64_t lda, const void *B,
              int64_t ldb, bool accumulate, void *D, int64_t ldd, void *workspace, size_t ws_bytes,
              hipStream_t stream, const char **err);

// Gated LoRA kernels (mga_lora.hip).
struct LoraDownArgs {
  const void *x; int64_t x_rs;         // [S, K] bf16
  const void *A; int64_t a_rs;         // lora_A weight [rank, K]
  const float *gate;                   // [S] or null (= 1)
  float scaling, keep_scale;           // alpha / rank; 1 / (1 - p)
  uint32_t thr;                        // 16-bit drop threshold, 0 = no dropout
  uint64_t seed;
  void *h; int64_t h_rs;               // dropout output [S, K] (thr > 0)
  void *t; int64_t t_rs;               // [S, rpad] bf16 out
  float *part;                         // split-K partial sums: 8 x S x 96 fp32, or null (no split)
  void *packed;                        // lora_A in MFMA-operand order: K / 16 x 3 blocks of 1 KB
  int32_t S, K, rank;
};
struct LoraDxArgs {
  const void *da; int64_t da_rs;       // [S, rpad] bf16
  const void *At; int64_t at_rs;       // [K, rpad] bf16
  void *dx; int64_t dx_rs;             // [S, K] bf16, updated in place
  float keep_scale;
  uint32_t thr;
  uint64_t seed;
  int32_t S, K, rank;
};
struct LoraDaArgs {
  const void *x; int64_t x_rs;         // [S, K] bf16, the layer input
  const void *da; int64_t da_rs;       // [S, rpad] bf16 gradient at lora_A's output (zero past the rank)
  void *dA; int64_t dA_rs;             // [rank, K] bf16 out
  float *part;                         // split partial sums [nsplit, 32 ceil(rank / 32), K] fp32
  float keep_scale;
  uint32_t thr;                        // 16-bit drop threshold (> 0)
  uint64_t seed;
  int32_t S, K, rank;
};
constexpr int kDaMaxSplit = 16;
// lora_B's backward products over the streamed dY (mga_lora.hip): dB = dY^T t
// (small = t [S, >= rank]) and u = dY B (small = lora_B [N, rank]); rank <= 128,
// rows 16-byte aligned with strides a multiple of 8, N a multiple of 8.
struct LoraSkinnyArgs {
  const void *dy; int64_t dy_rs;       // [S, N] bf16
  const void *sm; int64_t sm_rs;       // t or lora_B
  float *part;                         // split partial sums [nsplit, lines, rp] fp32
  int32_t S, N, rank, rp;
};
constexpr int kSkinnyMaxSplit = 8;
void launch_lora_grad_b(const LoraSkinnyArgs &a, void *db, int64_t db_rs, hipStream_t stream);
void launch_lora_grad_u(const LoraSkinnyArgs &a, const float *gate, float scaling, void *da, int64_t da_rs,
                        hipStream_t stream);
void launch_lora_down(const LoraDownArgs &a, hipStream_t stream);
void launch_lora_da(const LoraDaArgs &a, hipStream_t stream);
void launch_lora_dx(const LoraDxArgs &a, hipStream_t stream);
void launch_lora_scale_rows(const void *u, int64_t u_rs, const float *gate, float scaling, int32_t S,
                            int32_t rank, int32_t rpad, void *da, int64_t da_rs, hipStream_t stream);
void launch_lora_transpose(const void *A, int64_t a_rs, int32_t rank, int32_t K, int32_t rpad, void *At,
                           int64_t at_rs, hipStream_t stream);
// The general path (fp16 and fp32 operands, dtype kDtF16 / kDtF32): the
// elementwise steps around its hipBLASLt GEMMs, with the bf16 path's dropout
// bits (element pair j of the flattened [S, K] input, same hash and seed).
// h = T(x / (1 - p)) where kept, else 0.
void launch_lora_gen_dropout(int dtype, const void *x, int64_t x_rs, int32_t S, int32_t K, uint32_t thr,
                             float keep_scale, uint64_t seed, void *h, int64_t h_rs, hipStream_t stream);
// out = T(T(u * gate) * scaling) (gate_first) or T(T(u * scaling) * gate), rows
// of rank entries then zeros up to rpad (may be in place).
void launch_lora_gen_scale_rows(int dtype, const void *u, int64_t u_rs, const float *gate, float scaling, bool gate_first,
                                int32_t S, int32_t rank, int32_t rpad, void *out, int64_t out_rs, hipStream_t stream);
// dx = T(dx / (1 - p)) where kept, else 0 (in place).
void launch_lora_gen_dx_mask(int dtype, void *dx, int64_t dx_rs, int32_t S, int32_t K, uint32_t thr, float keep_scale,
                             uint64_t seed, hipStream_t stream);

// Stable soft cross-entropy (mga_soft_ce.hip). Rows of V columns; row strides
// in elements; vec: 16-byte vector loads (every row start 16-byte aligned).
int64_t soft_ce_workspace_floats(int32_t n_rows, int32_t n_cols);
void launch_soft_ce_fwd(const void *x, int64_t xs, const void *t, int64_t ts, int32_t N, int32_t V, int dtype,
                        bool vec, float *loss, float *stats, float *ws, hipStream_t stream);
void launch_soft_ce_bwd(const void *x, int64_t xs, const void *t, int64_t ts, int32_t N, int32_t V, int dtype,
                        bool vec, const float *grad_out, const float *stats, void *g, int64_t gs,
                        hipStream_t stream);

// Compute units of the current device (queried once per device).
int device_cu_count();

}  // namespace mga
