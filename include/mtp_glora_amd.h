/*
 * mtp_glora_amd.h - C ABI of the MI355X (gfx950) streaming-KV-cache and
 * MTP block-masked attention library (libmtp_glora_amd.so).
 *
 * Every entry point takes plain device pointers, element strides and sizes,
 * enqueues its kernels on `stream` (a hipStream_t, NULL = default stream) and
 * returns MGA_OK or an error code; mga_last_error() gives the message of the
 * last failure on the calling thread. Nothing here allocates device memory:
 * callers own every buffer (outputs and workspaces included); the one device
 * array the library holds itself is the fixed workspace of
 * mga_attn_bwd_noalloc, created with the library's code object.
 *
 * Layout conventions (batch size 1, as the reference assumes everywhere,
 * mtp_glora/data_utils/collator.py:123-124, 242-243, 308-309):
 *   - a [heads, seq, head_dim] operand is addressed as
 *       base + h * stride_h + s * stride_s + d     (elements; d contiguous)
 *   - dtype codes: MGA_DTYPE_BF16, MGA_DTYPE_F16 or MGA_DTYPE_F32 (the
 *     model dtype). Attention arithmetic: bf16 operands run bf16 MFMAs and
 *     fp16 operands fp16 MFMAs, with fp32 accumulation and the probabilities
 *     and dS rounded to the operand type before their products; fp32
 *     operands run fp32 MFMAs (fp32 products, softmax and gradients).
 *   - the MTP mask is carried by one int32 code per chunk token:
 *       -1 pad, -2 regular token (x), >= 0 mask token (m) = its
 *       num_prefix_x value; every cached prefix key counts as x.
 *   - block-mask tensors are the eight int32 arrays of a torch BlockMask with
 *     B = H = 1 and 128 x 128 tiles: kv_num[nQ], kv_idx[nQ * nKV] (partial
 *     tiles), full_kv_num / full_kv_idx (full tiles) and the q-major
 *     transposes q_num[nKV], q_idx[nKV * nQ], full_q_num / full_q_idx.
 *     The attention kernels read them on the device, so they cannot be
 *     checked before the launch: counts are clamped to [0, n] and indices to
 *     [0, n - 1] (n = tiles per row). Lists that are not what
 *     mga_mtp_block_mask writes give wrong results, never an access outside
 *     the operands.
 */
#ifndef MTP_GLORA_AMD_H
#define MTP_GLORA_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MGA_OK 0
#define MGA_ERR_INVALID 1   /* bad argument (shape, stride, alignment, dtype) */
#define MGA_ERR_CAPACITY 2  /* cache capacity exceeded */
#define MGA_ERR_HIP 3       /* HIP launch / runtime error */

#define MGA_DTYPE_BF16 0
#define MGA_DTYPE_F32 1
#define MGA_DTYPE_F16 2

#define MGA_BWD_DQ 1        /* mga_attn_bwd: delta = rowsum(o * dout), then dQ */
#define MGA_BWD_DKDV 2      /* mga_attn_bwd: dK / dV (reads the delta of the dQ pass) */
#define MGA_BWD_WS_WORDS_PER_ROW 3   /* delta workspace words per (query head, row) */

#define MGA_BLOCK 128       /* BlockMask tile edge, [torch]nn/attention/flex_attention.py:395 */

/* Library version (major * 10000 + minor * 100 + patch). */
int mga_version(void);

/* Message of the last error raised on the calling thread ("" if none). */
const char *mga_last_error(void);

/*
 * Row copy into the preallocated cache:
 *   dst[h, dst_offset + r, :] = src[h, idx ? idx[r] : r, :]   for r < n_rows, h < n_heads
 * for K and V together. src_rows: rows of the source per head. Without idx,
 * n_rows > src_rows is rejected (MGA_ERR_INVALID) before any launch; idx
 * lives in device memory, so its entries are checked on the device: a row
 * whose idx[r] falls outside [0, src_rows) is left unwritten.
 * Replaces, with idx == NULL, the torch.cat of DynamicLayer.update
 * ([tf]cache_utils.py:144-146; called at mtp_glora/models/modeling_qwen3.py:284
 * and modeling_llama.py:317), and, with idx = the chunk's regular-token
 * indices, the split + gather + cat + detach of
 * mtp_glora/data_utils/collator.py:273-282.
 * Errors: MGA_ERR_CAPACITY when dst_offset + n_rows > dst_capacity.
 */
int mga_kv_append(const void *src_k, const void *src_v, int64_t src_stride_h, int64_t src_stride_s,
                  int64_t src_rows, const int32_t *idx, int32_t n_rows,
                  void *dst_k, void *dst_v, int64_t dst_stride_h, int64_t dst_stride_s,
                  int64_t dst_offset, int64_t dst_capacity,
                  int32_t n_heads, int32_t head_dim, int32_t dtype, void *stream);

/*
 * Indices of the regular tokens of a chunk: idx[0..count) = positions r with
 * regular_mask[r * stride] != 0, ascending; *count written on the device.
 * Replaces chunk['regular_token_mask'][0].nonzero() (collator.py:249).
 */
int mga_regular_index(const int64_t *regular_mask, int64_t stride, int32_t n,
                      int32_t *idx, int32_t *count, void *stream);

/*
 * MTP block mask of a chunk with S tokens against a P-token cached prefix:
 * writes the per-token codes and the eight BlockMask tensors that
 * create_block_mask(mask_mod, B=None, H=None, Q_LEN=S, KV_LEN=P+S) returns for
 * the mask_mod of collator.py:311-355 (collator.py:290-363), with
 * nQ = ceil(S / 128), nKV = ceil((P + S) / 128).
 * gate: the chunk's gate_mask (int64, -1 pad / 0 / 1), element stride gate_stride.
 * tile_class: workspace of nQ * nKV bytes.
 */
int mga_mtp_block_mask(const int64_t *gate, int64_t gate_stride, int32_t S, int64_t P,
                       int32_t *code, int8_t *tile_class,
                       int32_t *kv_num, int32_t *kv_idx, int32_t *full_kv_num, int32_t *full_kv_idx,
                       int32_t *q_num, int32_t *q_idx, int32_t *full_q_num, int32_t *full_q_idx,
                       void *stream);

/*
 * MTP block-masked GQA attention forward over L = P + S keys:
 *   o[s, h, :] = softmax_j(scale * q[h, s] . k[h / G, j], allowed(s, j)) v[h / G, j]
 *   lse[h * S + s] = natural-log logsumexp (-inf, with o = 0, for a fully masked row)
 * q: [Hq, S, D]; k, v: [Hkv, L, D]; o: [Hq, S, D] addressed with (o_sh, o_ss)
 * (o_sh = D, o_ss = Hq * D gives the [S, Hq, D] layout the attention wrapper returns).
 * Tiles are visited from the block-mask lists: empty tiles are skipped, partial
 * tiles evaluate the mask per element from `code`, full tiles do not.
 * scale must be positive and finite (the models pass head_dim ** -0.5,
 * modeling_qwen3.py:199); other values return MGA_ERR_INVALID, here and in
 * the backward.
 * Replaces flex_attention_forward ([tf]integrations/flex_attention.py:262-368)
 * -> flex_attention ([torch]nn/attention/flex_attention.py:1396) as called from
 * modeling_qwen3.py:286-300 / modeling_llama.py:320-332.
 */
int mga_attn_fwd(const void *q, int64_t q_sh, int64_t q_ss,
                 const void *k, int64_t k_sh, int64_t k_ss,
                 const void *v, int64_t v_sh, int64_t v_ss,
                 void *o, int64_t o_sh, int64_t o_ss,
                 float *lse, const int32_t *code,
                 const int32_t *kv_num, const int32_t *kv_idx,
                 const int32_t *full_kv_num, const int32_t *full_kv_idx,
                 int32_t S, int32_t L, int32_t P, int32_t Hq, int32_t Hkv,
                 int32_t head_dim, int32_t dtype, float scale, void *stream);

/*
 * Backward of mga_attn_fwd with grad_lse = 0 (the decoder discards the LSE,
 * modeling_qwen3.py:341):
 *   dq [Hq, S, D] for every visited tile (cached prefix included);
 *   dk, dv [Hkv, L - grad_start, D] for keys j >= grad_start only, summed over
 *   the G query heads of each kv head. With grad_start = P the detached
 *   prefix (collator.py:279-280) gets no gradient and costs no dK/dV work.
 * delta: workspace of MGA_BWD_WS_WORDS_PER_ROW * Hq * S 32-bit words (16-byte
 *   aligned): the row data of each (query head, row) -- -lse / scale, -delta
 *   with delta = rowsum(o * dout), and the row's mask threshold -- written by
 *   the dQ pass and read by the dK/dV pass. dK/dV are summed over the G query
 *   heads inside the pass, in a fixed order (no other workspace, no atomics).
 * passes: MGA_BWD_DQ | MGA_BWD_DKDV for the full backward. MGA_BWD_DQ alone
 *   serves a caller whose K/V need no gradient; the passes may also be issued
 *   as two calls in stream order (MGA_BWD_DQ first: it writes delta).
 * Replaces flex_attention's backward ([torch]_higher_order_ops/flex_attention.py:826-990)
 * followed by the cat-backward of DynamicLayer.update.
 * dq, dk, dv are fully written (no accumulation into existing contents).
 */
int mga_attn_bwd(const void *q, int64_t q_sh, int64_t q_ss,
                 const void *k, int64_t k_sh, int64_t k_ss,
                 const void *v, int64_t v_sh, int64_t v_ss,
                 const void *o, int64_t o_sh, int64_t o_ss,
                 const void *dout, int64_t do_sh, int64_t do_ss,
                 const float *lse, float *delta,
                 void *dq, int64_t dq_sh, int64_t dq_ss,
                 void *dk, int64_t dk_sh, int64_t dk_ss,
                 void *dv, int64_t dv_sh, int64_t dv_ss,
                 int32_t grad_start, const int32_t *code,
                 const int32_t *kv_num, const int32_t *kv_idx,
                 const int32_t *full_kv_num, const int32_t *full_kv_idx,
                 const int32_t *q_num, const int32_t *q_idx,
                 const int32_t *full_q_num, const int32_t *full_q_idx,
                 int32_t S, int32_t L, int32_t P, int32_t Hq, int32_t Hkv,
                 int32_t head_dim, int32_t dtype, float scale, int32_t passes, void *stream);

/*
 * mga_attn_bwd without the delta workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). No counterpart in the reference. delta
 * lives in a fixed device array of 3 * 2 097 152 words (24 MiB) that the
 * library holds on every GPU it runs on until the process ends; calls with
 * Hq * S > 2 097 152 are rejected with MGA_ERR_INVALID before any device work.
 * The call itself allocates nothing (no hipMalloc, no library allocation).
 * Every call on a GPU shares that GPU's array and it keeps the last call's
 * contents: calls that overlap on one GPU (e.g. on two streams) race, and an
 * MGA_BWD_DKDV-only call reads the delta the last MGA_BWD_DQ call on that GPU
 * wrote. The calling thread's current device must be the stream's device.
 * Results are bit-for-bit those of mga_attn_bwd.
 */
int mga_attn_bwd_noalloc(const void *q, int64_t q_sh, int64_t q_ss,
                         const void *k, int64_t k_sh, int64_t k_ss,
                         const void *v, int64_t v_sh, int64_t v_ss,
                         const void *o, int64_t o_sh, int64_t o_ss,
                         const void *dout, int64_t do_sh, int64_t do_ss,
                         const float *lse,
                         void *dq, int64_t dq_sh, int64_t dq_ss,
                         void *dk, int64_t dk_sh, int64_t dk_ss,
                         void *dv, int64_t dv_sh, int64_t dv_ss,
                         int32_t grad_start, const int32_t *code,
                         const int32_t *kv_num, const int32_t *kv_idx,
                         const int32_t *full_kv_num, const int32_t *full_kv_idx,
                         const int32_t *q_num, const int32_t *q_idx,
                         const int32_t *full_q_num, const int32_t *full_q_idx,
                         int32_t S, int32_t L, int32_t P, int32_t Hq, int32_t Hkv,
                         int32_t head_dim, int32_t dtype, float scale, int32_t passes, void *stream);

/*
 * Qwen3 query / key normalisation and rotary embedding, fused:
 *   for every token s and head h of q [S, Hq, D] (weight q_weight) and of
 *   k [S, Hkv, D] (weight k_weight), with x = the row in fp32:
 *     r = 1 / sqrt(mean(x * x) + eps),  n = T(w * T(x * r)),
 *     out = T(T(n * cos[s]) + T(rotate_half(n) * sin[s])),
 *     rotate_half(n) = [-n[D/2:], n[:D/2]],
 *   T = rounding to the model dtype after each op, as the reference's torch ops
 *   do; rstd[s * (Hq + Hkv) + row] = r (rows: the Hq query heads, then the Hkv
 *   key heads) is saved for the backward.
 * Operands are addressed base + s * token_stride + h * head_stride + d
 * (elements); cos / sin are [S, D] with token stride cs_stride; D even, <= 128.
 * Replaces q_norm / k_norm (Qwen3RMSNorm.forward,
 * mtp_glora/models/modeling_qwen3.py:61-67) and apply_rotary_pos_emb
 * (:118-149) as called by Qwen3Attention.forward (:274-279).
 */
int mga_qk_norm_rope_fwd(const void *q, int64_t q_token_stride, int64_t q_head_stride,
                         const void *k, int64_t k_token_stride, int64_t k_head_stride,
                         const void *q_weight, const void *k_weight,
                         const void *cos, const void *sin, int64_t cs_stride,
                         float eps, int32_t S, int32_t Hq, int32_t Hkv, int32_t head_dim, int32_t dtype,
                         void *q_out, int64_t qo_token_stride, int64_t qo_head_stride,
                         void *k_out, int64_t ko_token_stride, int64_t ko_head_stride,
                         float *rstd, void *stream);

/*
 * mga_qk_norm_rope_fwd that also copies the value rows v [S, Hkv, D] to
 * v_out unchanged, in the same launch: with k_out / v_out pointing at a
 * layer's KV-cache rows [P, P + S) (for a [Hkv, capacity, D] cache buffer:
 * base + P * D, token stride D, head stride capacity * D) it writes the
 * chunk's post-RoPE keys and its values where the cache update
 * (DynamicLayer.update via Cache.update, [tf]cache_utils.py:1349-1381, called
 * at modeling_qwen3.py:281-284) would copy them, so no separate append runs.
 *   - q may be null (with q_weight, q_out and rstd ignored / null): keys and
 *     values only, e.g. to re-stage a chunk's regular rows into the prefix;
 *   - rows may be null; else output row s (s < S) reads input row rows[s] of
 *     q / k / v and cos / sin row rows[s], and rows outside [0, src_rows) are
 *     skipped (the regular-token gather of collator.py:270-277);
 *   - rstd may be null (nothing saved for a backward).
 */
int mga_qk_norm_rope_stage_fwd(const void *q, int64_t q_token_stride, int64_t q_head_stride,
                               const void *k, int64_t k_token_stride, int64_t k_head_stride,
                               const void *v, int64_t v_token_stride, int64_t v_head_stride,
                               const void *q_weight, const void *k_weight,
                               const void *cos, const void *sin, int64_t cs_stride, float eps,
                               const int32_t *rows, int32_t src_rows,
                               int32_t S, int32_t Hq, int32_t Hkv, int32_t head_dim, int32_t dtype,
                               void *q_out, int64_t qo_token_stride, int64_t qo_head_stride,
                               void *k_out, int64_t ko_token_stride, int64_t ko_head_stride,
                               void *v_out, int64_t vo_token_stride, int64_t vo_head_stride,
                               float *rstd, void *stream);

/*
 * Backward of mga_qk_norm_rope_fwd for q and k (the norm weights, cos and sin
 * get no gradient): given the output gradients dq_out / dk_out, writes
 *   dx = r * dy - (r^3 / D) * x * sum(dy * x),  dy = w * dn,
 *   dn = g * cos + [g[D/2:] * sin[D/2:], -g[:D/2] * sin[:D/2]]
 * (fp32, the forward's roundings taken as identity).
 * Replaces the autograd backward of the ops above.
 */
int mga_qk_norm_rope_bwd(const void *q, int64_t q_token_stride, int64_t q_head_stride,
                         const void *k, int64_t k_token_stride, int64_t k_head_stride,
                         const void *q_weight, const void *k_weight,
                         const void *cos, const void *sin, int64_t cs_stride, const float *rstd,
                         int32_t S, int32_t Hq, int32_t Hkv, int32_t head_dim, int32_t dtype,
                         const void *dq_out, int64_t dqo_token_stride, int64_t dqo_head_stride,
                         const void *dk_out, int64_t dko_token_stride, int64_t dko_head_stride,
                         void *dq, int64_t dq_token_stride, int64_t dq_head_stride,
                         void *dk, int64_t dk_token_stride, int64_t dk_head_stride, void *stream);

/*
 * Gated LoRA linear layer (GatedLoRALinear.forward,
 * mtp_glora/models/layers/gated_lora.py:51-53), operands of one dtype code
 * (MGA_DTYPE_BF16, MGA_DTYPE_F16 or MGA_DTYPE_F32, the reference's model
 * dtypes, args.py:15):
 *   y = x W^T + scaling * B(A(dropout(x))) * gate,
 * computed as y = T(x W^T + T(t B^T)) (the base GEMM accumulates onto the
 * rounded LoRA term), for x [S, K] (row stride x_rs), W [N, K], A =
 * lora_A.weight [rank, K],
 * B = lora_B.weight [N, rank], gate [S] fp32 (NULL = 1; the reference's
 * clamped gate mask). Writes y [S, N] and, for the backward, t [S, rpad]
 * (rpad = rank rounded up to 32; t = T(T(scaling * T(h A^T)) * gate), T =
 * rounding to the dtype, h = dropout(x)) and, when dropout_p > 0 and h is not
 * NULL, h [S, K] (NULL, bf16 only: h is not kept and the backward draws the
 * mask again from x, which needs K a multiple of 128; fp16 and fp32 need h).
 * Dropout keeps element i of the flattened [S, K] input by a hash of
 * (seed, i) with probability 1 - round(65536 p) / 65536 and scales kept
 * elements by 1 / (1 - p). K must be a multiple of 16; with bf16, x, lora_A
 * and h are read or written with 16-byte vectors (aligned rows, strides
 * multiples of 8). workspace: mga_gated_lora_workspace_bytes(S, K, N, rank)
 * bytes. bf16 runs the HIP down-projection kernel (dropout, scaling and gate
 * fused); fp16 and fp32 run every product in hipBLASLt in the operand type
 * (fp32 compute) with HIP kernels for the dropout and the row scaling. The
 * plain GEMMs run in hipBLASLt on the same stream.
 */
int64_t mga_gated_lora_workspace_bytes(int32_t S, int32_t K, int32_t N, int32_t rank);
int mga_gated_lora_fwd(const void *x, int64_t x_rs, const void *weight, int64_t w_rs,
                       const void *lora_a, int64_t a_rs, const void *lora_b, int64_t b_rs,
                       const float *gate, float scaling, double dropout_p, uint64_t seed,
                       int32_t S, int32_t K, int32_t N, int32_t rank,
                       void *y, int64_t y_rs, void *t, int64_t t_rs, void *h, int64_t h_rs,
                       void *workspace, int64_t workspace_bytes, int32_t dtype, void *stream);

/*
 * Backward of mga_gated_lora_fwd (the autograd backward of the reference's
 * GatedLoRALinear.forward with the base weight frozen, gated_lora.py:51-53,
 * :56-58): from grad_y [S, N] and the forward's x, h, t and seed,
 *   grad_B = grad_y^T t,  d_a = T(T((grad_y B) * gate) * scaling),
 *   grad_x = T(grad_y W + T(mask * T(d_a A) / (1 - p))),  grad_A = d_a^T h.
 * grad_x, grad_a, grad_b may be NULL to skip them; h may be NULL when the
 * forward kept no dropout output (bf16: grad_A then recomputes it from x
 * and the seed; K a multiple of 128). With bf16 and dropout on, grad_x is
 * written with vector accesses: its start must be 16-byte aligned and its
 * row stride a multiple of 4 (of 8 for the 16-byte path). With bf16, grad_y B
 * and grad_y^T t run as one streaming pass over grad_y each (fp32 split sums
 * added in a fixed order) when rank <= 128, N is a multiple of 8 and grad_y,
 * lora_B and t have 16-byte aligned rows (strides multiples of 8); otherwise,
 * and for fp16 and fp32, in hipBLASLt, as grad_y W is.
 */
int mga_gated_lora_bwd(const void *grad_y, int64_t gy_rs, const void *x, int64_t x_rs,
                       const void *h, int64_t h_rs, const void *weight, int64_t w_rs,
                       const void *lora_a, int64_t a_rs, const void *lora_b, int64_t b_rs,
                       const void *t, int64_t t_rs, const float *gate, float scaling,
                       double dropout_p, uint64_t seed, int32_t S, int32_t K, int32_t N, int32_t rank,
                       void *grad_x, int64_t gx_rs, void *grad_a, int64_t ga_rs,
                       void *grad_b, int64_t gb_rs, void *workspace, int64_t workspace_bytes,
                       int32_t dtype, void *stream);

/*
 * Stable soft cross-entropy of the MTP sampler loss, row by row over n_rows
 * rows of n_cols logits (row r of a [rows, cols] operand starts at
 * base + r * row_stride elements; columns contiguous). For student logits x
 * and teacher logits t (the same dtype code, MGA_DTYPE_BF16, MGA_DTYPE_F16 or MGA_DTYPE_F32):
 *   mx = max x, dx = max(sum e^{x - mx}, 1e-20), mt = max t,
 *   dt = max(sum e^{t - mt}, 1e-20),
 *   row_loss[r] = -(sum e^{t - mt} x) / dt + mx + log dx,
 *   stats = [mx[n_rows], dx[n_rows], mt[n_rows], dt[n_rows]] (fp32).
 * The caller sums row_loss (StableSoftCrossEntropy.forward returns that sum).
 * workspace: mga_soft_ce_workspace_floats(n_rows, n_cols) fp32 values.
 * Replaces stable_soft_ce_forward_kernel_{auto,manual}
 * (mtp_glora/core/loss.py:63-179) as launched by
 * StableSoftCrossEntropy.forward (loss.py:259-296).
 */
int64_t mga_soft_ce_workspace_floats(int32_t n_rows, int32_t n_cols);
int mga_soft_ce_fwd(const void *student, int64_t student_row_stride,
                    const void *teacher, int64_t teacher_row_stride,
                    int32_t n_rows, int32_t n_cols, int32_t dtype,
                    float *row_loss, float *stats, float *workspace, void *stream);

/*
 * Backward of mga_soft_ce_fwd for the student (the teacher gets none):
 *   grad[r, j] = grad_output * (e^{x - mx} / dx - e^{t - mt} / dt)
 * written in the student's dtype; grad_output: one fp32 value in device
 * memory (the upstream gradient of the summed loss); stats from the forward.
 * Replaces stable_soft_ce_backward_kernel_{auto,manual} (loss.py:182-256) and
 * the dtype cast of StableSoftCrossEntropy.backward (loss.py:298-330).
 */
int mga_soft_ce_bwd(const void *student, int64_t student_row_stride,
                    const void *teacher, int64_t teacher_row_stride,
                    int32_t n_rows, int32_t n_cols, int32_t dtype,
                    const float *grad_output, const float *stats,
                    void *grad, int64_t grad_row_stride, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* MTP_GLORA_AMD_H */
