// MTP block-mask construction on the GPU: per-token codes, 128x128 tile
// classes, and the eight ordered BlockMask index tensors.
//
// The tensors equal what create_block_mask returns for the reference's
// mask_mod (mtp_glora/data_utils/collator.py:290-363): tiles are padded with
// False to a multiple of 128 ([torch]nn/attention/flex_attention.py:979-1022),
// a tile is "full" when all 128*128 entries are allowed and "partial" when some
// are, and every index row is the selected tiles ascending followed by the
// rest ascending (the stable descending argsort of :429-436; the q-major lists
// are the transposes of :439-441).
#include "mga_common.hpp"
#include "mga_internal.hpp"

namespace mga {

// ---- codes ----------------------------------------------------------------
// code[i] = -1 pad, -2 regular, else P + #(gate == 0 in [0, i]) -- the
// num_prefix_x of collator.py:320 for a mask token (the P cached tokens are
// all regular, collator.py:311-318).
__global__ __launch_bounds__(1024) void mtp_codes_kernel(const int64_t *__restrict__ gate,
                                                         int64_t stride, int32_t n, int64_t P,
                                                         int32_t *__restrict__ code) {
  __shared__ int scan[1024];
  const int t = threadIdx.x;
  const int seg = (n + 1023) / 1024;
  const int b = t * seg;
  const int e = min(n, b + seg);
  int c = 0;
  for (int i = b; i < e; ++i) c += gate[(int64_t)i * stride] == 0;
  scan[t] = c;
  __syncthreads();
  for (int off = 1; off < 1024; off <<= 1) {
    const int v = t >= off ? scan[t - off] : 0;
    __syncthreads();
    scan[t] += v;
    __syncthreads();
  }
  int run = scan[t] - c;  // zeros before this segment
  for (int i = b; i < e; ++i) {
    const int64_t g = gate[(int64_t)i * stride];
    run += g == 0;
    code[i] = g == -1 ? kCodePad : (g == 0 ? kCodeX : (int)(P + run));
  }
}

// ---- tile classes -----------------------------------------------------------
// grid (nKV, nQ); class 0 empty, 1 partial, 2 full.
__global__ __launch_bounds__(256) void tile_class_kernel(const int32_t *__restrict__ code, int32_t S,
                                                         int32_t P, int32_t L, int32_t nKV,
                                                         int8_t *__restrict__ cls) {
  __shared__ int sq[kBlock];
  __shared__ int sk[kBlock];
  __shared__ int red[8];
  const int t = threadIdx.x;
  const int kt = blockIdx.x, qt = blockIdx.y;
  const int q0 = qt * kBlock, k0 = kt * kBlock;
  const int nq = min(kBlock, S - q0);
  const int nk = min(kBlock, L - k0);
  if (k0 > q0 + nq - 1 + P) {
    // every key follows every query of the tile: causally empty
    if (t == 0) cls[(int64_t)qt * nKV + kt] = 0;
    return;
  }
  if (t < kBlock) sq[t] = t < nq ? code[q0 + t] : kCodePad;
  else sk[t - kBlock] = (t - kBlock) < nk ? key_code(code, k0 + t - kBlock, P, L) : kCodePad;
  __syncthreads();
  int cnt = 0;
  if (k0 + nk <= P) {
    // every key is a cached regular token and precedes every chunk query
    if (t < kBlock) cnt = (sq[t] != kCodePad) ? nk : 0;
  } else {
    const int row = t & (kBlock - 1);
    const int half = t >> 7;
    const int qc = sq[row];
    const int qg = q0 + row + P;
#pragma unroll 8
    for (int j = half * 64; j < half * 64 + 64; ++j)
      cnt += (int)(j < nk && row < nq && mtp_allowed(qg, qc, k0 + j, sk[j]));
  }
  // block reduce
  for (int off = 32; off > 0; off >>= 1) cnt += __shfl_down(cnt, off, 64);
  if ((t & 63) == 0) red[t >> 6] = cnt;
  __syncthreads();
  if (t == 0) {
    const int tot = red[0] + red[1] + red[2] + red[3];
    cls[(int64_t)qt * nKV + kt] = tot == kBlock * kBlock ? 2 : (tot > 0 ? 1 : 0);
  }
}

// ---- ordered lists ------------------------------------------------------------
// Block-wide exclusive scan of one flag per thread (256 threads).
__device__ __forceinline__ int block_excl_scan(int f, int *buf, int &total) {
  const int t = threadIdx.x;
  buf[t] = f;
  __syncthreads();
  for (int off = 1; off < 256; off <<= 1) {
    const int v = t >= off ? buf[t - off] : 0;
    __syncthreads();
    buf[t] += v;
    __syncthreads();
  }
  total = buf[255];
  const int r = buf[t] - f;
  __syncthreads();
  return r;
}

// Writes num = #selected and idx[0..n) = selected ascending then the rest ascending.
__device__ void ordered_row(const int8_t *cls, int64_t step, int n, int want, int32_t *num,
                            int32_t *idx, int *buf) {
  int tot_sel = 0;
  for (int b = 0; b < n; b += 256) {
    const int j = b + threadIdx.x;
    const int f = (j < n) && cls[j * step] == want;
    int chunk_tot;
    block_excl_scan(f, buf, chunk_tot);
    tot_sel += chunk_tot;
  }
  int carry = 0;
  for (int b = 0; b < n; b += 256) {
    const int j = b + threadIdx.x;
    const int f = (j < n) && cls[j * step] == want;
    int chunk_tot;
    const int before = block_excl_scan(f, buf, chunk_tot);
    if (j < n) {
      const int sel_before = carry + before;
      const int pos = f ? sel_before : tot_sel + (j - sel_before);
      idx[pos] = j;
    }
    carry += chunk_tot;
  }
  if (threadIdx.x == 0) *num = tot_sel;
}

// grid nQ + nKV: rows (kv lists per q tile) then columns (q lists per kv tile).
__global__ __launch_bounds__(256) void block_lists_kernel(
    const int8_t *__restrict__ cls, int32_t nQ, int32_t nKV, int32_t *kv_num, int32_t *kv_idx,
    int32_t *full_kv_num, int32_t *full_kv_idx, int32_t *q_num, int32_t *q_idx,
    int32_t *full_q_num, int32_t *full_q_idx) {
  __shared__ int buf[256];
  const int b = blockIdx.x;
  if (b < nQ) {
    const int8_t *row = cls + (int64_t)b * nKV;
    ordered_row(row, 1, nKV, 1, kv_num + b, kv_idx + (int64_t)b * nKV, buf);
    ordered_row(row, 1, nKV, 2, full_kv_num + b, full_kv_idx + (int64_t)b * nKV, buf);
  } else {
    const int c = b - nQ;
    const int8_t *col = cls + c;
    ordered_row(col, nKV, nQ, 1, q_num + c, q_idx + (int64_t)c * nQ, buf);
    ordered_row(col, nKV, nQ, 2, full_q_num + c, full_q_idx + (int64_t)c * nQ, buf);
  }
}

void launch_mtp_block_mask(const int64_t *gate, int64_t gate_stride, int32_t S, int64_t P,
                           int32_t *code, int8_t *cls, int32_t *kv_num, int32_t *kv_idx,
                           int32_t *full_kv_num, int32_t *full_kv_idx, int32_t *q_num,
                           int32_t *q_idx, int32_t *full_q_num, int32_t *full_q_idx,
                           hipStream_t stream) {
  const int L = (int)(P + S);
  const int nQ = (S + kBlock - 1) / kBlock;
  const int nKV = (L + kBlock - 1) / kBlock;
  hipLaunchKernelGGL(mtp_codes_kernel, dim3(1), dim3(1024), 0, stream, gate, gate_stride, S, P,
                     code);
  hipLaunchKernelGGL(tile_class_kernel, dim3(nKV, nQ), dim3(256), 0, stream, code, S, (int)P, L,
                     nKV, cls);
  hipLaunchKernelGGL(block_lists_kernel, dim3(nQ + nKV), dim3(256), 0, stream, cls, nQ, nKV, kv_num,
                     kv_idx, full_kv_num, full_kv_idx, q_num, q_idx, full_q_num, full_q_idx);
}

}  // namespace mga
