// Streaming KV cache kernels: row copy / gather into the preallocated
// per-layer [heads, capacity, head_dim] buffers, and the regular-token index.
#include "mga_common.hpp"
#include "mga_internal.hpp"

namespace mga {

// grid.y = tensor * n_heads + head (tensor 0 = K, 1 = V); grid.x covers the
// (row, 16-byte vector) pairs of that head with the vector index fastest, so
// each source row is one contiguous run and the destination of a head is one
// sequential stream. Each thread keeps kVecPerThread loads in flight; the
// stores are non-temporal (no cache allocation: the rows written are not read
// again by this kernel, and the next reader's first touch comes from HBM
// anyway). Measured on the 4096-row commit (16.8 MB each way): 4.3 us
// (97 % of HBM) against 6.4 us with 4 vectors per thread, 256 threads and
// ordinary stores.
constexpr int kVecPerThread = 2;
constexpr int kCopyThreads = 512;

__global__ __launch_bounds__(kCopyThreads) void kv_copy_rows_kernel(
    const char *__restrict__ src_k, const char *__restrict__ src_v,
    int64_t src_sh, int64_t src_ss,                 // bytes
    const int32_t *__restrict__ idx, int64_t src_rows, uint32_t n_rows,
    char *__restrict__ dst_k, char *__restrict__ dst_v,
    int64_t dst_sh, int64_t dst_ss, int64_t dst_off, // bytes, rows
    uint32_t n_heads, uint32_t vpr_shift) {
  const uint32_t th = blockIdx.y;
  const bool is_v = th >= n_heads;
  const uint32_t h = is_v ? th - n_heads : th;
  const char *src = (is_v ? src_v : src_k) + (int64_t)h * src_sh;
  char *dst = (is_v ? dst_v : dst_k) + (int64_t)h * dst_sh + dst_off * dst_ss;
  const uint32_t per_head = n_rows << vpr_shift;
  const uint32_t vmask = (1u << vpr_shift) - 1;
  const uint32_t base = blockIdx.x * (kCopyThreads * kVecPerThread) + threadIdx.x;
  i32x4 buf[kVecPerThread];
  bool ok[kVecPerThread];
#pragma unroll
  for (int i = 0; i < kVecPerThread; ++i) {
    const uint32_t w = base + i * kCopyThreads;
    ok[i] = w < per_head;
    if (ok[i]) {
      const uint32_t r = w >> vpr_shift;
      const uint32_t vec = w & vmask;
      const int64_t srow = idx ? (int64_t)idx[r] : (int64_t)r;
      // a gather index outside the source leaves its row unwritten
      ok[i] = srow >= 0 && srow < src_rows;
      if (ok[i]) buf[i] = *reinterpret_cast<const i32x4 *>(src + srow * src_ss + vec * 16);
    }
  }
#pragma unroll
  for (int i = 0; i < kVecPerThread; ++i) {
    const uint32_t w = base + i * kCopyThreads;
    if (ok[i]) {
      const uint32_t r = w >> vpr_shift;
      const uint32_t vec = w & vmask;
      __builtin_nontemporal_store(buf[i], reinterpret_cast<i32x4 *>(dst + (int64_t)r * dst_ss + vec * 16));
    }
  }
}

void launch_kv_copy_rows(const void *src_k, const void *src_v, int64_t src_sh_b, int64_t src_ss_b,
                         int64_t src_rows, const int32_t *idx, int32_t n_rows, void *dst_k, void *dst_v,
                         int64_t dst_sh_b, int64_t dst_ss_b, int64_t dst_off, int32_t n_heads,
                         int32_t row_bytes, hipStream_t stream) {
  uint32_t shift = 0;
  while ((16u << shift) < (uint32_t)row_bytes) ++shift;
  const uint64_t per_head = (uint64_t)n_rows << shift;
  if (per_head == 0) return;
  const uint64_t per_block = (uint64_t)kCopyThreads * kVecPerThread;
  const uint32_t gx = (uint32_t)((per_head + per_block - 1) / per_block);
  hipLaunchKernelGGL(kv_copy_rows_kernel, dim3(gx, 2 * n_heads), dim3(kCopyThreads), 0, stream,
                     (const char *)src_k, (const char *)src_v, src_sh_b, src_ss_b, idx, src_rows,
                     (uint32_t)n_rows, (char *)dst_k, (char *)dst_v, dst_sh_b, dst_ss_b, dst_off,
                     (uint32_t)n_heads, shift);
}

// Single-workgroup stream compaction: each thread owns a contiguous segment,
// counts its nonzeros, a block scan gives its output offset.
__global__ __launch_bounds__(1024) void regular_index_kernel(const int64_t *__restrict__ mask,
                                                             int64_t stride, int32_t n,
                                                             int32_t *__restrict__ idx,
                                                             int32_t *__restrict__ count) {
  __shared__ int scan[1024];
  const int t = threadIdx.x;
  const int seg = (n + 1023) / 1024;
  const int b = t * seg;
  const int e = min(n, b + seg);
  int c = 0;
  for (int i = b; i < e; ++i) c += mask[(int64_t)i * stride] != 0;
  scan[t] = c;
  __syncthreads();
  for (int off = 1; off < 1024; off <<= 1) {
    const int v = t >= off ? scan[t - off] : 0;
    __syncthreads();
    scan[t] += v;
    __syncthreads();
  }
  int pos = scan[t] - c;
  for (int i = b; i < e; ++i)
    if (mask[(int64_t)i * stride] != 0) idx[pos++] = i;
  if (t == 1023) *count = scan[1023];
}

void launch_regular_index(const int64_t *mask, int64_t stride, int32_t n, int32_t *idx,
                          int32_t *count, hipStream_t stream) {
  hipLaunchKernelGGL(regular_index_kernel, dim3(1), dim3(1024), 0, stream, mask, stride, n, idx,
                     count);
}

}  // namespace mga
