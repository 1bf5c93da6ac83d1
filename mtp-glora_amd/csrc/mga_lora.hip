// Gated LoRA (mtp_glora/models/layers/gated_lora.py:51-53), the parts that
// are not plain GEMMs:
//
//   out = base(x) + s * B(A(dropout(x))) * gate
//
// The plain GEMMs (x W^T, the rank-r up-projection accumulated into the
// output, dY W, dY B, dY^T t, d_a^T h) go to hipBLASLt (mga_blas.hip). The
// kernels here fuse what a library GEMM cannot:
//
// * lora_down_kernel: t = T(T(s * T(h A^T)) * gate) for every row, h =
//   dropout(x) drawn on the fly (and written out when dropout is on: the
//   backward's dA GEMM reads it, as the reference keeps its dropout output).
//   HBM-bound on x: 32 rows per workgroup, the K dimension split over 8 waves
//   (v_mfma_f32_32x32x16_bf16, operands straight from global memory), the
//   partial sums reduced through LDS.
// * lora_dx_kernel (dropout on): dX = T(dX + T(mask * scale * T(d_a A))) in
//   place over the base gradient dY W: HBM-bound on dX, the rank-r product on
//   MFMA with the output's columns along each lane's four rows.
// * lora_scale_rows_kernel: d_a = T(T(u * gate) * s), u = dY B.
// * lora_transpose_kernel: A^T padded to a multiple of 32 ranks (the dX
//   kernel's MFMA operand wants rank-contiguous rows).
//
// T rounds to bf16. With the scaling a power of two and gate values 0 / 1 (the
// reference's alpha = 2 * rank and clamped gate mask), applying s and the gate
// to t instead of to B(t) changes nothing but the rounding of B(t) itself.
//
// Dropout: keep / drop bits come from a counter-based hash, not from torch's
// generator (whose stream cannot be reproduced here): element pair j of the
// flattened [S, K] input (elements 2j, 2j + 1) gets
//   bits = fmix32(fmix32(lo(j) ^ lo(seed)) ^ hi(j) ^ hi(seed)),
// fmix32 being MurmurHash3's 32-bit finaliser; element 2j is kept when
// bits & 0xffff >= thr, element 2j + 1 when bits >> 16 >= thr, thr =
// round(p * 65536). Kept elements are multiplied by 1 / (1 - p), as
// torch's dropout does. The backward draws the same bits again.
#include "mga_common.hpp"
#include "mga_internal.hpp"

namespace mga {

namespace {

__device__ __forceinline__ uint32_t fmix32(uint32_t h) {
  h ^= h >> 16;
  h *= 0x85ebca6bu;
  h ^= h >> 13;
  h *= 0xc2b2ae35u;
  h ^= h >> 16;
  return h;
}

__device__ __forceinline__ uint32_t pair_bits(uint64_t seed, uint64_t pair) {
  return fmix32(fmix32((uint32_t)pair ^ (uint32_t)seed) ^ (uint32_t)(pair >> 32) ^ (uint32_t)(seed >> 32));
}

__device__ __forceinline__ float rnd(float v) { return (float)(bf16_t)v; }

__device__ __forceinline__ bf16x8 zero8() {
  bf16x8 z;
#pragma unroll
  for (int i = 0; i < 8; ++i) z[i] = (bf16_t)0.f;
  return z;
}

constexpr int kDownWaves = 8;

}  // namespace

// Grid: ceil(S / 32) workgroups of 8 waves. Wave w takes the 16-wide k steps
// w, w + 8, ... of the workgroup's 32 rows; NB = ranks / 32 accumulator blocks.
template <int NB, bool DROP>
__global__ __launch_bounds__(kDownWaves * 64) void lora_down_kernel(LoraDownArgs a) {
  const int w = wave_id(), lane = threadIdx.x & 63;
  const int s0 = blockIdx.x * 32;
  const int row = s0 + (lane & 31);
  const bool row_ok = row < a.S;
  const int kq = 8 * (lane >> 5);
  const bf16_t *xr = reinterpret_cast<const bf16_t *>(a.x) + (int64_t)(row_ok ? row : 0) * a.x_rs + kq;
  bf16_t *hr = (DROP && a.h) ? reinterpret_cast<bf16_t *>(a.h) + (int64_t)(row_ok ? row : 0) * a.h_rs + kq : nullptr;
  const bf16_t *ar[NB];
  bool a_ok[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    const int r = nb * 32 + (lane & 31);
    a_ok[nb] = r < a.rank;
    ar[nb] = reinterpret_cast<const bf16_t *>(a.A) + (int64_t)(a_ok[nb] ? r : 0) * a.a_rs + kq;
  }
  f32x16 acc[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) acc[nb] = zero16();
  const uint64_t pair0 = ((uint64_t)(row_ok ? row : 0) * (uint64_t)a.K + (uint64_t)kq) >> 1;

#pragma unroll 4
  for (int k0 = 16 * w; k0 < a.K; k0 += 16 * kDownWaves) {
    bf16x8 xv = row_ok ? load8(xr + k0) : zero8();
    if constexpr (DROP) {
      const uint64_t pj = pair0 + ((uint64_t)k0 >> 1);
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        const uint32_t bits = pair_bits(a.seed, pj + (e >> 1));
        const bool k_lo = (bits & 0xffffu) >= a.thr, k_hi = (bits >> 16) >= a.thr;
        xv[e] = k_lo ? (bf16_t)((float)xv[e] * a.keep_scale) : (bf16_t)0.f;
        xv[e + 1] = k_hi ? (bf16_t)((float)xv[e + 1] * a.keep_scale) : (bf16_t)0.f;
      }
      if (row_ok && hr) *reinterpret_cast<i32x4 *>(hr + k0) = __builtin_bit_cast(i32x4, xv);
    }
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      const bf16x8 av = a_ok[nb] ? load8(ar[nb] + k0) : zero8();
      acc[nb] = mfma32(xv, av, acc[nb]);
    }
  }

  // fixed-order reduction of the 8 waves' partial sums: 4..7 into 0..3, then 1..3 into 0
  __shared__ float red[4][NB][16][64];
  if (w >= 4) {
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int q = 0; q < 16; ++q) red[w - 4][nb][q][lane] = acc[nb][q];
  }
  __syncthreads();
  if (w < 4) {
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int q = 0; q < 16; ++q) acc[nb][q] += red[w][nb][q][lane];
  }
  __syncthreads();
  if (w >= 1 && w < 4) {
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int q = 0; q < 16; ++q) red[w - 1][nb][q][lane] = acc[nb][q];
  }
  __syncthreads();
  if (w != 0) return;
#pragma unroll
  for (int nb = 0; nb < NB; ++nb)
#pragma unroll
    for (int q = 0; q < 16; ++q) acc[nb][q] += red[0][nb][q][lane] + red[1][nb][q][lane] + red[2][nb][q][lane];

  bf16_t *t = reinterpret_cast<bf16_t *>(a.t);
#pragma unroll
  for (int q = 0; q < 16; ++q) {
    const int s = s0 + 8 * (q >> 2) + 4 * (lane >> 5) + (q & 3);
    if (s >= a.S) continue;
    const float g = a.gate ? a.gate[s] : 1.f;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      const int r = nb * 32 + (lane & 31);
      // lora_A output in bf16, then the scaling and the gate, each rounded
      t[(int64_t)s * a.t_rs + r] = (bf16_t)(rnd(rnd(acc[nb][q]) * a.scaling) * g);
    }
  }
}

// Grid: (ceil(K / 512), ceil(S / 32)), 4 waves; wave w covers 32 rows x 128
// columns of dX. D^T[k][s] = sum_r A^T[k][r] d_a[s][r]; each lane holds one
// row s and four runs of four consecutive columns per 32-column block.
__global__ __launch_bounds__(256) void lora_dx_kernel(LoraDxArgs a) {
  const int w = wave_id(), lane = threadIdx.x & 63;
  const int s = blockIdx.y * 32 + (lane & 31);
  const bool s_ok = s < a.S;
  const int rq = 8 * (lane >> 5);
  const int nsteps = (a.rank + 15) / 16;   // d_a and A^T are zero-padded to a multiple of 32 ranks
  const bf16_t *dar = reinterpret_cast<const bf16_t *>(a.da) + (int64_t)(s_ok ? s : 0) * a.da_rs + rq;
  bf16_t *dxr = reinterpret_cast<bf16_t *>(a.dx) + (int64_t)(s_ok ? s : 0) * a.dx_rs;
  const int kb0 = blockIdx.x * 512 + w * 128;
  for (int blk = 0; blk < 4; ++blk) {
    const int kbase = kb0 + blk * 32;
    if (kbase >= a.K) break;
    const int kr = kbase + (lane & 31);
    const bf16_t *atr = reinterpret_cast<const bf16_t *>(a.At) + (int64_t)(kr < a.K ? kr : 0) * a.at_rs + rq;
    f32x16 acc = zero16();
    for (int j = 0; j < nsteps; ++j) {
      const bf16x8 av = kr < a.K ? load8(atr + 16 * j) : zero8();
      const bf16x8 dv = s_ok ? load8(dar + 16 * j) : zero8();
      acc = mfma32(av, dv, acc);
    }
    if (!s_ok) continue;
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      const int k = kbase + 8 * g4 + 4 * (lane >> 5);
      if (k >= a.K) continue;
      const uint64_t pj = ((uint64_t)s * (uint64_t)a.K + (uint64_t)k) >> 1;
      const uint32_t b0 = pair_bits(a.seed, pj), b1 = pair_bits(a.seed, pj + 1);
      const bool keep[4] = {(b0 & 0xffffu) >= a.thr, (b0 >> 16) >= a.thr, (b1 & 0xffffu) >= a.thr,
                            (b1 >> 16) >= a.thr};
      bf16x4 cur = *reinterpret_cast<const bf16x4 *>(dxr + k);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float dh = rnd(acc[4 * g4 + e]);                      // d(dropout(x)) = T(d_a A)
        const float dl = keep[e] ? rnd(dh * a.keep_scale) : 0.f;   // dropout backward
        cur[e] = (bf16_t)((float)cur[e] + dl);                     // + base gradient
      }
      *reinterpret_cast<bf16x4 *>(dxr + k) = cur;
    }
  }
}

// d_a[s][r] = T(T(u[s][r] * gate[s]) * s) for r < rank, 0 up to rpad.
__global__ __launch_bounds__(256) void lora_scale_rows_kernel(const bf16_t *u, int64_t u_rs, const float *gate,
                                                              float scaling, int32_t S, int32_t rank, int32_t rpad,
                                                              bf16_t *da, int64_t da_rs) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)S * rpad) return;
  const int s = (int)(i / rpad), r = (int)(i - (int64_t)s * rpad);
  float v = 0.f;
  if (r < rank) {
    const float g = gate ? gate[s] : 1.f;
    v = rnd(rnd((float)u[(int64_t)s * u_rs + r] * g) * scaling);
  }
  da[(int64_t)s * da_rs + r] = (bf16_t)v;
}

// At[k][r] = A[r][k] for r < rank, 0 up to rpad. 32 x 32 tiles through LDS.
__global__ __launch_bounds__(256) void lora_transpose_kernel(const bf16_t *A, int64_t a_rs, int32_t rank, int32_t K,
                                                             int32_t rpad, bf16_t *At, int64_t at_rs) {
  __shared__ bf16_t tile[32][33];
  const int k0 = blockIdx.x * 32, r0 = blockIdx.y * 32;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;   // 32 x 8
  for (int y = ty; y < 32; y += 8) {
    const int r = r0 + y, k = k0 + tx;
    tile[y][tx] = (r < rank && k < K) ? A[(int64_t)r * a_rs + k] : (bf16_t)0.f;
  }
  __syncthreads();
  for (int y = ty; y < 32; y += 8) {
    const int k = k0 + y, r = r0 + tx;
    if (k < K && r < rpad) At[(int64_t)k * at_rs + r] = tile[tx][y];
  }
}

namespace {

template <int NB>
void launch_down_nb(const LoraDownArgs &a, hipStream_t st) {
  const dim3 grid((unsigned)((a.S + 31) / 32)), block(kDownWaves * 64);
  if (a.thr > 0) hipLaunchKernelGGL((lora_down_kernel<NB, true>), grid, block, 0, st, a);
  else hipLaunchKernelGGL((lora_down_kernel<NB, false>), grid, block, 0, st, a);
}

}  // namespace

// Ranks in chunks of up to 96 (three accumulator blocks per wave); the
// dropout output is written by the first chunk only (every chunk draws the
// same bits).
void launch_lora_down(const LoraDownArgs &a, hipStream_t st) {
  for (int r0 = 0; r0 < a.rank; r0 += 96) {
    LoraDownArgs c = a;
    c.rank = a.rank - r0 < 96 ? a.rank - r0 : 96;
    c.A = reinterpret_cast<const bf16_t *>(a.A) + (int64_t)r0 * a.a_rs;
    c.t = reinterpret_cast<bf16_t *>(a.t) + r0;
    if (r0 > 0) c.h = nullptr;
    switch ((c.rank + 31) / 32) {
      case 1: launch_down_nb<1>(c, st); break;
      case 2: launch_down_nb<2>(c, st); break;
      default: launch_down_nb<3>(c, st); break;
    }
  }
}

void launch_lora_dx(const LoraDxArgs &a, hipStream_t st) {
  const dim3 grid((unsigned)((a.K + 511) / 512), (unsigned)((a.S + 31) / 32)), block(256);
  hipLaunchKernelGGL(lora_dx_kernel, grid, block, 0, st, a);
}

void launch_lora_scale_rows(const void *u, int64_t u_rs, const float *gate, float scaling, int32_t S, int32_t rank,
                            int32_t rpad, void *da, int64_t da_rs, hipStream_t st) {
  const int64_t n = (int64_t)S * rpad;
  hipLaunchKernelGGL(lora_scale_rows_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                     reinterpret_cast<const bf16_t *>(u), u_rs, gate, scaling, S, rank, rpad,
                     reinterpret_cast<bf16_t *>(da), da_rs);
}

void launch_lora_transpose(const void *A, int64_t a_rs, int32_t rank, int32_t K, int32_t rpad, void *At,
                           int64_t at_rs, hipStream_t st) {
  hipLaunchKernelGGL(lora_transpose_kernel, dim3((unsigned)((K + 31) / 32), (unsigned)(rpad / 32)), dim3(256), 0, st,
                     reinterpret_cast<const bf16_t *>(A), a_rs, rank, K, rpad, reinterpret_cast<bf16_t *>(At), at_rs);
}

}  // namespace mga
