// Gated LoRA (mtp_glora/models/layers/gated_lora.py:51-53), the parts that
// are not plain GEMMs:
//
//   out = base(x) + s * B(A(dropout(x))) * gate
//
// The plain GEMMs (x W^T, the rank-r up-projection accumulated into the
// output, dY W, and d_a^T h when the forward kept h) go to hipBLASLt
// (mga_blas.hip). The kernels here fuse what a library GEMM cannot, or stream
// what it runs far from the HBM bound:
//
// * the down-projection t = T(T(s * T(h A^T)) * gate) for every row, h =
//   dropout(x) drawn on the fly (written out only on request: the backward's
//   lora_da_kernel draws the same mask again from x).
//   HBM-bound on x; v_mfma_f32_32x32x16_bf16 with 32 rows per workgroup.
//   lora_down_ring_kernel (K a multiple of 128) streams 128-wide chunks of
//   the x rows through a ring of four LDS buffers with direct loads (1 KB per
//   instruction, three chunks ahead) and reads A's operands from a copy in
//   MFMA-operand order (lora_pack_a_kernel: one contiguous 1 KB read per
//   operand); it splits K over up to 8 workgroups per row block, whose fp32
//   partial sums lora_down_finish_kernel adds in a fixed order.
//   lora_down_kernel (other K) reads its operands straight from global
//   memory, K split over 8 waves. Operand loads that give each lane its own
//   row touch 32 cache lines per instruction; staging x through LDS and
//   packing A is what makes the first kernel faster.
// * lora_dx_kernel (dropout on): the LoRA path's input gradient
//   L = T(mask * T(scale * T(d_a A))), written to dX; the base gradient dY W
//   is then accumulated on top by hipBLASLt (beta = 1), so dX is written once
//   here and read once inside that compute-bound GEMM. The rank-r product
//   runs on MFMA. A workgroup covers 128 columns x 128 rows: the A^T tile of
//   its columns is shared through LDS, d_a goes straight into MFMA operands,
//   and each wave transposes its rounded 32 x 32 result blocks through a
//   small LDS tile so that a lane owns 8 consecutive columns of a row: dX is
//   written in 16-byte runs with one hash per element pair.
//   lora_dx_rows_kernel serves K not a multiple of 128, ranks above 128 and
//   8-byte-aligned rows: one row per lane, the output's columns along the
//   lane's registers.
// * lora_skinny_kernel: lora_B's backward products u = dY B and dB = dY^T t,
//   each one streaming pass over dY (the rank-r side staged beside it), fp32
//   split sums added in a fixed order by lora_u_finish_kernel (which also
//   forms d_a = T(T(T(u) * gate) * s)) and lora_db_finish_kernel.
// * lora_scale_rows_kernel: d_a = T(T(u * gate) * s), u = dY B, when u comes
//   from hipBLASLt (ranks above 128, unaligned rows).
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
#include <algorithm>
#include <type_traits>

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

// s_waitcnt immediate waiting for vmcnt <= n only (gfx9 encoding: vmcnt[3:0]
// in bits 3:0, vmcnt[5:4] in bits 15:14; expcnt and lgkmcnt at their maxima)
constexpr int vmcnt_imm(int n) { return (n & 0xf) | (0x7 << 4) | (0xf << 8) | ((n >> 4) << 14); }

constexpr int kDownWaves = 8;
constexpr int kDownMaxSplit = 8;   // split-K parts of the LDS down-projection (partials: 8 x S x 96 fp32)

}  // namespace

// Grid: ceil(S / 32) workgroups of 8 waves. Wave w takes the 16-wide k steps
// w, w + 8, ... of the workgroup's 32 rows; NB = ranks / 32 accumulator blocks.
// Loads are unconditional (rows past S and ranks past the rank read a clamped,
// valid address; their sums land only in outputs that are dropped or zeroed)
// and issued kU steps ahead of the MFMAs that use them.
template <int NB, bool DROP>
__global__ __launch_bounds__(kDownWaves * 64) void lora_down_kernel(LoraDownArgs a) {
  constexpr int kU = NB >= 3 ? 4 : 8;
  const int w = wave_id(), lane = threadIdx.x & 63;
  const int s0 = blockIdx.x * 32;
  const int row = s0 + (lane & 31);
  const bool row_ok = row < a.S;
  const int rowc = row_ok ? row : a.S - 1;
  const int kq = 8 * (lane >> 5);
  const bf16_t *xr = reinterpret_cast<const bf16_t *>(a.x) + (int64_t)rowc * a.x_rs + kq;
  bf16_t *hr = (DROP && a.h) ? reinterpret_cast<bf16_t *>(a.h) + (int64_t)rowc * a.h_rs + kq : nullptr;
  const bf16_t *ar[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    const int r = nb * 32 + (lane & 31);
    ar[nb] = reinterpret_cast<const bf16_t *>(a.A) + (int64_t)(r < a.rank ? r : a.rank - 1) * a.a_rs + kq;
  }
  f32x16 acc[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) acc[nb] = zero16();
  const uint64_t pair0 = ((uint64_t)rowc * (uint64_t)a.K + (uint64_t)kq) >> 1;
  const int nsteps = (a.K / 16 - w + kDownWaves - 1) / kDownWaves;   // wave-uniform

  // one k step: dropout on the x operand (h written out), then the MFMAs
  auto consume = [&](bf16x8 &xv, const bf16x8 (&av)[NB], int step) {
    if constexpr (DROP) {
      const int k0 = 16 * (w + kDownWaves * step);
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
    for (int nb = 0; nb < NB; ++nb) acc[nb] = mfma32<bf16_t>(xv, av[nb], acc[nb]);
  };
  auto load_step = [&](bf16x8 &xv, bf16x8 (&av)[NB], int step) {
    const int k0 = 16 * (w + kDownWaves * step);
    xv = load8(xr + k0);
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) av[nb] = load8(ar[nb] + k0);
  };

  // full groups of kU steps: all loads of a group issued before its MFMAs,
  // with no branch in between
  const int nfull = nsteps / kU * kU;
  for (int i = 0; i < nfull; i += kU) {
    bf16x8 xv[kU], av[kU][NB];
#pragma unroll
    for (int u = 0; u < kU; ++u) load_step(xv[u], av[u], i + u);
#pragma unroll
    for (int u = 0; u < kU; ++u) consume(xv[u], av[u], i + u);
  }
  for (int i = nfull; i < nsteps; ++i) {
    bf16x8 xv, av[NB];
    load_step(xv, av, i);
    consume(xv, av, i);
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
      const float v = r < a.rank ? rnd(rnd(acc[nb][q]) * a.scaling) * g : 0.f;
      t[(int64_t)s * a.t_rs + r] = (bf16_t)v;
    }
  }
}

// lora_A in MFMA-operand order: 1 KB block (kstep, nb) = K/16 k-steps x NB
// rank blocks, lane (l32, hi) holding A[32 nb + l32][16 kstep + 8 hi .. + 8]
// (zero past the rank), so every operand load of the down-projection below is
// one contiguous 1 KB wave read. One thread per 16-byte granule.
__global__ __launch_bounds__(256) void lora_pack_a_kernel(const bf16_t *A, int64_t a_rs, int32_t rank, int32_t K,
                                                          int32_t nb_n, i32x4 *pk) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (int64_t)(K / 16) * nb_n * 64) return;
  const int lane = (int)(i & 63);
  const int64_t blk = i >> 6;
  const int nb = (int)(blk % nb_n);
  const int64_t kstep = blk / nb_n;
  const int r = nb * 32 + (lane & 31);
  const int64_t k = kstep * 16 + 8 * (lane >> 5);
  i32x4 v = {0, 0, 0, 0};
  if (r < rank) v = *reinterpret_cast<const i32x4 *>(A + (int64_t)r * a_rs + k);
  pk[i] = v;
}

// Down-projection for K a multiple of 128 with the x rows streamed through a
// ring of four LDS buffers (direct loads, three 128-column chunks ahead) and
// lora_A's operands read straight from the packed copy (L2-resident, one 1 KB
// read per operand). Grid (ceil(S / 32), nsplit): a workgroup of 4 waves owns
// 32 rows and a contiguous share of the chunks; wave w takes k-steps 2w, 2w+1
// of every chunk, and the waves' sums are added in a fixed order at the end.
// Every wave issues the same memory instructions in every iteration (a chunk
// past the share reloads the share's last chunk into its free buffer; the
// operand loads of a chunk past the share read the last one), so the waits
// can name exact counts: the chunk's own loads, and its operands. vmcnt
// retires loads in issue order but stores out of order with them, so when
// the kernel also writes the dropout output it waits for everything instead.
template <int NB, bool DROP, bool WRITE_H>
__global__ __launch_bounds__(256) void lora_down_ring_kernel(LoraDownArgs a) {
  constexpr int HD = 128, NRA = 32 * NB, RING = 4, TILE = 32 * HD;
  // per-iteration vector-memory loads of a wave after its chunk loads: the
  // next chunk's operands (2 NB)
  constexpr int kOps = 2 * NB;
  __shared__ __attribute__((aligned(16))) bf16_t sX[RING * TILE];
  const int w = wave_id(), lane = threadIdx.x & 63;
  const int l32 = lane & 31, hi = lane >> 5;
  const int s0 = blockIdx.x * 32;
  const int row = s0 + l32;
  const bool row_ok = row < a.S;
  const int nrows = a.S - s0 < 32 ? a.S - s0 : 32;
  const bf16_t *xb = reinterpret_cast<const bf16_t *>(a.x) + (int64_t)s0 * a.x_rs;
  const i32x4 *pk = reinterpret_cast<const i32x4 *>(a.packed);
  DmaLane<HD, 32> dx;
  dx.init();
  const uint32_t lrx = dx.lane_row(a.x_rs);
  const auto rowsx = dx.rows(a.x_rs);
  const uint32_t orow = opaque_u32((uint32_t)(l32 * HD + (((uint32_t)hi ^ swz<HD>(l32)) << 3)) * 2u);
  bf16_t *hr = WRITE_H ? reinterpret_cast<bf16_t *>(a.h) + (int64_t)(row_ok ? row : 0) * a.h_rs : nullptr;
  const uint64_t prow = (uint64_t)(row_ok ? row : 0) * (uint64_t)a.K;
  const int nall = a.K / HD;
  const int cbeg = (int)((int64_t)nall * blockIdx.y / gridDim.y);
  const int nchunks = (int)((int64_t)nall * (blockIdx.y + 1) / gridDim.y) - cbeg;

  auto issue = [&](int c) {   // chunk c of the share into buffer c % RING (past the share: its last chunk)
    const int col = (cbeg + min(c, nchunks - 1)) * HD;
    bf16_t *tx = sX + (c % RING) * TILE;
    if (nrows == 32) dx.issue(tx, xb + col, rowsx, lrx);
    else dx.issue_clamped(tx, xb + col, a.x_rs, nrows);
  };
  auto load_ops = [&](int c, bf16x8 (&op)[2][NB]) {
    const int64_t kstep0 = (int64_t)(cbeg + min(c, nchunks - 1)) * (HD / 16) + 2 * w;
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
        op[j][nb] = __builtin_bit_cast(bf16x8, pk[((kstep0 + j) * NB + nb) * 64 + lane]);
  };

  f32x16 acc[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) acc[nb] = zero16();
  // operands of the current / next chunk in two named register sets that
  // swap roles each iteration (the loop runs two chunks per trip)
  bf16x8 opa[2][NB], opb[2][NB];
  auto chunk = [&](int c, bf16x8 (&opc)[2][NB], bf16x8 (&opn)[2][NB]) {
    // this wave's loads of chunk c have landed (the first iterations wait for
    // everything). vmcnt counts in issue order only while no store is in
    // flight, so with the dropout output written here the wait is a full one.
    if (c >= RING - 1 && !WRITE_H) __builtin_amdgcn_s_waitcnt(vmcnt_imm(3 * kOps + 4));
    else __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
    // every wave's part of chunk c is in; chunk c - 1's buffer is free. A bare
    // barrier between compiler fences: __syncthreads' memory fence would make
    // the compiler wait for every load in flight, the ring's included.
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    issue(c + RING - 1);
    // the operands of chunk c (issued before the two loads just above)
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(2));
    const uint32_t ob = orow + (uint32_t)((c % RING) * TILE * 2);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int ks = 2 * w + j;
      bf16x8 xv = lds_read8(reinterpret_cast<const bf16_t *>(lds_at(sX, ob ^ (uint32_t)(ks << 5))));
      if constexpr (DROP) {
        const int k0 = (cbeg + c) * HD + ks * 16 + 8 * hi;
        const uint64_t pj = (prow + (uint64_t)k0) >> 1;
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
          const uint32_t bits = pair_bits(a.seed, pj + (e >> 1));
          const bool k_lo = (bits & 0xffffu) >= a.thr, k_hi = (bits >> 16) >= a.thr;
          xv[e] = k_lo ? (bf16_t)((float)xv[e] * a.keep_scale) : (bf16_t)0.f;
          xv[e + 1] = k_hi ? (bf16_t)((float)xv[e + 1] * a.keep_scale) : (bf16_t)0.f;
        }
        // one store instruction per k-step (lanes of rows past S masked off;
        // a wave always has a row below S, so the store is never skipped)
        if constexpr (WRITE_H)
          if (row_ok) *reinterpret_cast<i32x4 *>(hr + k0) = __builtin_bit_cast(i32x4, xv);
      }
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) acc[nb] = mfma32<bf16_t>(xv, opc[j][nb], acc[nb]);
    }
    load_ops(c + 1, opn);
  };

  issue(0);
  issue(1);
  issue(2);
  load_ops(0, opa);
  for (int c = 0; c < nchunks; c += 2) {
    chunk(c, opa, opb);
    if (c + 1 < nchunks) chunk(c + 1, opb, opa);
  }
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));   // the ring's trailing loads
  __syncthreads();

  // fixed-order reduction through the ring, one rank block at a time
  float *park = reinterpret_cast<float *>(sX);
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    if (w > 0)
#pragma unroll
      for (int q = 0; q < 16; ++q) park[((w - 1) * 16 + q) * 64 + lane] = acc[nb][q];
    __syncthreads();
    if (w == 0)
#pragma unroll
      for (int q = 0; q < 16; ++q) {
        const int o = q * 64 + lane;
        acc[nb][q] += park[o] + park[16 * 64 + o] + park[32 * 64 + o];
      }
    __syncthreads();
  }
  if (w != 0) return;
  if (gridDim.y > 1) {   // fp32 partial sums [split][S][32 NB]; lora_down_finish_kernel adds them
    float *part = a.part + (int64_t)blockIdx.y * a.S * NRA;
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      const int s = s0 + 8 * (q >> 2) + 4 * hi + (q & 3);
      if (s >= a.S) continue;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) part[(int64_t)s * NRA + nb * 32 + l32] = acc[nb][q];
    }
    return;
  }
  bf16_t *t = reinterpret_cast<bf16_t *>(a.t);
#pragma unroll
  for (int q = 0; q < 16; ++q) {
    const int s = s0 + 8 * (q >> 2) + 4 * hi + (q & 3);
    if (s >= a.S) continue;
    const float g = a.gate ? a.gate[s] : 1.f;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      const int r = nb * 32 + l32;
      const float v = r < a.rank ? rnd(rnd(acc[nb][q]) * a.scaling) * g : 0.f;
      t[(int64_t)s * a.t_rs + r] = (bf16_t)v;
    }
  }
}

// t[s][r] = T(T(s * T(sum over the splits, in order)) * gate) from the partial
// sums of the split-K down-projection (ranks nr = 32 NB of this launch).
__global__ __launch_bounds__(256) void lora_down_finish_kernel(LoraDownArgs a, int nsplit, int nr) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)a.S * nr) return;
  const int s = (int)(i / nr), r = (int)(i - (int64_t)s * nr);
  float v = 0.f;
  for (int k = 0; k < nsplit; ++k) v += a.part[(int64_t)k * a.S * nr + i];
  const float g = a.gate ? a.gate[s] : 1.f;
  const float out = r < a.rank ? rnd(rnd(v) * a.scaling) * g : 0.f;
  reinterpret_cast<bf16_t *>(a.t)[(int64_t)s * a.t_rs + r] = (bf16_t)out;
}

// Grid: (K / 128, ceil(S / 128)), 4 waves. The workgroup's 128 columns of
// A^T (rank-padded rows) are copied once into LDS and shared; wave w computes
// rows 32 w .. 32 w + 31 of the 128-row block, one 32 x 32 block at a time:
// D[s][k] = sum_r d_a[s][r] A^T[k][r] (A operand: the lane's d_a row from
// global memory; B operand: the A^T row of the lane's column, from LDS). The
// rounded block T(D) goes through a per-wave LDS tile so that each lane then
// owns 8 consecutive columns of one row: dX is written with 16-byte stores
// and each dropout hash serves its element pair. NK = 16-rank steps of the
// padded rank (even).
template <int NK>
__global__ __launch_bounds__(256) void lora_dx_kernel(LoraDxArgs a) {
  constexpr int RP = NK * 16;          // padded rank
  constexpr int LS = RP + 8;           // LDS row stride of A^T (elements)
  constexpr int TS = 40;               // row stride of a wave's 32 x 32 result tile (80 bytes)
  __shared__ __attribute__((aligned(16))) bf16_t sAt[128 * LS];
  __shared__ __attribute__((aligned(16))) bf16_t sT[4][32 * TS];
  const int w = wave_id(), lane = threadIdx.x & 63, tid = threadIdx.x;
  const int l32 = lane & 31, hi = lane >> 5;
  const int kb0 = blockIdx.x * 128;
  const int s0 = blockIdx.y * 128 + w * 32;
  {
    // every granule load issued before the first LDS write (one memory wait)
    constexpr int kGran = RP / 8;      // 16-byte granules per row
    constexpr int kPer = 128 * kGran / 256;
    const bf16_t *src = reinterpret_cast<const bf16_t *>(a.At) + (int64_t)kb0 * a.at_rs;
    i32x4 g16[kPer];
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int i = tid + 256 * j, r = i / kGran, g = i - r * kGran;
      g16[j] = *reinterpret_cast<const i32x4 *>(src + (int64_t)r * a.at_rs + g * 8);
    }
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int i = tid + 256 * j, r = i / kGran, g = i - r * kGran;
      *reinterpret_cast<i32x4 *>(sAt + r * LS + g * 8) = g16[j];
    }
  }
  const int srow = s0 + l32 < a.S ? s0 + l32 : a.S - 1;   // rows past S: computed, never stored
  const bf16_t *dar = reinterpret_cast<const bf16_t *>(a.da) + (int64_t)srow * a.da_rs + 8 * hi;
  bf16x8 dv[NK];
#pragma unroll
  for (int j = 0; j < NK; ++j) dv[j] = load8(dar + 16 * j);
  // epilogue ownership: lane -> row er (+16 for the second half), columns ec .. ec + 7
  const int er = lane >> 2, ec = (lane & 3) * 8;
  bf16_t *dx = reinterpret_cast<bf16_t *>(a.dx);
  bf16_t *tile = sT[w];
  auto dx_at = [&](int r, int blk) {
    const int s = s0 + r;
    return dx + (int64_t)(s < a.S ? s : a.S - 1) * a.dx_rs + kb0 + blk * 32 + ec;
  };
  __syncthreads();
#pragma unroll
  for (int blk = 0; blk < 4; ++blk) {
    f32x16 acc = zero16();
    const bf16_t *brow = sAt + (blk * 32 + l32) * LS + 8 * hi;
#pragma unroll
    for (int j = 0; j < NK; ++j) acc = mfma32<bf16_t>(dv[j], lds_read8(brow + 16 * j), acc);
    // d(dropout(x)) = T(d_a A): lane holds column l32 of rows 8 (q / 4) + 4 hi + q % 4
#pragma unroll
    for (int q = 0; q < 16; ++q) tile[(8 * (q >> 2) + 4 * hi + (q & 3)) * TS + l32] = (bf16_t)acc[q];
    __builtin_amdgcn_s_waitcnt(0xc07f);   // lgkmcnt(0): this wave's tile writes done
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int r = er + 16 * h, s = s0 + r;
      const bf16x8 dh = lds_read8(tile + r * TS + ec);
      if (s < a.S) {
        const int k = kb0 + blk * 32 + ec;
        const uint64_t pj = ((uint64_t)s * (uint64_t)a.K + (uint64_t)k) >> 1;
        bf16x8 o;
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
          const uint32_t bits = pair_bits(a.seed, pj + (e >> 1));
          const bool k_lo = (bits & 0xffffu) >= a.thr, k_hi = (bits >> 16) >= a.thr;
          o[e] = (bf16_t)(k_lo ? (float)dh[e] * a.keep_scale : 0.f);           // dropout backward
          o[e + 1] = (bf16_t)(k_hi ? (float)dh[e + 1] * a.keep_scale : 0.f);
        }
        *reinterpret_cast<i32x4 *>(dx_at(r, blk)) = __builtin_bit_cast(i32x4, o);
      }
    }
    __builtin_amdgcn_wave_barrier();   // the tile is rewritten by the next block
  }
}

// General variant (any K multiple of 16, any rank). Grid: (ceil(K / 512),
// ceil(S / 32)), 4 waves; wave w covers 32 rows x 128 columns of dX. D^T[k][s] = sum_r A^T[k][r] d_a[s][r]; each lane holds one
// row s and four runs of four consecutive columns per 32-column block. Every
// load (its d_a row, the A^T rows of its four blocks) is issued before the
// first MFMA when the rank is at most 16 NK (larger ranks go in chunks of NK
// steps). d_a and A^T are zero-padded to a multiple of 32
// ranks, so the step count is even.
template <int NK>
__global__ __launch_bounds__(256) void lora_dx_rows_kernel(LoraDxArgs a) {
  const int w = wave_id(), lane = threadIdx.x & 63;
  const int l32 = lane & 31, hi = lane >> 5;
  const int s = blockIdx.y * 32 + l32;
  const bool s_ok = s < a.S;
  const int sc = s_ok ? s : a.S - 1;     // clamped rows: their sums are never stored
  const int rq = 8 * hi;
  const int kb0 = blockIdx.x * 512 + w * 128;
  bf16_t *dxr = reinterpret_cast<bf16_t *>(a.dx) + (int64_t)sc * a.dx_rs;
  const bf16_t *dar = reinterpret_cast<const bf16_t *>(a.da) + (int64_t)sc * a.da_rs + rq;
  const bf16_t *atr[4];
#pragma unroll
  for (int blk = 0; blk < 4; ++blk) {
    const int kr = kb0 + blk * 32 + l32;
    atr[blk] = reinterpret_cast<const bf16_t *>(a.At) + (int64_t)(kr < a.K ? kr : a.K - 1) * a.at_rs + rq;
  }
  f32x16 acc[4];
#pragma unroll
  for (int blk = 0; blk < 4; ++blk) acc[blk] = zero16();
  // ranks in chunks of NK steps (one chunk when the rank is at most 16 NK)
  const int nsteps = (a.rank + 31) / 32 * 2;
  for (int j0 = 0; j0 < nsteps; j0 += NK) {
    bf16x8 dv[NK], av[4][NK];
#pragma unroll
    for (int j = 0; j < NK; ++j) dv[j] = load8(dar + 16 * (j0 + j));
#pragma unroll
    for (int blk = 0; blk < 4; ++blk)
#pragma unroll
      for (int j = 0; j < NK; ++j) av[blk][j] = load8(atr[blk] + 16 * (j0 + j));
#pragma unroll
    for (int blk = 0; blk < 4; ++blk)
#pragma unroll
      for (int j = 0; j < NK; ++j) acc[blk] = mfma32<bf16_t>(av[blk][j], dv[j], acc[blk]);
  }
#pragma unroll
  for (int blk = 0; blk < 4; ++blk) {
    const int kbase = kb0 + blk * 32;
    if (!s_ok || kbase >= a.K) continue;
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      const int k = kbase + 8 * g4 + 4 * hi;
      if (k >= a.K) continue;
      const uint64_t pj = ((uint64_t)s * (uint64_t)a.K + (uint64_t)k) >> 1;
      const uint32_t b0 = pair_bits(a.seed, pj), b1 = pair_bits(a.seed, pj + 1);
      const bool keep[4] = {(b0 & 0xffffu) >= a.thr, (b0 >> 16) >= a.thr, (b1 & 0xffffu) >= a.thr,
                            (b1 >> 16) >= a.thr};
      bf16x4 o;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float dh = rnd(acc[blk][4 * g4 + e]);                 // d(dropout(x)) = T(d_a A)
        o[e] = (bf16_t)(keep[e] ? dh * a.keep_scale : 0.f);         // dropout backward
      }
      *reinterpret_cast<bf16x4 *>(dxr + k) = o;
    }
  }
}

// grad_A = d_a^T dropout(x) with the dropout drawn again from x (so the
// forward need not keep its dropout output): K a multiple of 128, ranks in
// launches of up to 128. Grid (K / 128, nsplit): a workgroup owns 128
// columns and a share of the rows, 32 at a time. Each step stages the rows'
// dropout(x) (one hash per element pair, as in the forward) and their d_a
// through registers into LDS (double-buffered), and wave w accumulates
// D[r][k] = sum_s d_a[s][r] h[s][k] for its 32 columns and every rank block,
// both MFMA operands read with the transposed LDS read (lane = r or k,
// 8 consecutive rows s). Split partial sums go to fp32 [split][r][k] and
// lora_da_finish_kernel adds them in a fixed order.
template <int NB>
__global__ __launch_bounds__(256) void lora_da_kernel(LoraDaArgs a, int r0) {
  constexpr int HD = 128, TILE = 32 * HD;
  __shared__ __attribute__((aligned(16))) bf16_t sX0[TILE], sX1[TILE], sD0[TILE], sD1[TILE];
  const int w = wave_id(), tid = threadIdx.x, lane = tid & 63;
  const int l32 = lane & 31, hi = lane >> 5;
  const int kc0 = blockIdx.x * HD;
  const int nst = (a.S + 31) / 32;
  const int st0 = (int)((int64_t)nst * blockIdx.y / gridDim.y);
  const int st1 = (int)((int64_t)nst * (blockIdx.y + 1) / gridDim.y);
  const int rc = min(a.rank - r0, 32 * NB);   // ranks of this launch
  const bf16_t *xb = reinterpret_cast<const bf16_t *>(a.x);
  const bf16_t *db = reinterpret_cast<const bf16_t *>(a.da) + r0;
  TrOffsets<HD> tro;
  tro.init(lane);
  // staged granules of one step: x 2 per thread, d_a NB / 2 per thread (rounded up)
  constexpr int kDG = (32 * NB * 4 + 255) / 256;
  i32x4 gx[2], gd[kDG];
  auto load = [&](int st) {
    const int s0 = st * 32;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int gi = tid + 256 * i, r = gi >> 4, g = gi & 15;
      const int s = s0 + r;
      const i32x4 v = *reinterpret_cast<const i32x4 *>(xb + (int64_t)min(s, a.S - 1) * a.x_rs + kc0 + 8 * g);
      bf16x8 h = __builtin_bit_cast(bf16x8, v);
      const uint64_t pj = ((uint64_t)min(s, a.S - 1) * (uint64_t)a.K + (uint64_t)(kc0 + 8 * g)) >> 1;
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        const uint32_t bits = pair_bits(a.seed, pj + (e >> 1));
        const bool k_lo = s < a.S && (bits & 0xffffu) >= a.thr, k_hi = s < a.S && (bits >> 16) >= a.thr;
        h[e] = k_lo ? (bf16_t)((float)h[e] * a.keep_scale) : (bf16_t)0.f;
        h[e + 1] = k_hi ? (bf16_t)((float)h[e + 1] * a.keep_scale) : (bf16_t)0.f;
      }
      gx[i] = __builtin_bit_cast(i32x4, h);
    }
#pragma unroll
    for (int i = 0; i < kDG; ++i) {
      const int gi = tid + 256 * i, r = gi / (4 * NB), g = gi % (4 * NB);
      const int s = s0 + r;
      i32x4 v = {0, 0, 0, 0};
      if (gi < 32 * 4 * NB && s < a.S) v = *reinterpret_cast<const i32x4 *>(db + (int64_t)s * a.da_rs + 8 * g);
      gd[i] = v;
    }
  };
  auto store = [&](bf16_t *tx, bf16_t *td) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int gi = tid + 256 * i;
      *reinterpret_cast<i32x4 *>(tx + tile_off<HD>(gi >> 4, gi & 15)) = gx[i];
    }
#pragma unroll
    for (int i = 0; i < kDG; ++i) {
      const int gi = tid + 256 * i;
      if (gi < 32 * 4 * NB) *reinterpret_cast<i32x4 *>(td + tile_off<HD>(gi / (4 * NB), gi % (4 * NB))) = gd[i];
    }
  };
  f32x16 acc[NB];
#pragma unroll
  for (int rb = 0; rb < NB; ++rb) acc[rb] = zero16();
  auto step = [&](auto bsel, int st) {
    constexpr int B = decltype(bsel)::value;
    const bf16_t *tx = B ? sX1 : sX0;
    const bf16_t *td = B ? sD1 : sD0;
    if (st + 1 < st1) load(st + 1);
#pragma unroll
    for (int ss = 0; ss < 2; ++ss) {
      const bf16x8 hb = tro.operand(tx, 16 * ss, w);
#pragma unroll
      for (int rb = 0; rb < NB; ++rb) acc[rb] = mfma32<bf16_t>(tro.operand(td, 16 * ss, rb), hb, acc[rb]);
    }
    if (st + 1 < st1) store(B ? sX0 : sX1, B ? sD0 : sD1);
    __syncthreads();
  };
  if (st0 < st1) {
    load(st0);
    store(sX0, sD0);
  }
  __syncthreads();
  for (int st = st0; st < st1; st += 2) {
    step(std::integral_constant<int, 0>{}, st);
    if (st + 1 < st1) step(std::integral_constant<int, 1>{}, st + 1);
  }
  // lane holds column kc0 + 32 w + l32 of rows 8 (q / 4) + 4 hi + q % 4 of each rank block
  const int k = kc0 + 32 * w + l32;
  const int rp = (a.rank + 31) / 32 * 32;
#pragma unroll
  for (int rb = 0; rb < NB; ++rb)
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      const int r = 32 * rb + 8 * (q >> 2) + 4 * hi + (q & 3);
      if (r >= rc) continue;
      if (gridDim.y > 1)
        a.part[((int64_t)blockIdx.y * rp + r0 + r) * a.K + k] = acc[rb][q];
      else
        reinterpret_cast<bf16_t *>(a.dA)[(int64_t)(r0 + r) * a.dA_rs + k] = (bf16_t)acc[rb][q];
    }
}

// grad_A[r][k] = T(sum over the splits, in order) of lora_da_kernel's partials.
__global__ __launch_bounds__(256) void lora_da_finish_kernel(LoraDaArgs a, int nsplit) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)a.rank * a.K) return;
  const int r = (int)(i / a.K), k = (int)(i - (int64_t)r * a.K);
  const int rp = (a.rank + 31) / 32 * 32;
  float v = 0.f;
  for (int y = 0; y < nsplit; ++y) v += a.part[((int64_t)y * rp + r) * a.K + k];
  reinterpret_cast<bf16_t *>(a.dA)[(int64_t)r * a.dA_rs + k] = (bf16_t)v;
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


// ---- lora_B's backward: the two skinny products over the streamed dY -------
// MODE 0: dB^T partials   part[split][n][r] = sum over the split's rows s of dY[s][n] t[s][r]
// MODE 1: u^T partials    part[split][s][r] = sum over the split's columns n of dY[s][n] B[n][r]
// HBM-bound on dY (each element read once per product). A workgroup of 4
// waves owns 64 output lines (columns n for MODE 0, rows s for MODE 1) and a
// share of the 64-wide chunks of the reduced dimension. Each chunk stages a
// 64 x 64 dY tile (rows s, columns n, swizzled) and the chunk's 64 rows of the
// small matrix (t for MODE 0, B for MODE 1) as compact rows of RP = 32 RB
// elements, in a ring of four named buffers (three chunks ahead) filled with
// direct loads. Every wave issues the same loads per chunk, and every load in
// flight is a direct load, so the waits name exact counts. Wave w takes
// k-step w (16 of the 64) of every chunk for all (rank block, line block)
// outputs:
//   MODE 0: dB^T[r][n] += t^T[r][s] dY[s][n]      A: t^T, B: dY  (transposed LDS reads)
//   MODE 1: u^T[r][s]  += B^T[r][n] dY^T[n][s]    A: B^T (transposed read), B: dY rows (8-byte reads)
// so a lane holds one output line and 16 ranks of each rank block, written
// as 16-byte runs. The waves' sums are added in a fixed order at the end.
// Rank columns past the rank and lines past the end hold junk that no
// finishing kernel reads; reduced-dimension entries past the end are zeroed
// in an operand. CLAMP (S or N not a multiple of 64) clamps each lane's rows
// and columns at the edges; without it every address is a wave-uniform base
// plus a loop-invariant lane offset, which also keeps the compiler from
// waiting on loads in flight whose address registers a later read would reuse.
template <int MODE, int RB, bool CLAMP>
__device__ __forceinline__ void lora_skinny_body(const LoraSkinnyArgs &a) {
  constexpr int RP = 32 * RB;                 // compact small-tile row (elements)
  constexpr int YT = 64 * 64, MT = 64 * RP;
  constexpr int MG = RP / 8;                  // granules per small-tile row
  constexpr int MI = 64 * MG / 256;           // small-tile loads per thread (1 .. 4)
  constexpr int NL = 2 + MI;                  // loads per thread per chunk
  __shared__ __attribute__((aligned(16))) bf16_t sY0[YT], sY1[YT], sY2[YT], sY3[YT];
  __shared__ __attribute__((aligned(16))) bf16_t sM0[MT], sM1[MT], sM2[MT], sM3[MT];
  const int w = wave_id(), tid = threadIdx.x, lane = tid & 63;
  const int l32 = lane & 31, hi = lane >> 5;
  const int line0 = blockIdx.x * 64;
  const int nlines = MODE == 0 ? a.N : a.S;   // output lines
  const int kdim = MODE == 0 ? a.S : a.N;     // reduced dimension
  const int nall = (kdim + 63) / 64;
  const int c0 = (int)((int64_t)nall * blockIdx.y / gridDim.y);
  const int nch = (int)((int64_t)nall * (blockIdx.y + 1) / gridDim.y) - c0;
  const bf16_t *dy = reinterpret_cast<const bf16_t *>(a.dy);
  const bf16_t *sm = reinterpret_cast<const bf16_t *>(a.sm);
  // granules of a small-matrix row that hold rank columns (a slot past them
  // reads the last one again: its columns are never used)
  const int mg_last = (a.rank + 7) / 8 - 1;

  // Per-lane sources. dY tile: 8 granules per row, 8 rows per load, wave w
  // loads rows 16 w .. 16 w + 15 (two loads). Small tile: MG granules per row,
  // load i of thread t fills slot 256 i + t (row slot / MG, granule slot % MG).
  const int yp = lane & 7, yr = lane >> 3;
  int mrow[MI], mgr[MI];
#pragma unroll
  for (int i = 0; i < MI; ++i) {
    const int slot = 256 * i + tid;
    mrow[i] = slot / MG;
    mgr[i] = min(slot % MG, mg_last);
  }
  // full chunks: a wave-uniform base plus these 32-bit lane offsets (bytes)
  uint32_t yo[2], mo[MI];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int r = 16 * w + 8 * i + yr;
    yo[i] = opaque_u32((uint32_t)((r * a.dy_rs + 8 * (yp ^ swz<64>(r))) * 2));
  }
#pragma unroll
  for (int i = 0; i < MI; ++i) mo[i] = opaque_u32((uint32_t)((mrow[i] * a.sm_rs + 8 * mgr[i]) * 2));
  // Workgroups start their share at different chunks (rotated by the line
  // block), so that the many workgroups streaming the same share at the same
  // time do not all read the same rows of the small matrix at once.
  const int rot = blockIdx.x % nch;
  auto chunk_of = [&](int c) { const int r = c + rot; return c0 + (r >= nch ? r - nch : r); };
  auto issue = [&](int c, bf16_t *tY, bf16_t *tM) {
    const int cc = chunk_of(min(c, nch - 1));   // past the share: the share's last chunk again
    const int k0 = cc * 64;
    const int yrow0 = MODE == 0 ? k0 : line0, ycol0 = MODE == 0 ? line0 : k0;
    bf16_t *dY = tY + 16 * w * 64;
    if (!CLAMP || (yrow0 + 64 <= a.S && ycol0 + 64 <= a.N)) {
      const char *b = reinterpret_cast<const char *>(dy + (int64_t)yrow0 * a.dy_rs + ycol0);
#pragma unroll
      for (int i = 0; i < 2; ++i) __builtin_amdgcn_global_load_lds(b + yo[i], (lds_void *)(dY + 8 * i * 64), 16, 0, 0);
    } else {   // rows past S repeat the last row, columns past N the last granule
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int r = 16 * w + 8 * i + yr;
        const int g = yp ^ swz<64>(r);
        const int srow = min(yrow0 + r, a.S - 1), ncol = min(ycol0 + 8 * g, a.N - 8);
        __builtin_amdgcn_global_load_lds(dy + (int64_t)srow * a.dy_rs + ncol, (lds_void *)(dY + 8 * i * 64), 16, 0, 0);
      }
    }
    if (!CLAMP || k0 + 64 <= kdim) {
      const char *b = reinterpret_cast<const char *>(sm + (int64_t)k0 * a.sm_rs);
#pragma unroll
      for (int i = 0; i < MI; ++i)
        __builtin_amdgcn_global_load_lds(b + mo[i], (lds_void *)(tM + 2048 * i + 512 * w), 16, 0, 0);
    } else {
#pragma unroll
      for (int i = 0; i < MI; ++i)
        __builtin_amdgcn_global_load_lds(sm + (int64_t)min(k0 + mrow[i], kdim - 1) * a.sm_rs + 8 * mgr[i],
                                         (lds_void *)(tM + 2048 * i + 512 * w), 16, 0, 0);
    }
  };

  // A operand from a compact k-major tile (rows k, RP columns): lane (l32, hi)
  // takes column 32 rb + l32 at rows k0 + 4 hi + 0..3 and k0 + 8 + 4 hi + 0..3
  // (the k order of TrLane), by two transposed reads
  const int ti = lane & 15;
  const uint32_t mro[2] = {
      opaque_u32((uint32_t)(((4 * hi + (ti >> 2)) * RP + 16 * ((lane >> 4) & 1) + 4 * (ti & 3)) * 2)),
      opaque_u32((uint32_t)(((8 + 4 * hi + (ti >> 2)) * RP + 16 * ((lane >> 4) & 1) + 4 * (ti & 3)) * 2))};
  auto m_operand = [&](const bf16_t *tM, int k0, int rb) {
    const char *b = reinterpret_cast<const char *>(tM) + (k0 * RP + 32 * rb) * 2;
    return join8(lds_tr4(reinterpret_cast<const bf16_t *>(b + mro[0])),
                 lds_tr4(reinterpret_cast<const bf16_t *>(b + mro[1])));
  };
  TrOffsets<64> try_;
  try_.init(lane);
  f32x16 acc[RB][2];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) acc[rb][0] = acc[rb][1] = zero16();

  auto compute = [&](int c, const bf16_t *tY, const bf16_t *tM) {
    const int kb = chunk_of(c) * 64 + 16 * w;        // first reduced index of this wave's k-step
    const bool tail = CLAMP && kb + 16 > kdim;
    bf16x8 av[RB], bv[2];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) av[rb] = m_operand(tM, 16 * w, rb);
    if (MODE == 0) {
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) bv[nb] = try_.operand(tY, 16 * w, nb);
    } else {
      // dY row 32 sb + l32, columns 16 w + 4 hi + 0..3 and 16 w + 8 + 4 hi + 0..3
#pragma unroll
      for (int sb = 0; sb < 2; ++sb) {
        const int r = 32 * sb + l32;
        const i32x2 x = *reinterpret_cast<const i32x2 *>(tY + tile_off<64>(r, 2 * w) + 4 * hi);
        const i32x2 y = *reinterpret_cast<const i32x2 *>(tY + tile_off<64>(r, 2 * w + 1) + 4 * hi);
        const i32x4 v = {x[0], x[1], y[0], y[1]};
        bv[sb] = __builtin_bit_cast(bf16x8, v);
      }
    }
    if (tail) {   // reduced entries kb + 4 hi + e and kb + 8 + 4 hi + e past the end are zeroed
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const bool out = kb + 4 * hi + (e & 3) + 8 * (e >> 2) >= kdim;
        if (MODE == 0) {
#pragma unroll
          for (int rb = 0; rb < RB; ++rb) av[rb][e] = out ? (bf16_t)0.f : av[rb][e];
        } else {
#pragma unroll
          for (int sb = 0; sb < 2; ++sb) bv[sb][e] = out ? (bf16_t)0.f : bv[sb][e];
        }
      }
    }
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int lb = 0; lb < 2; ++lb) acc[rb][lb] = mfma32<bf16_t>(av[rb], bv[lb], acc[rb][lb]);
  };

  // chunk c: its loads landed (the next two chunks' loads may still be in
  // flight), a bare barrier (every wave's part is in, and the buffer of chunk
  // c - 1 is free), then the loads of chunk c + 3 and the products of chunk c
  // (every iteration runs all four chunks, those past the share without
  // products, so the loads in flight at the loop head are the same on every
  // path and the compiler adds no wait of its own)
  auto chunk = [&](auto bsel, int c) {
    constexpr int B = decltype(bsel)::value;
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(2 * NL));
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    issue(c + 3, B == 0 ? sY3 : (B == 1 ? sY0 : (B == 2 ? sY1 : sY2)),
          B == 0 ? sM3 : (B == 1 ? sM0 : (B == 2 ? sM1 : sM2)));
    if (c < nch)
      compute(c, B == 0 ? sY0 : (B == 1 ? sY1 : (B == 2 ? sY2 : sY3)),
              B == 0 ? sM0 : (B == 1 ? sM1 : (B == 2 ? sM2 : sM3)));
  };
  issue(0, sY0, sM0);
  issue(1, sY1, sM1);
  issue(2, sY2, sM2);
  for (int c = 0; c < nch; c += 4) {
    chunk(std::integral_constant<int, 0>{}, c);
    chunk(std::integral_constant<int, 1>{}, c + 1);
    chunk(std::integral_constant<int, 2>{}, c + 2);
    chunk(std::integral_constant<int, 3>{}, c + 3);
  }
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));   // the ring's trailing loads
  __syncthreads();

  // fixed-order sum of the waves' accumulators through LDS (the ring's dY
  // buffers, 3 x 16 x 64 floats), then this split's partial: lane = line
  // 32 lb + l32, registers = ranks 32 rb + 8 (q / 4) + 4 hi + q % 4
  float *park = reinterpret_cast<float *>(sY0);
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int lb = 0; lb < 2; ++lb) {
      if (w > 0)
#pragma unroll
        for (int q = 0; q < 16; ++q) park[((w - 1) * 16 + q) * 64 + lane] = acc[rb][lb][q];
      __syncthreads();
      if (w == 0) {
#pragma unroll
        for (int v = 0; v < 3; ++v)
#pragma unroll
          for (int q = 0; q < 16; ++q) acc[rb][lb][q] += park[(v * 16 + q) * 64 + lane];
        const int line = line0 + 32 * lb + l32;
        if (line < nlines) {
          float *out = a.part + ((int64_t)blockIdx.y * nlines + line) * a.rp + 32 * rb + 4 * hi;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const f32x4 v = {acc[rb][lb][4 * i], acc[rb][lb][4 * i + 1], acc[rb][lb][4 * i + 2],
                             acc[rb][lb][4 * i + 3]};
            *reinterpret_cast<f32x4 *>(out + 8 * i) = v;
          }
        }
      }
      __syncthreads();
    }
}

template <int MODE, int RB>
__global__ __launch_bounds__(256, 2) void lora_skinny_kernel(LoraSkinnyArgs a) {
  lora_skinny_body<MODE, RB, false>(a);
}
template <int MODE, int RB>
__global__ __launch_bounds__(256, 2) void lora_skinny_clamp_kernel(LoraSkinnyArgs a) {
  lora_skinny_body<MODE, RB, true>(a);
}

// dB[n][r] = T(sum over the splits, in order), r < rank.
__global__ __launch_bounds__(256) void lora_db_finish_kernel(LoraSkinnyArgs a, int nsplit, bf16_t *db, int64_t db_rs) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)a.N * a.rank) return;
  const int n = (int)(i / a.rank), r = (int)(i - (int64_t)n * a.rank);
  float v = 0.f;
  for (int y = 0; y < nsplit; ++y) v += a.part[((int64_t)y * a.N + n) * a.rp + r];
  db[(int64_t)n * db_rs + r] = (bf16_t)v;
}

// d_a[s][r] = T(T(T(u) * gate[s]) * scaling), u = the sum over the splits in
// order; 0 for rank <= r < rpad. The roundings of the chain dY B (bf16), then
// lora_scale_rows.
__global__ __launch_bounds__(256) void lora_u_finish_kernel(LoraSkinnyArgs a, int nsplit, const float *gate,
                                                            float scaling, bf16_t *da, int64_t da_rs) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)a.S * a.rp) return;
  const int s = (int)(i / a.rp), r = (int)(i - (int64_t)s * a.rp);
  float v = 0.f;
  if (r < a.rank) {
    for (int y = 0; y < nsplit; ++y) v += a.part[((int64_t)y * a.S + s) * a.rp + r];
    const float g = gate ? gate[s] : 1.f;
    v = rnd(rnd(rnd(v) * g) * scaling);
  }
  da[(int64_t)s * da_rs + r] = (bf16_t)v;
}

namespace {

template <int NB>
void launch_down_nb(const LoraDownArgs &a, hipStream_t st) {
  const dim3 grid((unsigned)((a.S + 31) / 32));
  if (a.K % 128 == 0 && a.packed) {
    // lora_A into operand order, then the ring kernel; split K until every CU
    // has about two workgroups, each keeping at least four chunks
    const int64_t ng = (int64_t)(a.K / 16) * NB * 64;
    hipLaunchKernelGGL(lora_pack_a_kernel, dim3((unsigned)((ng + 255) / 256)), dim3(256), 0, st,
                       reinterpret_cast<const bf16_t *>(a.A), a.a_rs, a.rank, a.K, NB,
                       reinterpret_cast<i32x4 *>(a.packed));
    const int nrb = (a.S + 31) / 32, nch = a.K / 128;
    int nsplit = 1;
    if (a.part)
      while (nsplit < kDownMaxSplit && nrb * nsplit < 512 && nch / (2 * nsplit) >= 4) nsplit *= 2;
    const dim3 g2((unsigned)nrb, (unsigned)nsplit);
    if (a.thr > 0 && a.h) hipLaunchKernelGGL((lora_down_ring_kernel<NB, true, true>), g2, dim3(256), 0, st, a);
    else if (a.thr > 0) hipLaunchKernelGGL((lora_down_ring_kernel<NB, true, false>), g2, dim3(256), 0, st, a);
    else hipLaunchKernelGGL((lora_down_ring_kernel<NB, false, false>), g2, dim3(256), 0, st, a);
    if (nsplit > 1) {
      const int64_t n = (int64_t)a.S * 32 * NB;
      hipLaunchKernelGGL(lora_down_finish_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, a, nsplit,
                         32 * NB);
    }
    return;
  }
  if (a.thr > 0) hipLaunchKernelGGL((lora_down_kernel<NB, true>), grid, dim3(kDownWaves * 64), 0, st, a);
  else hipLaunchKernelGGL((lora_down_kernel<NB, false>), grid, dim3(kDownWaves * 64), 0, st, a);
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
  // the LDS-staged kernel moves dX in 16-byte runs: rows must start 16-byte aligned
  if (a.K % 128 || a.rank > 128 || a.dx_rs % 8) {
    const dim3 grid((unsigned)((a.K + 511) / 512), (unsigned)((a.S + 31) / 32)), block(256);
    switch ((a.rank + 31) / 32) {
      case 1: hipLaunchKernelGGL((lora_dx_rows_kernel<2>), grid, block, 0, st, a); break;
      case 2: hipLaunchKernelGGL((lora_dx_rows_kernel<4>), grid, block, 0, st, a); break;
      case 3: hipLaunchKernelGGL((lora_dx_rows_kernel<6>), grid, block, 0, st, a); break;
      case 4: hipLaunchKernelGGL((lora_dx_rows_kernel<8>), grid, block, 0, st, a); break;
      default: hipLaunchKernelGGL((lora_dx_rows_kernel<2>), grid, block, 0, st, a); break;   // 2-step chunks
    }
    return;
  }
  const dim3 grid((unsigned)(a.K / 128), (unsigned)((a.S + 127) / 128)), block(256);
  switch ((a.rank + 31) / 32) {
    case 1: hipLaunchKernelGGL((lora_dx_kernel<2>), grid, block, 0, st, a); break;
    case 2: hipLaunchKernelGGL((lora_dx_kernel<4>), grid, block, 0, st, a); break;
    case 3: hipLaunchKernelGGL((lora_dx_kernel<6>), grid, block, 0, st, a); break;
    default: hipLaunchKernelGGL((lora_dx_kernel<8>), grid, block, 0, st, a); break;
  }
}

void launch_lora_da(const LoraDaArgs &a, hipStream_t st) {
  const int nkb = a.K / 128, nst = (a.S + 31) / 32;
  int nsplit = 1;
  while (nsplit < kDaMaxSplit && nkb * nsplit < 512 && nst / (2 * nsplit) >= 4) nsplit *= 2;
  const dim3 grid((unsigned)nkb, (unsigned)nsplit), block(256);
  for (int r0 = 0; r0 < a.rank; r0 += 128) {
    switch ((min(a.rank - r0, 128) + 31) / 32) {
      case 1: hipLaunchKernelGGL((lora_da_kernel<1>), grid, block, 0, st, a, r0); break;
      case 2: hipLaunchKernelGGL((lora_da_kernel<2>), grid, block, 0, st, a, r0); break;
      case 3: hipLaunchKernelGGL((lora_da_kernel<3>), grid, block, 0, st, a, r0); break;
      default: hipLaunchKernelGGL((lora_da_kernel<4>), grid, block, 0, st, a, r0); break;
    }
  }
  if (nsplit > 1) {
    const int64_t n = (int64_t)a.rank * a.K;
    hipLaunchKernelGGL(lora_da_finish_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, a, nsplit);
  }
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

// ---- the general path (fp16 / fp32 operands) ------------------------------
// HBM-bound elementwise kernels: one thread per element pair (dropout) or
// element (scale rows); the products run in hipBLASLt.

namespace {

template <typename T> __device__ __forceinline__ float to_f(T v) { return (float)v; }
template <typename T> __device__ __forceinline__ T from_f(float v) { return (T)v; }

template <typename T>
__global__ __launch_bounds__(256) void lora_gen_dropout_kernel(const T *x, int64_t x_rs, int32_t S, int32_t K,
                                                               uint32_t thr, float ks, uint64_t seed, T *h,
                                                               int64_t h_rs, int32_t in_place) {
  const int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;   // element pair of the flattened [S, K]
  if (j >= (int64_t)S * K / 2) return;
  const int64_t e = 2 * j;
  const int s = (int)(e / K), k = (int)(e - (int64_t)s * K);   // K is even: the pair stays in the row
  const uint32_t bits = pair_bits(seed, (uint64_t)j);
  const T *xr = in_place ? h + (int64_t)s * h_rs : x + (int64_t)s * x_rs;
  T *hr = h + (int64_t)s * h_rs;
  const float v0 = to_f(xr[k]), v1 = to_f(xr[k + 1]);
  hr[k] = (bits & 0xffffu) >= thr ? from_f<T>(v0 * ks) : from_f<T>(0.f);
  hr[k + 1] = (bits >> 16) >= thr ? from_f<T>(v1 * ks) : from_f<T>(0.f);
}

// rows of rank entries, then zeros up to rpad (the padded columns the bf16
// kernels write as zeros too)
template <typename T>
__global__ __launch_bounds__(256) void lora_gen_scale_rows_kernel(const T *u, int64_t u_rs, const float *gate,
                                                                  float scaling, int32_t gate_first, int32_t S,
                                                                  int32_t rank, int32_t rpad, T *out, int64_t out_rs) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)S * rpad) return;
  const int s = (int)(i / rpad), r = (int)(i - (int64_t)s * rpad);
  float w = 0.f;
  if (r < rank) {
    const float g = gate ? gate[s] : 1.f;
    const float v = to_f(u[(int64_t)s * u_rs + r]);
    w = gate_first ? to_f(from_f<T>(to_f(from_f<T>(v * g)) * scaling))
                   : to_f(from_f<T>(to_f(from_f<T>(v * scaling)) * g));
  }
  out[(int64_t)s * out_rs + r] = from_f<T>(w);
}

template <typename T>
void gen_launch(int64_t n, void (*k)(const T *, int64_t, int32_t, int32_t, uint32_t, float, uint64_t, T *, int64_t, int32_t),
                const void *x, int64_t x_rs, int32_t S, int32_t K, uint32_t thr, float ks, uint64_t seed, void *h,
                int64_t h_rs, int32_t in_place, hipStream_t st) {
  hipLaunchKernelGGL(k, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, reinterpret_cast<const T *>(x), x_rs, S,
                     K, thr, ks, seed, reinterpret_cast<T *>(h), h_rs, in_place);
}

}  // namespace

void launch_lora_gen_dropout(int dtype, const void *x, int64_t x_rs, int32_t S, int32_t K, uint32_t thr,
                             float keep_scale, uint64_t seed, void *h, int64_t h_rs, hipStream_t st) {
  const int64_t n = (int64_t)S * K / 2;
  if (dtype == kDtF32) gen_launch<float>(n, lora_gen_dropout_kernel<float>, x, x_rs, S, K, thr, keep_scale, seed, h, h_rs, 0, st);
  else gen_launch<f16_t>(n, lora_gen_dropout_kernel<f16_t>, x, x_rs, S, K, thr, keep_scale, seed, h, h_rs, 0, st);
}

void launch_lora_gen_dx_mask(int dtype, void *dx, int64_t dx_rs, int32_t S, int32_t K, uint32_t thr, float keep_scale,
                             uint64_t seed, hipStream_t st) {
  const int64_t n = (int64_t)S * K / 2;
  if (dtype == kDtF32) gen_launch<float>(n, lora_gen_dropout_kernel<float>, dx, dx_rs, S, K, thr, keep_scale, seed, dx, dx_rs, 1, st);
  else gen_launch<f16_t>(n, lora_gen_dropout_kernel<f16_t>, dx, dx_rs, S, K, thr, keep_scale, seed, dx, dx_rs, 1, st);
}

void launch_lora_gen_scale_rows(int dtype, const void *u, int64_t u_rs, const float *gate, float scaling, bool gate_first,
                                int32_t S, int32_t rank, int32_t rpad, void *out, int64_t out_rs, hipStream_t st) {
  const int64_t n = (int64_t)S * rpad;
  const dim3 grid((unsigned)((n + 255) / 256));
  if (dtype == kDtF32)
    hipLaunchKernelGGL(lora_gen_scale_rows_kernel<float>, grid, dim3(256), 0, st, reinterpret_cast<const float *>(u),
                       u_rs, gate, scaling, (int32_t)gate_first, S, rank, rpad, reinterpret_cast<float *>(out), out_rs);
  else
    hipLaunchKernelGGL(lora_gen_scale_rows_kernel<f16_t>, grid, dim3(256), 0, st, reinterpret_cast<const f16_t *>(u),
                       u_rs, gate, scaling, (int32_t)gate_first, S, rank, rpad, reinterpret_cast<f16_t *>(out), out_rs);
}

namespace {

// splits of the reduced dimension: about two workgroups per CU, at most
// kSkinnyMaxSplit, at least one 64-wide chunk each
int skinny_splits(int lines, int kdim) {
  const int nblk = (lines + 63) / 64, nch = (kdim + 63) / 64;
  const int want = (2 * 256 + nblk - 1) / nblk;
  return std::max(1, std::min({want, kSkinnyMaxSplit, nch}));
}

template <int MODE>
void launch_skinny(const LoraSkinnyArgs &a, int nsplit, hipStream_t st) {
  const int lines = MODE == 0 ? a.N : a.S;
  const dim3 grid((unsigned)((lines + 63) / 64), (unsigned)nsplit), blk(256);
  if (a.S % 64 == 0 && a.N % 64 == 0) {
    switch (a.rp / 32) {
      case 1: hipLaunchKernelGGL((lora_skinny_kernel<MODE, 1>), grid, blk, 0, st, a); break;
      case 2: hipLaunchKernelGGL((lora_skinny_kernel<MODE, 2>), grid, blk, 0, st, a); break;
      case 3: hipLaunchKernelGGL((lora_skinny_kernel<MODE, 3>), grid, blk, 0, st, a); break;
      default: hipLaunchKernelGGL((lora_skinny_kernel<MODE, 4>), grid, blk, 0, st, a); break;
    }
  } else {
    switch (a.rp / 32) {
      case 1: hipLaunchKernelGGL((lora_skinny_clamp_kernel<MODE, 1>), grid, blk, 0, st, a); break;
      case 2: hipLaunchKernelGGL((lora_skinny_clamp_kernel<MODE, 2>), grid, blk, 0, st, a); break;
      case 3: hipLaunchKernelGGL((lora_skinny_clamp_kernel<MODE, 3>), grid, blk, 0, st, a); break;
      default: hipLaunchKernelGGL((lora_skinny_clamp_kernel<MODE, 4>), grid, blk, 0, st, a); break;
    }
  }
}

}  // namespace

void launch_lora_grad_b(const LoraSkinnyArgs &a, void *db, int64_t db_rs, hipStream_t st) {
  const int ns = skinny_splits(a.N, a.S);
  launch_skinny<0>(a, ns, st);
  const int64_t n = (int64_t)a.N * a.rank;
  hipLaunchKernelGGL(lora_db_finish_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, a, ns,
                     reinterpret_cast<bf16_t *>(db), db_rs);
}

void launch_lora_grad_u(const LoraSkinnyArgs &a, const float *gate, float scaling, void *da, int64_t da_rs,
                        hipStream_t st) {
  const int ns = skinny_splits(a.S, a.N);
  launch_skinny<1>(a, ns, st);
  const int64_t n = (int64_t)a.S * a.rp;
  hipLaunchKernelGGL(lora_u_finish_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, a, ns, gate, scaling,
                     reinterpret_cast<bf16_t *>(da), da_rs);
}

}  // namespace mga
