// MTP block-masked GQA attention backward, dQ pass, for gfx950.
//
// Work item = (kv head, slice of HPW of its query heads, block of query
// rows); a wave holds one (query head, 32-row block) pair, and every row of a
// workgroup lies in one 128-row query tile (one tile list). Three forms:
// * kDqPair (heads in slices of 2 or 4): 8 waves, one workgroup per CU (2
//   waves per SIMD), two 32-row blocks per head; each staged K/V tile feeds
//   all 8 waves, half the tile loads and LDS writes per MFMA of two 4-wave
//   workgroups sharing the CU.
// * kDqSplit: the last round of kDqPair items when it would fill at most half
//   of the CUs: each half of an item (one 32-row block per head) runs as an
//   8-wave workgroup whose two 4-wave groups take alternate tiles of the list;
//   group 1 hands its dQ partial sums to group 0 through LDS at the end, added
//   in a fixed order.
// * kDq4 (odd G, one head per slice): 4 waves over 4 row blocks of one head,
//   two workgroups per CU.
// Each XCD (workgroup id mod 8) runs a contiguous share of the kDqPair items,
// kv head major and longest first, so the tail round holds the shortest.
// Q and dO stay in registers. K/V tiles are staged 64 keys at a time (one
// barrier and one set of direct loads per step); per 32-key block of a step
// each wave computes
//   S^T  = K Q^T,  dP^T = V dO^T                    (A operands: K, V rows)
//   P    = exp2(S^T * scale_log2 - lse_log2)         (0 where masked)
//   dS^T = P (dP^T - delta)
//   dQ^T += K^T dS^T                                  (A operand: K^T by transpose read)
// and finally dQ = scale * dQ^T^T. The prologue forms delta = rowsum(O * dO)
// for the wave's rows (fp32, from the stored operands) and writes it for the
// dK/dV pass. Semantics: [torch]_higher_order_ops/flex_attention.py:826-990
// with grad_lse = 0; a fully masked row (LSE -inf) gets dQ = 0.
#include <type_traits>

#include "mga_common.hpp"
#include "mga_internal.hpp"

namespace mga {

namespace {

constexpr float kNegInfD = -__builtin_huge_valf();
constexpr int kStep = 64;   // keys per staged step (one barrier, one load set)
constexpr int kSubKeys = 32;   // keys per compute block (the accumulators hold 32 keys)

__host__ __device__ __forceinline__ int heads_per_wg_dq(int G) { return (G % 4 == 0) ? 4 : (G % 2 == 0 ? 2 : 1); }

enum { kDq4 = 0, kDqPair = 1, kDqSplit = 2 };

// Sum over this lane's half of the row (dims ks*16 + hi*8 .. +8) of o * d.
template <int HD, typename T>
__device__ __forceinline__ float half_row_dot(const T *o, const T *d, int hi) {
  float acc = 0.f;
#pragma unroll
  for (int ks = 0; ks < HD / 16; ++ks) {
    const int c = ks * 16 + hi * 8;
    const auto x = __builtin_bit_cast(typename Elem<T>::v8, load8(o + c));
    const auto y = __builtin_bit_cast(typename Elem<T>::v8, load8(d + c));
#pragma unroll
    for (int e = 0; e < 8; ++e) acc += (float)x[e] * (float)y[e];
  }
  return acc;
}

}  // namespace

template <int HD, typename T, int MODE>
__global__ __launch_bounds__(MODE == kDq4 ? 256 : 512, 2) void attn_bwd_dq_kernel(AttnArgs a, int k1, int kn) {
  constexpr int NG = MODE == kDqSplit ? 2 : 1;    // groups splitting the tile list
  constexpr int NWD = MODE == kDqPair ? 8 : 4;    // waves sharing each staged tile
  typedef typename MfmaElem<T>::type E;
  constexpr int KS = HD / 16;
  constexpr int DB = HD / 32;
  constexpr int TILE = kStep * HD;
  // two named buffers per operand (not one array of two): distinct LDS objects
  // let the compiler see that the direct loads into one buffer never alias the
  // reads of the other, so it does not wait for them before computing
  // [group][TILE]: each group stages the tiles of its own keys
  __shared__ __attribute__((aligned(16))) bf16_t sK0[NG * TILE], sK1[NG * TILE];
  __shared__ __attribute__((aligned(16))) bf16_t sV0[NG * TILE], sV1[NG * TILE];
  __shared__ __attribute__((aligned(16))) int sW0[NG * kStep], sW1[NG * kStep];

  const int tid = threadIdx.x, lane = tid & 63;
  const int grp = NG == 2 ? wave_id() >> 2 : 0;
  const int wave = NG == 2 ? wave_id() & 3 : wave_id();   // wave among those holding the rows
  const int gtid = NG == 2 ? tid & 255 : tid;
  const int l32 = lane & 31, hi = lane >> 5;
  const int G = a.Hq / a.Hkv;
  const int HPW = heads_per_wg_dq(G);
  const int QR4 = 32 * (4 / HPW);   // rows of 4 waves: 32, 64 or 128
  const int nslice = G / HPW;
  int li, nqb, qr_item;
  if constexpr (MODE == kDq4) {
    qr_item = QR4;
    nqb = (a.S + QR4 - 1) / QR4;
    li = xcd_swizzle(blockIdx.x, a.Hkv * nslice * nqb);
  } else {
    qr_item = 2 * QR4;
    nqb = (a.S + qr_item - 1) / qr_item;
    const int n_items = a.Hkv * nslice * nqb;
    const int xcd = blockIdx.x & 7;
    const int o = k1 + (int)(MODE == kDqSplit ? blockIdx.x >> 4 : blockIdx.x >> 3);
    const int n_x = n_items / 8 + (xcd < n_items % 8 ? 1 : 0);
    if (o >= n_x || o >= k1 + kn) return;
    li = xcd * (n_items / 8) + min(xcd, n_items % 8) + o;
  }
  const int g = li / (nslice * nqb);
  const int rem = li % (nslice * nqb);
  const int qb = nqb - 1 - rem / nslice;
  const int slice = rem % nslice;
  const int wg_row0 = qb * qr_item + (MODE == kDqSplit ? (int)((blockIdx.x >> 3) & 1) * QR4 : 0);
  const int h = g * G + slice * HPW + wave % HPW;
  const int row = wg_row0 + (wave / HPW) * 32 + l32;
  const int qt = wg_row0 / kBlock;
  const bool in = row < a.S;
  const int qr = min(row, a.S - 1);

  const T *qp = reinterpret_cast<const T *>(a.q) + h * a.q_sh + (int64_t)qr * a.q_ss;
  const T *dop = reinterpret_cast<const T *>(a.dout) + h * a.do_sh + (int64_t)qr * a.do_ss;
  const T *op = reinterpret_cast<const T *>(a.o) + h * a.o_sh + (int64_t)qr * a.o_ss;
  const T *kp = reinterpret_cast<const T *>(a.k) + g * a.k_sh;
  const T *vp = reinterpret_cast<const T *>(a.v) + g * a.v_sh;

  // Q and dO fragments (B operands of S^T and dP^T) in registers
  bf16x8 qf[KS], dof[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    qf[ks] = load8(qp + ks * 16 + hi * 8);
    dof[ks] = load8(dop + ks * 16 + hi * 8);
  }
  float del = half_row_dot<HD, T>(op, dop, hi);
  del += xor32(del);
  if (!in) del = 0.f;
  const float lse = in ? a.lse[(int64_t)h * a.S + row] : kNegInfD;
  // a fully masked row has LSE -inf: it reaches no key (qlim = -1) and its P is 0
  const float lse2 = lse == kNegInfD ? 0.f : lse * kLog2e;
  const float c = a.scale_log2;
  const int qcode = in ? a.code[row] : kCodePad;
  const int qv = query_v(qcode);
  const bool none = qcode == kCodePad || lse == kNegInfD;
  const int qlim = none ? -1 : row + a.P;
  // row data of the dK/dV pass, three planes of Hq * S words: -lse / scale
  // (0 for a row that sees no key), -delta, and the row's mask threshold
  // (0: sees no key; 1: regular row, sees the regular keys; 2^31 - 1 - c: mask
  // row of code c, sees the mask keys of codes >= c). A row past S reads as 0.
  if (in && hi == 0 && grp == 0) {
    const int64_t plane = (int64_t)a.Hq * a.S, at = (int64_t)h * a.S + row;
    a.delta[at] = none ? 0.f : -lse * (1.f / a.scale);
    a.delta[plane + at] = -del;
    reinterpret_cast<uint32_t *>(a.delta)[2 * plane + at] =
        none ? 0u : (qcode == kCodeX ? 1u : 0x7fffffffu - (uint32_t)qcode);
  }
  // keys up to here precede every query of the wave (pad rows are masked by
  // the ordered compare alone: their qv sits above every key)
  const int diag = row - l32 + a.P;

  TileList tiles = tile_list(a.kv_num, a.kv_idx, a.fkv_num, a.fkv_idx, qt, a.nKV);
  const int npart = tiles.npart;
  const int ntot = tiles.ntot;
  constexpr int kSub = kBlock / kStep;      // steps per 128-key tile
  const int nstep = kSub * ((ntot - grp + NG - 1) / NG);   // this group's steps
  const int nloop = kSub * ((ntot + NG - 1) / NG);        // group 0's (>= group 1's)
  auto tile_of = [&](int j) { return NG * (j / kSub) + grp; };
  auto step_base = [&](int j) { return tiles.at(tile_of(j)) * kBlock + (j % kSub) * kStep; };

  // K / V / dO operand of k-step ks: row l32, granule (2 ks + hi) ^ swz(l32),
  // i.e. byte offset krow ^ (ks << 5); K^T through the transpose reads
  const uint32_t gofs = (uint32_t)(grp * TILE * 2);   // the group's part of every tile buffer (bytes)
  const uint32_t krow = opaque_u32(gofs + (uint32_t)(l32 * HD + (((uint32_t)hi ^ swz<HD>(l32)) << 3)) * 2u);
  TrOffsets<HD> tro;
  tro.init(lane);
  if constexpr (NG == 2) {
#pragma unroll
    for (int sx = 0; sx < 2; ++sx)
#pragma unroll
      for (int mb = 0; mb < DB; ++mb) tro.off[sx][mb] = opaque_u32(tro.off[sx][mb] + gofs);
  }

  // K/V tiles go global -> LDS directly (no staging registers) through
  // buffer resources: precomputed lane offsets, the tile's first row in the
  // resource base
  BufDma<HD, kStep, NWD> dmaK, dmaV;
  dmaK.init(a.k_ss);
  dmaV.init(a.v_ss);
  KeyCode knext;
  // rows past L arrive as zeros; a step past the keys is never computed
  auto load_step = [&](int j, bf16_t *dK, bf16_t *dV) {
    const int kb = step_base(j);
    const bf16_t *kr = reinterpret_cast<const bf16_t *>(kp) + (int64_t)kb * a.k_ss;
    const bf16_t *vr = reinterpret_cast<const bf16_t *>(vp) + (int64_t)kb * a.v_ss;
    // the code read first: the compiler, which does not see the tile loads,
    // waits for every outstanding load before it writes the code register
    if (gtid < kStep) knext.load(a.code, kb + gtid, a.P, a.L);   // converted at store time
    if (kb < a.L) {
      dmaK.issue(dK + grp * TILE, kr, a.k_ss, a.L - kb);
      dmaV.issue(dV + grp * TILE, vr, a.v_ss, a.L - kb);
    }
  };
  auto store_step = [&](bf16_t *, bf16_t *, int *dW) {
    __builtin_amdgcn_s_waitcnt(0);   // this thread's direct loads have landed
    if (gtid < kStep)
      *reinterpret_cast<int *>(const_cast<char *>(lds_at(dW + grp * kStep, opaque_u32(gtid * 4u)))) = knext.w();
  };

  f32x16 dqacc[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) dqacc[db] = zero16();

  // one 64-key step reading buffer B (two 32-key compute blocks) while the
  // next step loads into 1 - B
  auto run_step = [&](auto bsel, int j) {
    constexpr int B = decltype(bsel)::value;
    const bf16_t *tK = B ? sK1 : sK0;
    const bf16_t *tV = B ? sV1 : sV0;
    const int *tW = (B ? sW1 : sW0) + grp * kStep;
    const int kbase = j < nstep ? step_base(j) : a.L;   // past the group's steps: idle (barriers only)
    const bool partial = tile_of(j) < npart;
    if (j + 1 < nstep) load_step(j + 1, B ? sK0 : sK1, B ? sV0 : sV1);

#pragma unroll
    for (int kb = 0; kb < kStep / kSubKeys; ++kb) {
      const int sbase = kbase + kb * kSubKeys;
      if (sbase >= a.L) break;   // the rest of the step is past the keys
      const bf16_t *sK = tK + kb * kSubKeys * HD;
      const bf16_t *sV = tV + kb * kSubKeys * HD;
      const int *sW = tW + kb * kSubKeys;
      // S^T = K Q^T and dP^T - delta = V dO^T - delta (the accumulator starts at
      // -delta); register r is key sbase + 8 (r / 4) + 4 hi + r % 4
      f32x16 sacc = zero16(), dpacc;
#pragma unroll
      for (int r = 0; r < 16; ++r) dpacc[r] = -del;
      // the K and V operands of k-step ks + 1 are read before the MFMAs of ks
      // (kept in that order by the scheduling barriers)
      auto rd = [&](const bf16_t *t, int ks) {
        return lds_read8(reinterpret_cast<const bf16_t *>(lds_at(t, krow ^ (uint32_t)(ks << 5))));
      };
      bf16x8 kc = rd(sK, 0), vc = rd(sV, 0);
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        bf16x8 kn, vn;
        if (ks + 1 < KS) {
          kn = rd(sK, ks + 1);
          vn = rd(sV, ks + 1);
        }
        __builtin_amdgcn_sched_barrier(0);
        sacc = mfma32<E>(kc, qf[ks], sacc);
        dpacc = mfma32<E>(vc, dof[ks], dpacc);
        __builtin_amdgcn_sched_barrier(0);
        if (ks + 1 < KS) {
          kc = kn;
          vc = vn;
        }
      }
      if (partial) {
        // a real branch: if-converted, full tiles would pay for the masking
        asm volatile("");
        if (sbase + kSubKeys - 1 > diag) {   // keys past the wave's first query: causal bound too
          const int lim = qlim - sbase - 4 * hi;   // causal: key offset (without 4 hi) <= lim
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const i32x4 w4 = *reinterpret_cast<const i32x4 *>(&sW[8 * i + 4 * hi]);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const bool ok = (w4[e] >= qv) & (8 * i + e <= lim);
              sacc[4 * i + e] = ok ? sacc[4 * i + e] : kNegInfD;   // P = exp2(-inf) = 0
            }
          }
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const i32x4 w4 = *reinterpret_cast<const i32x4 *>(&sW[8 * i + 4 * hi]);
#pragma unroll
            for (int e = 0; e < 4; ++e) sacc[4 * i + e] = w4[e] >= qv ? sacc[4 * i + e] : kNegInfD;
          }
        }
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) dpacc[r] *= __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[r], c, -lse2));
      // dQ^T += K^T dS^T
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const bf16x8 dsb = pack8<E>(dpacc[8 * u + 0], dpacc[8 * u + 1], dpacc[8 * u + 2], dpacc[8 * u + 3],
                                 dpacc[8 * u + 4], dpacc[8 * u + 5], dpacc[8 * u + 6], dpacc[8 * u + 7]);
#pragma unroll
        for (int db = 0; db < DB; ++db)
          dqacc[db] = mfma32<E>(tro.operand(sK, 16 * u, db), dsb, dqacc[db]);
      }
      __builtin_amdgcn_sched_barrier(0);   // one block's registers at a time
    }

    if (j + 1 < nstep) store_step(B ? sK0 : sK1, B ? sV0 : sV1, B ? sW0 : sW1);
    __syncthreads();
  };

  if (nstep > 0) {
    load_step(0, sK0, sV0);
    store_step(sK0, sV0, sW0);
  }
  __syncthreads();
  for (int j = 0; j < nloop; j += 2) {
    run_step(std::integral_constant<int, 0>{}, j);
    if (j + 1 < nloop) run_step(std::integral_constant<int, 1>{}, j + 1);
  }

  if constexpr (NG == 2) {
    // group 1 hands its dQ^T partial sums to group 0 through LDS (the tile
    // buffers are free after the last barrier); group 0 adds them
    float *x = reinterpret_cast<float *>(wave < 2 ? sK0 : sV0) + (wave & 1) * (DB * 16 * 64);
    if (grp == 1) {
#pragma unroll
      for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) x[(db * 16 + r) * 64 + lane] = dqacc[db][r];
    }
    __syncthreads();
    if (grp == 1) return;
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int r = 0; r < 16; ++r) dqacc[db][r] += x[(db * 16 + r) * 64 + lane];
  }

  if (in) {
    T *row_out = reinterpret_cast<T *>(a.dq) + h * a.dq_sh + (int64_t)row * a.dq_ss;
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const f32x16 &c = dqacc[db];
        store4(row_out + db * 32 + 8 * i + 4 * hi, c[4 * i] * a.scale, c[4 * i + 1] * a.scale,
               c[4 * i + 2] * a.scale, c[4 * i + 3] * a.scale);
      }
  }
}

// kDqPair items per XCD (the rest run as kDqSplit): each XCD takes a
// contiguous 1/8 of the items on its CUs, one workgroup per CU. When the last
// round would fill at most half of them, that round's items run split (two
// workgroups per item, each in about half the time); when all items fill at
// most half a round, all of them do. Items of fewer than 16 tiles are not split.
int dq_split_point(int items, int L, int cus) {
  const int nmax = (items + 7) / 8;
  const int m = cus / 8 > 0 ? cus / 8 : 1;
  if (L < 16 * kBlock) return nmax;
  if (nmax <= m / 2) return 0;
  const int r = nmax % m;
  return (nmax > m && r > 0 && r <= m / 2) ? nmax - r : nmax;
}

template <int HD, typename T>
void dq_launch(const AttnArgs &a, hipStream_t st) {
  const int G = a.Hq / a.Hkv;
  const int HPW = heads_per_wg_dq(G);
  const int QR4 = 32 * (4 / HPW);
  if (HPW == 1) {
    const int nqb = (a.S + QR4 - 1) / QR4;
    hipLaunchKernelGGL((attn_bwd_dq_kernel<HD, T, kDq4>), dim3(a.Hkv * G * nqb), dim3(256), 0, st, a, 0, 0);
    return;
  }
  const int nqb = (a.S + 2 * QR4 - 1) / (2 * QR4);
  const int items = a.Hkv * (G / HPW) * nqb;
  const int nmax = (items + 7) / 8;
  const int k1 = dq_split_point(items, a.L, device_cu_count());
  if (k1 > 0) hipLaunchKernelGGL((attn_bwd_dq_kernel<HD, T, kDqPair>), dim3(8 * k1), dim3(512), 0, st, a, 0, k1);
  if (k1 < nmax)
    hipLaunchKernelGGL((attn_bwd_dq_kernel<HD, T, kDqSplit>), dim3(16 * (nmax - k1)), dim3(512), 0, st, a, k1,
                       nmax - k1);
}

template void dq_launch<128, bf16_t>(const AttnArgs &, hipStream_t);
template void dq_launch<64, bf16_t>(const AttnArgs &, hipStream_t);
template void dq_launch<128, f16_t>(const AttnArgs &, hipStream_t);
template void dq_launch<64, f16_t>(const AttnArgs &, hipStream_t);

}  // namespace mga
