// MTP block-masked GQA attention forward for gfx950.
//
// Work item = (kv head g, slice of the G query heads, block of query rows).
// A workgroup of 4 waves holds 4 (query head, NB x 32-row block) pairs of one
// kv head: with G a multiple of 4 that is 4 heads x the same rows, so every
// K/V tile staged in LDS feeds four heads. Each wave computes
//   S^T = K Q^T  (v_mfma_f32_32x32x16_bf16; lane = query column)
// over 64-key steps, keeps the online-softmax state of its queries in the lane
// (plus one exchange with the lane 32 away) and accumulates O^T += V^T P^T,
// feeding the probabilities from the accumulator registers straight into the
// B operand. V^T comes from the row-major V tile through the LDS transpose
// read. K/V tiles (bf16 or fp16) are loaded one step ahead straight into the
// other of two named LDS buffers, so one barrier per step suffices.
//
// NB = 1: 32 rows per wave, 2 waves per SIMD (256 registers each).
// NB = 2: 64 rows per wave, 1 wave per SIMD; every K and V^T operand read from
// LDS feeds two MFMAs and the larger register budget keeps reads in flight.
//
// Softmax without a per-step row max: probabilities are exp2(s * c - m) with
// m the row's running offset, and a step is accepted when every lane's partial
// row sum is at most 2^20 (so is every probability). Otherwise (a row's first
// unmasked scores, or a score more than 20 log2 units above m) the step takes
// the slow path: m moves to the exact running max, O and the row sum are
// rescaled and the probabilities recomputed from the scores still held in
// registers. Row sums are taken from the bf16-rounded probabilities the O
// update multiplies (v_dot2), so the normalisation matches the weights used.
// Masking is compiled only into the partial-tile variant of a step: one
// ordered compare per score (see key_w) plus the causal bound when the step
// crosses the diagonal.
// Semantics: [torch]_higher_order_ops/flex_attention.py:202-267 (masked
// scores -inf; a fully masked row has output 0 and LSE -inf).
#include <type_traits>

#include "mga_common.hpp"
#include "mga_internal.hpp"

namespace mga {

namespace {

constexpr float kNegInfF = -__builtin_huge_valf();
// Largest partial row sum of a step on the fast path (so also the largest
// probability): 2^20 for bf16, 2^15 for fp16 (whose largest finite is 65504).
template <typename E>
constexpr float kPBound = std::is_same_v<E, f16_t> ? 32768.f : 1048576.f;
constexpr int kStepKeys = 64;                 // keys per pipeline step (a multiple of 32)
constexpr int kStepBlocks = kStepKeys / 32;   // 32-key MFMA blocks per step
constexpr int kStepsPerTile = kBlock / kStepKeys;

__device__ __forceinline__ float exp2f_(float x) { return __builtin_amdgcn_exp2f(x); }

// Heads sharing a workgroup (a divisor of both G and 4).
__host__ __device__ __forceinline__ int heads_per_wg(int G) { return (G % 4 == 0) ? 4 : (G % 2 == 0 ? 2 : 1); }

}  // namespace

template <int NB, int HD, typename T>
__global__ __launch_bounds__(256, 3 - NB) void attn_fwd_kernel(AttnArgs a) {
  typedef typename MfmaElem<T>::type E;
  constexpr int KS = HD / 16;          // k-steps of QK^T over head_dim
  constexpr int DB = HD / 32;          // 32-dim blocks of O^T
  constexpr int TILE = kStepKeys * HD; // elements of one K or V step tile
  constexpr int WR = 32 * NB;          // query rows per wave
  __shared__ __attribute__((aligned(16))) bf16_t sK0[TILE], sK1[TILE];
  __shared__ __attribute__((aligned(16))) bf16_t sV0[TILE], sV1[TILE];
  __shared__ __attribute__((aligned(16))) int sW0[kStepKeys], sW1[kStepKeys];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, hi = lane >> 5;
  const int G = a.Hq / a.Hkv;
  const int HPW = heads_per_wg(G);
  const int QR = WR * (4 / HPW);          // query rows per workgroup (<= 128)
  const int nslice = G / HPW;
  const int nqb = (a.S + QR - 1) / QR;

  // logical item: kv head major (one kv head per XCD when Hkv = 8), then query
  // blocks from the last (longest) to the first, then the head slice
  const int li = xcd_swizzle(blockIdx.x, a.Hkv * nslice * nqb);
  const int g = li / (nslice * nqb);
  const int rem = li % (nslice * nqb);
  const int qb = nqb - 1 - rem / nslice;
  const int slice = rem % nslice;
  const int h = g * G + slice * HPW + wave % HPW;
  const int row0 = qb * QR + (wave / HPW) * WR;        // first row of this wave
  const int qt = (qb * QR) / kBlock;                   // block-mask query tile

  const T *qp = reinterpret_cast<const T *>(a.q) + h * a.q_sh;
  const T *kp = reinterpret_cast<const T *>(a.k) + g * a.k_sh;
  const T *vp = reinterpret_cast<const T *>(a.v) + g * a.v_sh;

  // per row block nb: lane owns query row0 + 32 nb + l32
  bf16x8 qf[NB][KS];
  int qv[NB], qlim[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    const int row = row0 + 32 * nb + l32;
    const int qr = min(row, a.S - 1);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) qf[nb][ks] = load8(qp + (int64_t)qr * a.q_ss + ks * 16 + hi * 8);
    const int qcode = row < a.S ? a.code[row] : kCodePad;
    qv[nb] = query_v(qcode);
    // a pad query (or a row past S) sees no key: fold that into the causal bound
    qlim[nb] = (qcode == kCodePad) ? -1 : row + a.P;
  }

  TileList tiles = tile_list(a.kv_num, a.kv_idx, a.fkv_num, a.fkv_idx, qt, a.nKV);
  const int npart = tiles.npart;
  const int ntot = tiles.ntot;
  const int nstep = kStepsPerTile * ntot;
  auto step_base = [&](int j) { return tiles.at(j / kStepsPerTile) * kBlock + (j % kStepsPerTile) * kStepKeys; };

  // per-lane LDS offsets: K rows (A operand of QK^T) and the V^T transpose reads
  // K operand of k-step ks: row l32 (+ 32 kb), granule (2 ks + hi) ^ swz(l32),
  // i.e. byte offset krow ^ (ks << 5)
  const uint32_t krow = opaque_u32((uint32_t)(l32 * HD + (((uint32_t)hi ^ swz<HD>(l32)) << 3)) * 2u);
  TrOffsets<HD> tro;
  tro.init(lane);

  DmaLane<HD, kStepKeys> dma;   // shared by the K and V tiles
  dma.init();
  const uint32_t lrowK = dma.lane_row(a.k_ss);
  const uint32_t lrowV = dma.lane_row(a.v_ss);
  KeyCode wkey;
  auto load_step = [&](int j, bf16_t *dK, bf16_t *dV) {
    const int kb = step_base(j);
    if (kb >= a.L) {
      // second half of the last tile, past the keys: never computed, nothing to load
    } else if (kb + kStepKeys <= a.L) {
      dma.issue(dK, reinterpret_cast<const bf16_t *>(kp) + (int64_t)kb * a.k_ss, a.k_ss, lrowK);
      dma.issue(dV, reinterpret_cast<const bf16_t *>(vp) + (int64_t)kb * a.v_ss, a.v_ss, lrowV);
    } else {
      dma.issue_clamped(dK, reinterpret_cast<const bf16_t *>(kp) + (int64_t)kb * a.k_ss, a.k_ss, a.L - kb);
      dma.issue_clamped(dV, reinterpret_cast<const bf16_t *>(vp) + (int64_t)kb * a.v_ss, a.v_ss, a.L - kb);
    }
    // raw code only: converting it here would wait for the tile loads too
    if (tid < kStepKeys) wkey.load(a.code, kb + tid, a.P, a.L);
  };
  auto store_step = [&](bf16_t *, bf16_t *, int *dW) {
    __builtin_amdgcn_s_waitcnt(0);   // this thread's direct loads have landed
    if (tid < kStepKeys) *reinterpret_cast<int *>(const_cast<char *>(lds_at(dW, opaque_u32(tid * 4u)))) = wkey.w();
  };

  const float c = a.scale_log2;
  float m_run[NB], l_run[NB];
  f32x16 oacc[NB][DB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    m_run[nb] = qlim[nb] < 0 ? 0.f : kNegInfF;   // a pad row never needs an offset
    l_run[nb] = 0.f;
#pragma unroll
    for (int db = 0; db < DB; ++db) oacc[nb][db] = zero16();
  }

  auto run_step = [&](auto bsel, int j) {
    constexpr int B = decltype(bsel)::value;
    const bf16_t *tK = B ? sK1 : sK0;
    const bf16_t *tV = B ? sV1 : sV0;
    const int *tW = B ? sW1 : sW0;
    const int kbase = step_base(j);
    const bool partial = (j / kStepsPerTile) < npart;
    if (j + 1 < nstep) load_step(j + 1, B ? sK0 : sK1, B ? sV0 : sV1);

    // S^T = K Q^T for 64 keys x WR queries; register r of sacc[kb][nb] is key
    // kb * 32 + 8 (r / 4) + 4 hi + r % 4 of the step, query row block nb.
    if (kbase < a.L) {
      f32x16 sacc[kStepBlocks][NB];
#pragma unroll
      for (int kb = 0; kb < kStepBlocks; ++kb)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) sacc[kb][nb] = zero16();
      // the K operands of k-step ks + 1 are read before the MFMAs of ks (the
      // scheduling barriers keep that order), so each LDS read has two MFMAs
      // of time to land instead of stalling the one that uses it
      auto kread = [&](int ks, int kb) {
        return lds_read8(reinterpret_cast<const bf16_t *>(lds_at(tK + kb * 32 * HD, krow ^ (uint32_t)(ks << 5))));
      };
      bf16x8 ka[kStepBlocks];
#pragma unroll
      for (int kb = 0; kb < kStepBlocks; ++kb) ka[kb] = kread(0, kb);
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        bf16x8 kn[kStepBlocks];
        if (ks + 1 < KS)
#pragma unroll
          for (int kb = 0; kb < kStepBlocks; ++kb) kn[kb] = kread(ks + 1, kb);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int kb = 0; kb < kStepBlocks; ++kb)
#pragma unroll
          for (int nb = 0; nb < NB; ++nb) sacc[kb][nb] = mfma32<E>(ka[kb], qf[nb][ks], sacc[kb][nb]);
        __builtin_amdgcn_sched_barrier(0);
        if (ks + 1 < KS)
#pragma unroll
          for (int kb = 0; kb < kStepBlocks; ++kb) ka[kb] = kn[kb];
      }
      bf16x8 pb[NB][2 * kStepBlocks];
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        if (partial) {
          // a real branch: if-converted, full tiles would pay for the masking
          asm volatile("");
          const int lim = qlim[nb] - kbase - 4 * hi;   // key offset (without 4 hi) must be <= lim
#pragma unroll
          for (int kb = 0; kb < kStepBlocks; ++kb)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const i32x4 w4 = *reinterpret_cast<const i32x4 *>(&tW[kb * 32 + 8 * i + 4 * hi]);
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                const bool ok = (w4[e] >= qv[nb]) & (kb * 32 + 8 * i + e <= lim);
                sacc[kb][nb][4 * i + e] = ok ? sacc[kb][nb][4 * i + e] : kNegInfF;
              }
            }
        }
        // probabilities against the running offset; the slow path when a
        // partial row sum leaves the bound (or the row had no offset yet)
        auto probs = [&](float m) {
          float ps = 0.f;
#pragma unroll
          for (int kb = 0; kb < kStepBlocks; ++kb)
#pragma unroll
            for (int u = 0; u < 2; ++u) {
              i32x4 wv;
#pragma unroll
              for (int t = 0; t < 4; ++t) {
                const float p0 = exp2f_(__builtin_fmaf(sacc[kb][nb][8 * u + 2 * t], c, -m));
                const float p1 = exp2f_(__builtin_fmaf(sacc[kb][nb][8 * u + 2 * t + 1], c, -m));
                const uint32_t w = cvt2<E>(p0, p1);
                wv[t] = (int)w;
                ps = add_pair<E>(w, ps);
              }
              pb[nb][2 * kb + u] = __builtin_bit_cast(bf16x8, wv);
            }
          return ps;
        };
        float ps = probs(m_run[nb]);
        if (__builtin_amdgcn_ballot_w64(!(ps <= kPBound<E>))) {
          float mx = kNegInfF;
#pragma unroll
          for (int kb = 0; kb < kStepBlocks; ++kb)
#pragma unroll
            for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sacc[kb][nb][r]);
          mx = fmaxf(mx, xor32(mx)) * c;
          const float m_new = fmaxf(m_run[nb], mx);
          if (m_new > m_run[nb]) {
            const float alpha = exp2f_(m_run[nb] - m_new);   // 0 when m_run = -inf
            l_run[nb] *= alpha;
#pragma unroll
            for (int db = 0; db < DB; ++db)
#pragma unroll
              for (int r = 0; r < 16; ++r) oacc[nb][db][r] *= alpha;
            m_run[nb] = m_new;
          }
          ps = probs(m_run[nb] == kNegInfF ? 0.f : m_run[nb]);
        }
        l_run[nb] += ps;
      }
      // O^T += V^T P^T (each V^T operand serves the NB row blocks); operand
      // t = (16-key slice t / DB, output block t % DB), read one ahead
      bf16x8 vcur = tro.operand(tV, 0, 0);
#pragma unroll
      for (int t = 0; t < 2 * kStepBlocks * DB; ++t) {
        bf16x8 vnext;
        if (t + 1 < 2 * kStepBlocks * DB) vnext = tro.operand(tV, ((t + 1) / DB) * 16, (t + 1) % DB);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) oacc[nb][t % DB] = mfma32<E>(vcur, pb[nb][t / DB], oacc[nb][t % DB]);
        __builtin_amdgcn_sched_barrier(0);
        if (t + 1 < 2 * kStepBlocks * DB) vcur = vnext;
      }
    }

    if (j + 1 < nstep) store_step(B ? sK0 : sK1, B ? sV0 : sV1, B ? sW0 : sW1);
    __syncthreads();
  };

  if (nstep > 0) {
    load_step(0, sK0, sV0);
    store_step(sK0, sV0, sW0);
  }
  __syncthreads();
  for (int j = 0; j < nstep; j += 2) {
    run_step(std::integral_constant<int, 0>{}, j);
    if (j + 1 < nstep) run_step(std::integral_constant<int, 1>{}, j + 1);
  }

  // ---- epilogue: normalise, write O [S, Hq, D] and the natural-log LSE -------
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    const int row = row0 + 32 * nb + l32;
    const float lt = l_run[nb] + xor32(l_run[nb]);
    if (row < a.S) {
      const float inv = lt > 0.f ? 1.f / lt : 0.f;
      if (hi == 0)
        a.lse[(int64_t)h * a.S + row] = lt > 0.f ? (m_run[nb] + __log2f(lt)) * kLn2 : kNegInfF;
      T *orow = reinterpret_cast<T *>(const_cast<void *>(a.o)) + h * a.o_sh + (int64_t)row * a.o_ss;
#pragma unroll
      for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const f32x16 &c = oacc[nb][db];
          store4(orow + db * 32 + 8 * i + 4 * hi, c[4 * i] * inv, c[4 * i + 1] * inv,
                 c[4 * i + 2] * inv, c[4 * i + 3] * inv);
        }
    }
  }
}

// explicit instantiations: clang otherwise drops some host launch stubs of
// this template (the bf16 ones), leaving undefined symbols
template __global__ void attn_fwd_kernel<1, 128, bf16_t>(AttnArgs);
template __global__ void attn_fwd_kernel<1, 64, bf16_t>(AttnArgs);
template __global__ void attn_fwd_kernel<1, 128, f16_t>(AttnArgs);
template __global__ void attn_fwd_kernel<1, 64, f16_t>(AttnArgs);

// NB = 1 (32 rows per wave, 2 waves per SIMD): measured 1.01 ms against
// 1.66 ms for NB = 2 at Qwen3-8B geometry (4096 + 1024 rows vs an 8192 prefix).
template <int HD, typename T>
static void fwd_launch(const AttnArgs &a, hipStream_t st) {
  constexpr int NB = 1;
  const int G = a.Hq / a.Hkv;
  const int HPW = heads_per_wg(G);
  const int QR = 32 * NB * (4 / HPW);
  const int nqb = (a.S + QR - 1) / QR;
  const int items = a.Hkv * (G / HPW) * nqb;
  hipLaunchKernelGGL((attn_fwd_kernel<NB, HD, T>), dim3(items), dim3(256), 0, st, a);
}

template <int HD>
static void fwd_launch_dt(const AttnArgs &a, int dtype, hipStream_t st) {
  if (dtype == kDtF16) fwd_launch<HD, f16_t>(a, st);
  else fwd_launch<HD, bf16_t>(a, st);
}

void launch_attn_fwd(const AttnArgs &a, int head_dim, int dtype, hipStream_t st) {
  if (dtype == kDtF32) launch_attn_fwd_f32(a, head_dim, st);
  else if (head_dim == 128) fwd_launch_dt<128>(a, dtype, st);
  else fwd_launch_dt<64>(a, dtype, st);
}

}  // namespace mga
