// MTP block-masked GQA attention backward, dK/dV pass, for gfx950.
//
// Work item = (128-key tile of the keys that receive gradient, query head h).
// Each of the 4 waves owns 32 keys and keeps their K and V rows in registers
// (B operands). The workgroup walks the q-major block-mask list of its key
// tile; per 64-row query step of head h (Q and dO staged by direct
// global -> LDS loads into double buffers) each wave computes
//   S  = Q K^T,  dP = dO V^T                  (A operands: Q, dO rows)
//   P  = exp2(S * scale_log2 - lse_log2)       (0 where masked)
//   dS = P (dP - delta)
//   dV^T += dO^T P,  dK^T += Q^T dS            (A operands by transpose read)
// With one query head per kv head (G = 1) the result is written directly;
// otherwise each head writes an fp32 partial and dkdv_reduce_kernel sums the
// G partials of a kv head in a fixed order (deterministic, no atomics).
// Semantics: [torch]_higher_order_ops/flex_attention.py:826-990 (dK/dV summed
// over the query heads of a kv head, :957-966), restricted to keys >= grad_start.
#include <type_traits>

#include "mga_common.hpp"
#include "mga_internal.hpp"

namespace mga {

namespace {

constexpr float kNegInfK = -__builtin_huge_valf();
constexpr int kQStep = 64;

typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2;

// two values -> one packed bf16 pair (round to nearest even)
__device__ __forceinline__ uint32_t cvt2(float x, float y) {
  bf16x2 v;
  v[0] = (bf16_t)x;
  v[1] = (bf16_t)y;
  return __builtin_bit_cast(uint32_t, v);
}

}  // namespace

template <int HD, typename T>
__global__ __launch_bounds__(256, 1) void attn_bwd_dkdv_kernel(AttnArgs a, int kt0, int nkt) {
  constexpr int KS = HD / 16;
  constexpr int DB = HD / 32;
  constexpr int TILE = kQStep * HD;
  __shared__ __attribute__((aligned(16))) bf16_t sQ0[TILE], sQ1[TILE];
  __shared__ __attribute__((aligned(16))) bf16_t sD0[TILE], sD1[TILE];
  // per query row of the step: lse * log2(e), delta, causal bound (-1: sees nothing),
  // ordered-compare value (query_v)
  __shared__ __attribute__((aligned(16))) float sL0[kQStep], sL1[kQStep];
  __shared__ __attribute__((aligned(16))) float sE0[kQStep], sE1[kQStep];
  __shared__ __attribute__((aligned(16))) int sM0[kQStep], sM1[kQStep];
  __shared__ __attribute__((aligned(16))) int sC0[kQStep], sC1[kQStep];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, hi = lane >> 5;
  const int G = a.Hq / a.Hkv;

  // logical item: kv head major (its G heads share an XCD), key tiles from the
  // first (most query tiles) to the last, then the head within the group
  const int li = xcd_swizzle(blockIdx.x, a.Hkv * nkt * G);
  const int g = li / (nkt * G);
  const int rem = li % (nkt * G);
  const int kt = kt0 + rem / G;
  const int hh = rem % G;
  const int h = g * G + hh;

  const int key = kt * kBlock + wave * 32 + l32;
  const int kr = min(key, a.L - 1);
  const int kw = key_w(a.code, key, a.P, a.L);

  bf16x8 kf[KS], vf[KS];
  {
    const T *kp = reinterpret_cast<const T *>(a.k) + g * a.k_sh + (int64_t)kr * a.k_ss;
    const T *vp = reinterpret_cast<const T *>(a.v) + g * a.v_sh + (int64_t)kr * a.v_ss;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      kf[ks] = load8(kp + ks * 16 + hi * 8);
      vf[ks] = load8(vp + ks * 16 + hi * 8);
    }
  }

  const T *qp = reinterpret_cast<const T *>(a.q) + h * a.q_sh;
  const T *dop = reinterpret_cast<const T *>(a.dout) + h * a.do_sh;
  TileList tiles = tile_list(a.q_num, a.q_idx, a.fq_num, a.fq_idx, kt, a.nQ);
  const int npart = tiles.npart;
  const int ntot = tiles.ntot;
  const int nstep = 2 * ntot;
  auto step_base = [&](int j) { return tiles.at(j >> 1) * kBlock + (j & 1) * kQStep; };

  // Q / dO operand of k-step ks for 32-row block qb: row qb * 32 + l32,
  // granule (2 ks + hi) ^ swz(l32), i.e. byte offset qrow ^ (ks << 5);
  // Q^T and dO^T through the transpose reads
  const uint32_t qrow = opaque_u32((uint32_t)(l32 * HD + (((uint32_t)hi ^ swz<HD>(l32)) << 3)) * 2u);
  TrOffsets<HD> tro;
  tro.init(lane);
  const float c = a.scale_log2;

  constexpr bool kDirect = sizeof(T) == 2;
  TileStage<HD, kDirect ? 0 : kQStep, T> stQ, stD;
  // per query row of the next step: raw lse, delta and code, converted at
  // store time (converting here would wait for the tile loads in flight)
  float rl = 0.f, re = 0.f;
  int rc = kCodePad, rq = 0;
  auto load_step = [&](int j, bf16_t *dQ, bf16_t *dD) {
    const int q0 = step_base(j);
    if constexpr (kDirect) {
      tile_dma<HD, kQStep>(dQ, reinterpret_cast<const bf16_t *>(qp), a.q_ss, q0, a.S - 1);
      tile_dma<HD, kQStep>(dD, reinterpret_cast<const bf16_t *>(dop), a.do_ss, q0, a.S - 1);
    } else {
      stQ.load(qp, a.q_ss, q0, a.S - 1);
      stD.load(dop, a.do_ss, q0, a.S - 1);
    }
    if (tid < kQStep) {
      rq = q0 + tid;
      if (rq < a.S) {
        rl = a.lse[(int64_t)h * a.S + rq];
        re = a.delta[(int64_t)h * a.S + rq];
        rc = a.code[rq];
      }
    }
  };
  auto store_step = [&](bf16_t *dQ, bf16_t *dD, float *dL, float *dE, int *dM, int *dC) {
    if constexpr (!kDirect) {
      stQ.store(dQ);
      stD.store(dD);
    } else {
      __builtin_amdgcn_s_waitcnt(0);
    }
    if (tid < kQStep) {
      const bool in = rq < a.S;
      const int code = in ? rc : kCodePad;
      const float lse = in ? rl : kNegInfK;
      dL[tid] = lse == kNegInfK ? 0.f : lse * kLog2e;
      dE[tid] = in ? re : 0.f;
      dM[tid] = (code == kCodePad || lse == kNegInfK) ? -1 : rq + a.P;   // causal bound, -1: sees nothing
      dC[tid] = query_v(code);
    }
  };

  f32x16 dkacc[DB], dvacc[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) { dkacc[db] = zero16(); dvacc[db] = zero16(); }

  auto run_step = [&](auto bsel, int j) {
    constexpr int B = decltype(bsel)::value;
    bf16_t *tQ = B ? sQ1 : sQ0;
    bf16_t *tD = B ? sD1 : sD0;
    const float *tL = B ? sL1 : sL0;
    const float *tE = B ? sE1 : sE0;
    const int *tM = B ? sM1 : sM0;
    const int *tC = B ? sC1 : sC0;
    const int q0 = step_base(j);
    const bool partial = (j >> 1) < npart;
    if (j + 1 < nstep) load_step(j + 1, B ? sQ0 : sQ1, B ? sD0 : sD1);

    // Program order is the schedule. A step is 4 blocks of 2 KS MFMAs:
    //   0: S / dP of rows 0..31,  1: S / dP of rows 32..63 (+ softmax of 0..31),
    //   2: dV / dK update of rows 0..31 (+ softmax of 32..63),  3: update of 32..63.
    // Every LDS operand is read kAhead MFMAs before its use (a ring of
    // registers) and a scheduling fence closes each MFMA slot, so the compiler
    // neither hoists all reads nor leaves a read next to its use. MASKED: a
    // partial tile (masking compiled in; a full tile's step has none).
    auto body = [&](auto masked) {
      constexpr bool MASKED = decltype(masked)::value;
      constexpr int kMm = 2 * KS;          // MFMAs of one block
      constexpr int kSlots = 4 * kMm;      // MFMAs of the step
      constexpr int kAhead = 4;
      f32x16 sacc[2], dpacc[2];
      i32x4 pb[2][2], dsb[2][2];   // packed P and dS operands (16 rows each)
      // operand of slot t
      auto read_op = [&](int t) -> bf16x8 {
        const int blk = t / kMm, i = t % kMm;
        if (blk < 2) {   // i = 2 ks + (0: Q row, 1: dO row)
          const uint32_t off = (qrow ^ (uint32_t)((i >> 1) << 5)) + (uint32_t)(blk * 32 * HD * 2);
          return lds_read8(reinterpret_cast<const bf16_t *>(lds_at((i & 1) ? tD : tQ, off)));
        }
        const int qb = blk - 2, u = (i >> 1) / DB, db = (i >> 1) % DB;   // i = 2 (u DB + db) + (0: dO^T, 1: Q^T)
        return tro.operand((i & 1) ? tQ : tD, qb * 32 + 16 * u, db);
      };
      auto mma = [&](int t, const bf16x8 &op) {
        const int blk = t / kMm, i = t % kMm;
        if (blk < 2) {
          if (i & 1) dpacc[blk] = mfma32(op, vf[i >> 1], dpacc[blk]);
          else sacc[blk] = mfma32(op, kf[i >> 1], sacc[blk]);
        } else {
          const int qb = blk - 2, u = (i >> 1) / DB, db = (i >> 1) % DB;
          if (i & 1) dkacc[db] = mfma32(op, __builtin_bit_cast(bf16x8, dsb[qb][u]), dkacc[db]);
          else dvacc[db] = mfma32(op, __builtin_bit_cast(bf16x8, pb[qb][u]), dvacc[db]);
        }
      };
      // scores 2 t, 2 t + 1 of row block qb: P (masked to 0) and dS, packed
      // straight into the operand words (the accumulators are only read)
      auto soft_pair = [&](int qb, int t) {
        const int r0 = 2 * t;
        const int ql = qb * 32 + 8 * (r0 >> 2) + 4 * hi + (r0 & 3);
        const float2 l2 = *reinterpret_cast<const float2 *>(&tL[ql]);
        const float2 e2 = *reinterpret_cast<const float2 *>(&tE[ql]);
        float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[qb][r0], c, -l2.x));
        float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[qb][r0 + 1], c, -l2.y));
        if constexpr (MASKED) {
          const int2 m2 = *reinterpret_cast<const int2 *>(&tM[ql]);
          const int2 c2 = *reinterpret_cast<const int2 *>(&tC[ql]);
          p0 = ((key <= m2.x) & (kw >= c2.x)) ? p0 : 0.f;
          p1 = ((key <= m2.y) & (kw >= c2.y)) ? p1 : 0.f;
        }
        pb[qb][t >> 2][t & 3] = (int)cvt2(p0, p1);
        dsb[qb][t >> 2][t & 3] = (int)cvt2(p0 * (dpacc[qb][r0] - e2.x), p1 * (dpacc[qb][r0 + 1] - e2.y));
      };
#pragma unroll
      for (int qb = 0; qb < 2; ++qb) {
        sacc[qb] = zero16();
        dpacc[qb] = zero16();
      }
      bf16x8 ring[kAhead];
#pragma unroll
      for (int t = 0; t < kAhead; ++t) ring[t] = read_op(t);
#pragma unroll
      for (int t = 0; t < kSlots; ++t) {
        const bf16x8 op = ring[t % kAhead];
        if (t + kAhead < kSlots) ring[t % kAhead] = read_op(t + kAhead);
        mma(t, op);
        // the softmax of a row block rides on the next block's MFMAs, one
        // pair of scores every other slot (8 pairs per block)
        const int blk = t / kMm, i = t % kMm;
        if ((blk == 1 || blk == 2) && (i & 1) && (i >> 1) < 8) soft_pair(blk - 1, i >> 1);
        if ((blk == 1 || blk == 2) && i == kMm - 1) {
#pragma unroll
          for (int pr = kMm / 2; pr < 8; ++pr) soft_pair(blk - 1, pr);   // HD = 64: the rest
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    };
    if (q0 < a.S) {
      if (partial) body(std::true_type{});
      else body(std::false_type{});
    }

    if (j + 1 < nstep)
      store_step(B ? sQ0 : sQ1, B ? sD0 : sD1, B ? sL0 : sL1, B ? sE0 : sE1, B ? sM0 : sM1,
                 B ? sC0 : sC1);
    __syncthreads();
  };

  if (nstep > 0) {
    load_step(0, sQ0, sD0);
    store_step(sQ0, sD0, sL0, sE0, sM0, sC0);
  }
  __syncthreads();
  for (int j = 0; j < nstep; j += 2) {
    run_step(std::integral_constant<int, 0>{}, j);
    if (j + 1 < nstep) run_step(std::integral_constant<int, 1>{}, j + 1);
  }

  // ---- epilogue: lane = key, registers = dims 8 (r / 4) + 4 hi + r % 4 ---------
  if (key >= a.grad_start && key < a.L) {
    const int64_t row = key - a.grad_start;
    if (G == 1) {
      T *dkr = reinterpret_cast<T *>(a.dk) + g * a.dk_sh + row * a.dk_ss;
      T *dvr = reinterpret_cast<T *>(a.dv) + g * a.dv_sh + row * a.dv_ss;
#pragma unroll
      for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int d0 = db * 32 + 8 * i + 4 * hi;
          const f32x16 &ck = dkacc[db];
          const f32x16 &cv = dvacc[db];
          store4(dkr + d0, ck[4 * i] * a.scale, ck[4 * i + 1] * a.scale, ck[4 * i + 2] * a.scale,
                 ck[4 * i + 3] * a.scale);
          store4(dvr + d0, cv[4 * i], cv[4 * i + 1], cv[4 * i + 2], cv[4 * i + 3]);
        }
    } else {
      // partial of head hh: ws[tensor][hh][row][g][d] (fp32)
      const int64_t Lg = a.L - a.grad_start;
      const int64_t plane = Lg * a.Hkv * HD;
      float *pk = a.dkv_ws + (int64_t)hh * plane + (row * a.Hkv + g) * HD;
      float *pv = pk + (int64_t)G * plane;
#pragma unroll
      for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int d0 = db * 32 + 8 * i + 4 * hi;
          const f32x16 &ck = dkacc[db];
          const f32x16 &cv = dvacc[db];
          store4(pk + d0, ck[4 * i] * a.scale, ck[4 * i + 1] * a.scale, ck[4 * i + 2] * a.scale,
                 ck[4 * i + 3] * a.scale);
          store4(pv + d0, cv[4 * i], cv[4 * i + 1], cv[4 * i + 2], cv[4 * i + 3]);
        }
    }
  }
}

// dk[row, g, :] = sum_hh ws_k[hh, row, g, :] (and dv), hh ascending. One thread
// per 4 consecutive values of one (tensor, row, g).
template <int HD, typename T>
__global__ __launch_bounds__(256) void dkdv_reduce_kernel(AttnArgs a) {
  const int64_t Lg = a.L - a.grad_start;
  const int64_t plane = Lg * a.Hkv * HD;
  const int64_t n4 = plane / 4;
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int G = a.Hq / a.Hkv;
  if (t >= 2 * n4) return;
  const int tensor = t >= n4;
  const int64_t e = (t - tensor * n4) * 4;       // element offset in one plane
  const float *src = a.dkv_ws + (int64_t)tensor * G * plane + e;
  f32x4 acc = *reinterpret_cast<const f32x4 *>(src);
  for (int hh = 1; hh < G; ++hh) {
    const f32x4 x = *reinterpret_cast<const f32x4 *>(src + hh * plane);
    acc[0] += x[0]; acc[1] += x[1]; acc[2] += x[2]; acc[3] += x[3];
  }
  const int64_t row = e / (a.Hkv * HD);
  const int g = (int)((e / HD) % a.Hkv);
  const int d = (int)(e % HD);
  T *dst = tensor ? reinterpret_cast<T *>(a.dv) + g * a.dv_sh + row * a.dv_ss
                  : reinterpret_cast<T *>(a.dk) + g * a.dk_sh + row * a.dk_ss;
  store4(dst + d, acc[0], acc[1], acc[2], acc[3]);
}

template <int HD, typename T>
void dkdv_launch(const AttnArgs &a, hipStream_t st) {
  const int kt0 = a.grad_start / kBlock;
  const int nkt = a.nKV - kt0;
  if (nkt <= 0 || a.grad_start >= a.L) return;
  const int G = a.Hq / a.Hkv;
  hipLaunchKernelGGL((attn_bwd_dkdv_kernel<HD, T>), dim3(a.Hkv * nkt * G), dim3(256), 0, st, a, kt0, nkt);
  if (G > 1) {
    const int64_t n = 2 * (int64_t)(a.L - a.grad_start) * a.Hkv * HD / 4;
    hipLaunchKernelGGL((dkdv_reduce_kernel<HD, T>), dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, a);
  }
}

template <int HD, typename T>
void dq_launch(const AttnArgs &a, hipStream_t st);   // mga_bwd_dq.hip

void launch_attn_bwd(const AttnArgs &a, int head_dim, bool is_f32, int passes, hipStream_t st) {
  if (head_dim == 128) {
    if (passes & kBwdDq) { if (is_f32) dq_launch<128, float>(a, st); else dq_launch<128, bf16_t>(a, st); }
    if (passes & kBwdDkDv) { if (is_f32) dkdv_launch<128, float>(a, st); else dkdv_launch<128, bf16_t>(a, st); }
  } else {
    if (passes & kBwdDq) { if (is_f32) dq_launch<64, float>(a, st); else dq_launch<64, bf16_t>(a, st); }
    if (passes & kBwdDkDv) { if (is_f32) dkdv_launch<64, float>(a, st); else dkdv_launch<64, bf16_t>(a, st); }
  }
}

}  // namespace mga
