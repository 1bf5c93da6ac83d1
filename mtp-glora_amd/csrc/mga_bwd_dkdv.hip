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
  const int npart = a.q_num[kt];
  const int ntot = npart + a.fq_num[kt];
  TileList tiles{a.q_idx + (int64_t)kt * a.nQ, a.fq_idx + (int64_t)kt * a.nQ, npart, ntot};
  const int nstep = 2 * ntot;
  auto step_base = [&](int j) { return tiles.at(j >> 1) * kBlock + (j & 1) * kQStep; };

  const int qrow_sw = swz<HD>(l32);
  const TrLane tl = tr_lane<HD>(lane);

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

    if (q0 < a.S) {
#pragma unroll
      for (int qb = 0; qb < 2; ++qb) {
        f32x16 sacc = zero16(), dpacc = zero16();
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          const int off = (qb * 32 + l32) * HD + (((2 * ks + hi) ^ qrow_sw) << 3);
          sacc = mfma32(lds_read8(tQ + off), kf[ks], sacc);
          dpacc = mfma32(lds_read8(tD + off), vf[ks], dpacc);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int ql0 = qb * 32 + 8 * i + 4 * hi;
          const f32x4 l4 = *reinterpret_cast<const f32x4 *>(&tL[ql0]);
          const f32x4 e4 = *reinterpret_cast<const f32x4 *>(&tE[ql0]);
          i32x4 m4 = {-1, -1, -1, -1}, v4 = {kWX, kWX, kWX, kWX};
          if (partial) {
            m4 = *reinterpret_cast<const i32x4 *>(&tM[ql0]);
            v4 = *reinterpret_cast<const i32x4 *>(&tC[ql0]);
          }
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int r = 4 * i + e;
            float p = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[r], a.scale_log2, -l4[e]));
            if (partial) {
              const bool ok = (key <= m4[e]) & (kw >= v4[e]);
              p = ok ? p : 0.f;
            }
            sacc[r] = p;
            dpacc[r] = p * (dpacc[r] - e4[e]);
          }
        }
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const bf16x8 pb = pack8(sacc[8 * u + 0], sacc[8 * u + 1], sacc[8 * u + 2], sacc[8 * u + 3],
                                  sacc[8 * u + 4], sacc[8 * u + 5], sacc[8 * u + 6], sacc[8 * u + 7]);
          const bf16x8 dsb = pack8(dpacc[8 * u + 0], dpacc[8 * u + 1], dpacc[8 * u + 2], dpacc[8 * u + 3],
                                   dpacc[8 * u + 4], dpacc[8 * u + 5], dpacc[8 * u + 6], dpacc[8 * u + 7]);
#pragma unroll
          for (int db = 0; db < DB; ++db) {
            dvacc[db] = mfma32(lds_tr_operand<HD>(tD, tl, qb * 32 + 16 * u, db), pb, dvacc[db]);
            dkacc[db] = mfma32(lds_tr_operand<HD>(tQ, tl, qb * 32 + 16 * u, db), dsb, dkacc[db]);
          }
        }
      }
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
