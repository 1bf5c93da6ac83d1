// MTP block-masked GQA attention backward for gfx950 (the forward is in mga_fwd.hip).
//
// Arithmetic: bf16 operands on v_mfma_f32_32x32x16_bf16, fp32 accumulation,
// softmax in the log2 domain (exp2 of scale*log2(e)*q.k). Semantics follow the
// dense definition of flex_attention ([torch]_higher_order_ops/flex_attention.py
// :202-267 fwd, :826-990 bwd): masked scores are -inf, a fully masked row has
// output 0 and LSE -inf and receives no gradient.
//
// MFMA fragment conventions used throughout (32x32x16, wave64, l32 = lane & 31,
// hi = lane >> 5):
//   A operand (32 x 16):  lane supplies row l32, 8 k-values selected by (hi, slot)
//   B operand (16 x 32):  lane supplies column l32, 8 k-values selected by (hi, slot)
//   C (32 x 32, 16 regs): lane holds column l32, rows 8*(r>>2) + 4*hi + (r&3)
// A and B pair their k-values by (hi, slot), so any fixed assignment of logical
// k indices to (hi, slot) used identically on both operands gives the same
// product. That is what lets an accumulator (C layout) feed the next MFMA as a
// B operand without a shuffle: regs 8u..8u+7 of a lane are the logical k indices
// 16u + 8*(t>>2) + 4*hi + (t&3), t = 0..7, and the A operand is read from LDS in
// the same order (two runs of 4 consecutive elements).
//
// Orientation: the forward and dQ passes compute S^T = K Q^T (keys x queries),
// so each lane owns one query column and the row softmax statistics stay in
// the lane (plus one exchange with the lane 32 away). The dK/dV pass computes
// S = Q K^T (queries x keys), so each lane owns one key column of dK^T / dV^T.
#include "mga_common.hpp"
#include "mga_internal.hpp"

namespace mga {

constexpr float kNegInf = -__builtin_huge_valf();

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// ---------------------------------------------------------------------------
// LDS staging helpers (rows of 8-element vectors; the transposed copy is
// written 4 keys x 1 dim at a time from 4 row loads).
// ---------------------------------------------------------------------------

// dst[r * ROW + c] = src[min(r0 + r, rmax) * ss + c] for r < NR, c < HD
template <int HD, int NR, int ROW, int NT, typename T>
__device__ __forceinline__ void stage_rows(bf16_t *dst, const T *src, int64_t ss, int r0, int rmax) {
  constexpr int V8 = HD / 8;
#pragma unroll
  for (int vi = threadIdx.x; vi < NR * V8; vi += NT) {
    const int r = vi / V8, c = (vi % V8) * 8;
    const int row = min(r0 + r, rmax);
    const bf16x8 x = load8(src + (int64_t)row * ss + c);
    *reinterpret_cast<i32x4 *>(dst + r * ROW + c) = __builtin_bit_cast(i32x4, x);
  }
}

// dst[c * ROW + r] = src[min(r0 + r, rmax) * ss + c] for r < NR, c < HD
template <int HD, int NR, int ROW, int NT, typename T>
__device__ __forceinline__ void stage_rows_t(bf16_t *dst, const T *src, int64_t ss, int r0, int rmax) {
  constexpr int V8 = HD / 8;
#pragma unroll
  for (int it = threadIdx.x; it < (NR / 4) * V8; it += NT) {
    const int dg = it % V8, kg = it / V8;
    bf16x8 rows[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int row = min(r0 + kg * 4 + j, rmax);
      rows[j] = load8(src + (int64_t)row * ss + dg * 8);
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      bf16x4 col;
      col[0] = rows[0][e]; col[1] = rows[1][e]; col[2] = rows[2][e]; col[3] = rows[3][e];
      *reinterpret_cast<i32x2 *>(dst + (dg * 8 + e) * ROW + kg * 4) = __builtin_bit_cast(i32x2, col);
    }
  }
}

// ---------------------------------------------------------------------------
// Backward dK/dV pass over the key tiles that receive gradient (keys >=
// grad_start). One workgroup = one 128-key tile of one kv head, four waves of
// 32 keys; the G query heads of the group are reduced inside the workgroup.
// Per 64-row query block of one head (staged natural and transposed):
//   S = Q K^T, dP = dO V^T, P = exp2(S*c - lse2), dS = P (dP - delta),
//   dV^T += dO^T P,  dK^T += Q^T dS.
// ---------------------------------------------------------------------------
template <int HD, typename T>
__global__ __launch_bounds__(256) void attn_bwd_dkdv_kernel(AttnArgs a, int kt0, int nkt) {
  constexpr int BQ = 64;
  constexpr int KS = HD / 16;
  constexpr int DB = HD / 32;
  constexpr int KROW = HD + 8;
  constexpr int TROW = BQ + 4;
  constexpr int NT = 256;
  __shared__ __attribute__((aligned(16))) bf16_t sQ[BQ * KROW];
  __shared__ __attribute__((aligned(16))) bf16_t sD[BQ * KROW];
  __shared__ __attribute__((aligned(16))) bf16_t sQt[HD * TROW];
  __shared__ __attribute__((aligned(16))) bf16_t sDt[HD * TROW];
  __shared__ __attribute__((aligned(16))) float sL[BQ];
  __shared__ __attribute__((aligned(16))) float sDel[BQ];
  __shared__ __attribute__((aligned(16))) int sC[BQ];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, hi = lane >> 5;
  const int G = a.Hq / a.Hkv;
  const int li = xcd_swizzle(blockIdx.x, nkt * a.Hkv);
  const int g = li / nkt;
  const int kt = kt0 + li % nkt;

  const int key = kt * kBlock + wave * 32 + l32;
  const int kr = min(key, a.L - 1);
  const int kcode = key_code(a.code, key, a.P, a.L);
  const T *kp = reinterpret_cast<const T *>(a.k) + g * a.k_sh + (int64_t)kr * a.k_ss;
  const T *vp = reinterpret_cast<const T *>(a.v) + g * a.v_sh + (int64_t)kr * a.v_ss;
  bf16x8 kf[KS], vf[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    kf[ks] = load8(kp + ks * 16 + hi * 8);
    vf[ks] = load8(vp + ks * 16 + hi * 8);
  }
  f32x16 dkacc[DB], dvacc[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) { dkacc[db] = zero16(); dvacc[db] = zero16(); }

  const int npart = a.q_num[kt];
  const int ntot = npart + a.fq_num[kt];
  const int32_t *pidx = a.q_idx + (int64_t)kt * a.nQ;
  const int32_t *fidx = a.fq_idx + (int64_t)kt * a.nQ;

  for (int it = 0; it < ntot; ++it) {
    const bool partial = it < npart;
    const int qt = partial ? pidx[it] : fidx[it - npart];
    for (int hh = 0; hh < G; ++hh) {
      const int h = g * G + hh;
      const T *qp = reinterpret_cast<const T *>(a.q) + h * a.q_sh;
      const T *dop = reinterpret_cast<const T *>(a.dout) + h * a.do_sh;
      for (int sub = 0; sub < kBlock / BQ; ++sub) {
        const int q0 = qt * kBlock + sub * BQ;
        if (q0 >= a.S) break;
        __syncthreads();
        stage_rows<HD, BQ, KROW, NT>(sQ, qp, a.q_ss, q0, a.S - 1);
        stage_rows<HD, BQ, KROW, NT>(sD, dop, a.do_ss, q0, a.S - 1);
        stage_rows_t<HD, BQ, TROW, NT>(sQt, qp, a.q_ss, q0, a.S - 1);
        stage_rows_t<HD, BQ, TROW, NT>(sDt, dop, a.do_ss, q0, a.S - 1);
        if (tid < BQ) {
          const int q = q0 + tid;
          const bool in = q < a.S;
          sL[tid] = in ? a.lse[(int64_t)h * a.S + q] * kLog2e : 0.f;
          sDel[tid] = in ? a.delta[(int64_t)h * a.S + q] : 0.f;
          sC[tid] = in ? a.code[q] : kCodePad;
        }
        __syncthreads();

#pragma unroll
        for (int qb = 0; qb < BQ / 32; ++qb) {
          f32x16 sacc = zero16(), dpacc = zero16();
#pragma unroll
          for (int ks = 0; ks < KS; ++ks) {
            const bf16x8 aq = lds_read8(sQ + (qb * 32 + l32) * KROW + ks * 16 + hi * 8);
            const bf16x8 ad = lds_read8(sD + (qb * 32 + l32) * KROW + ks * 16 + hi * 8);
            sacc = mfma32(aq, kf[ks], sacc);
            dpacc = mfma32(ad, vf[ks], dpacc);
          }
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int ql0 = qb * 32 + 8 * i + 4 * hi;
            const f32x4 l4 = *reinterpret_cast<const f32x4 *>(sL + ql0);
            const f32x4 d4 = *reinterpret_cast<const f32x4 *>(sDel + ql0);
            const i32x4 c4 = *reinterpret_cast<const i32x4 *>(sC + ql0);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              const int r = 4 * i + j;
              float p = fast_exp2(sacc[r] * a.scale_log2 - l4[j]);
              if (partial && !mtp_allowed(q0 + ql0 + j + a.P, c4[j], key, kcode)) p = 0.f;
              sacc[r] = p;
              dpacc[r] = p * (dpacc[r] - d4[j]);
            }
          }
#pragma unroll
          for (int u = 0; u < 2; ++u) {
            const bf16x8 pb = pack8(sacc[8 * u + 0], sacc[8 * u + 1], sacc[8 * u + 2], sacc[8 * u + 3],
                                    sacc[8 * u + 4], sacc[8 * u + 5], sacc[8 * u + 6], sacc[8 * u + 7]);
            const bf16x8 dsb = pack8(dpacc[8 * u + 0], dpacc[8 * u + 1], dpacc[8 * u + 2],
                                     dpacc[8 * u + 3], dpacc[8 * u + 4], dpacc[8 * u + 5],
                                     dpacc[8 * u + 6], dpacc[8 * u + 7]);
#pragma unroll
            for (int db = 0; db < DB; ++db) {
              const int off = (db * 32 + l32) * TROW + qb * 32 + 16 * u + 4 * hi;
              const bf16x8 adt = lds_read4x2(sDt + off, sDt + off + 8);
              const bf16x8 aqt = lds_read4x2(sQt + off, sQt + off + 8);
              dvacc[db] = mfma32(adt, pb, dvacc[db]);
              dkacc[db] = mfma32(aqt, dsb, dkacc[db]);
            }
          }
        }
      }
    }
  }

  if (key >= a.grad_start && key < a.L) {
    const int64_t row = key - a.grad_start;
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
  }
}

// ---------------------------------------------------------------------------
// Launchers
// ---------------------------------------------------------------------------
template <int HD, typename T>
void dq_launch(const AttnArgs &a, hipStream_t st);   // mga_bwd_dq.hip

template <int HD, typename T>
static void bwd_impl(const AttnArgs &a, int passes, hipStream_t st) {
  if (passes & kBwdDq) dq_launch<HD, T>(a, st);
  const int kt0 = a.grad_start / kBlock;
  const int nkt = a.nKV - kt0;
  if ((passes & kBwdDkDv) && nkt > 0 && a.grad_start < a.L)
    hipLaunchKernelGGL((attn_bwd_dkdv_kernel<HD, T>), dim3(nkt * a.Hkv), dim3(256), 0, st, a, kt0, nkt);
}

void launch_attn_bwd(const AttnArgs &a, int head_dim, bool is_f32, int passes, hipStream_t st) {
  if (head_dim == 128) {
    if (is_f32) bwd_impl<128, float>(a, passes, st); else bwd_impl<128, bf16_t>(a, passes, st);
  } else {
    if (is_f32) bwd_impl<64, float>(a, passes, st); else bwd_impl<64, bf16_t>(a, passes, st);
  }
}

}  // namespace mga
