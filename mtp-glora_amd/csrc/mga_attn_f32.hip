// MTP block-masked GQA attention for fp32 operands on gfx950: forward, dQ
// pass and dK/dV pass on the fp32 matrix cores (v_mfma_f32_32x32x2f32), so an
// fp32 model gets fp32 products and fp32 softmax end to end, as the
// reference's flex path computes in the operand dtype (mtp_glora/args.py:15,
// mtp_glora/trainer/utils.py:68). Semantics as the 16-bit kernels:
// [torch]_higher_order_ops/flex_attention.py:202-267 (forward; a fully masked
// row has output 0 and LSE -inf) and :826-990 (backward, grad_lse = 0).
//
// One MFMA multiplies a 32 x 2 A by a 2 x 32 B: lane (l32, hi) supplies
// A[l32][hi] and B[hi][l32], and its 16 accumulator registers hold column
// l32, rows 8 (r / 4) + 4 hi + r % 4. Products over head_dim pair d =
// (HD / 2) hi + s for s = 0 .. HD / 2 - 1 (any split of the sum works), so
// the lane reads four consecutive dims of one row per 16-byte access. The
// products over keys (or queries) take k-index key(s, hi) = 8 (s / 4) + 4 hi
// + s % 4: the row the lane's accumulator register s already holds, so the
// probabilities and dS feed the next MFMA's B operand from their registers.
//
// Tiles: 32 rows x HD fp32 in LDS with rows padded to HD + 4 floats, so 16
// consecutive rows start 4 banks apart (the 16-byte row reads of 16 lanes
// cover the 64 banks once) and every address is a lane base plus a constant
// (an XOR swizzle would cost one address register per read). A 4-wave
// workgroup stages each tile through registers one step ahead into the other
// of two buffers (one barrier per step).
//
//   forward:  S^T = K Q^T, exact running max per step, O^T += V^T P^T
//   dQ pass:  S^T, dP^T - delta = V dO^T - delta, dS^T = P (dP^T - delta),
//             dQ^T += K^T dS^T, delta = rowsum(O dO) written for the dK/dV pass
//   dK/dV:    a workgroup owns 128 keys of one kv head (32 per wave, keys in
//             the lanes, K and V in registers) and walks the query tiles of
//             the transposed block mask x the G query heads:
//             S = Q K^T, dP = dO V^T, dS = P (dP - delta),
//             dV^T += dO^T P, dK^T += Q^T dS.
#include "mga_common.hpp"
#include "mga_internal.hpp"

namespace mga {

namespace {

constexpr float kNegInfF32 = -__builtin_huge_valf();
constexpr int kR = 32;   // rows of a staged tile (keys or queries per step)

__device__ __forceinline__ f32x16 mfma_f32(float a, float b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

template <int HD>
constexpr int kStride = HD + 4;   // floats per LDS tile row

// the four dims 4 c .. 4 c + 3 of row r
template <int HD>
__device__ __forceinline__ f32x4 row4(const float *t, int r, int c) {
  return *reinterpret_cast<const f32x4 *>(t + r * kStride<HD> + 4 * c);
}

// element (r, col)
template <int HD>
__device__ __forceinline__ float elem(const float *t, int r, int col) {
  return t[r * kStride<HD> + col];
}

// Row index of accumulator register r (and k-index of operand step r) for
// the lane half hi.
__device__ __forceinline__ int acc_row(int r, int hi) { return 8 * (r / 4) + 4 * hi + r % 4; }

// 256 threads stage one 32 x HD fp32 tile: rows r0 .. r0 + 31 of src (row
// stride ss elements), rows past rmax repeating row rmax.
template <int HD>
struct Stage32 {
  static constexpr int kGran = kR * HD / 4 / 256;
  f32x4 reg[kGran];
  __device__ __forceinline__ void load(const float *src, int64_t ss, int r0, int rmax) {
#pragma unroll
    for (int i = 0; i < kGran; ++i) {
      const int gi = threadIdx.x + 256 * i;
      const int r = gi / (HD / 4), c = gi % (HD / 4);
      reg[i] = *reinterpret_cast<const f32x4 *>(src + (int64_t)min(r0 + r, rmax) * ss + 4 * c);
    }
  }
  __device__ __forceinline__ void store(float *tile) const {
#pragma unroll
    for (int i = 0; i < kGran; ++i) {
      const int gi = threadIdx.x + 256 * i;
      const int r = gi / (HD / 4), c = gi % (HD / 4);
      *reinterpret_cast<f32x4 *>(tile + r * kStride<HD> + 4 * c) = reg[i];
    }
  }
};

__host__ __device__ __forceinline__ int heads_per_wg_f32(int G) { return (G % 4 == 0) ? 4 : (G % 2 == 0 ? 2 : 1); }

// Query-side work item of the forward and dQ kernels: 4 waves = HPW heads of
// one kv head x (4 / HPW) blocks of 32 rows.
struct QItem {
  int g, h, row, qt;
};

__device__ __forceinline__ QItem q_item(const AttnArgs &a) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int G = a.Hq / a.Hkv;
  const int HPW = heads_per_wg_f32(G);
  const int QR = kR * (4 / HPW);
  const int nslice = G / HPW;
  const int nqb = (a.S + QR - 1) / QR;
  const int li = xcd_swizzle(blockIdx.x, a.Hkv * nslice * nqb);
  QItem it;
  it.g = li / (nslice * nqb);
  const int rem = li % (nslice * nqb);
  const int qb = nqb - 1 - rem / nslice;
  it.h = it.g * G + (rem % nslice) * HPW + wave % HPW;
  it.row = qb * QR + (wave / HPW) * kR + (lane & 31);
  it.qt = (qb * QR) / kBlock;
  return it;
}

}  // namespace

// ---------------------------------------------------------------------------
// Forward
// ---------------------------------------------------------------------------
template <int HD>
__global__ __launch_bounds__(256, 2) void attn_fwd_f32_kernel(AttnArgs a) {
  constexpr int KH = HD / 2;   // MFMA steps over head_dim
  constexpr int DB = HD / 32;  // 32-dim blocks of O^T
  constexpr int TILE = kR * kStride<HD>;
  __shared__ __attribute__((aligned(16))) float sK0[TILE], sK1[TILE], sV0[TILE], sV1[TILE];
  __shared__ int sW0[kR], sW1[kR];

  const int tid = threadIdx.x, lane = tid & 63, l32 = lane & 31, hi = lane >> 5;
  const QItem it = q_item(a);
  const int row = it.row, qr = min(row, a.S - 1);
  const float *qp = reinterpret_cast<const float *>(a.q) + it.h * a.q_sh + (int64_t)qr * a.q_ss + KH * hi;
  const float *kp = reinterpret_cast<const float *>(a.k) + it.g * a.k_sh;
  const float *vp = reinterpret_cast<const float *>(a.v) + it.g * a.v_sh;

  float qf[KH];
#pragma unroll
  for (int i = 0; i < KH / 4; ++i) {
    const f32x4 x = *reinterpret_cast<const f32x4 *>(qp + 4 * i);
    qf[4 * i] = x[0]; qf[4 * i + 1] = x[1]; qf[4 * i + 2] = x[2]; qf[4 * i + 3] = x[3];
  }
  const int qcode = row < a.S ? a.code[row] : kCodePad;
  const int qv = query_v(qcode);
  const int qlim = qcode == kCodePad ? -1 : row + a.P;   // a pad row (or past S) sees no key

  TileList tiles = tile_list(a.kv_num, a.kv_idx, a.fkv_num, a.fkv_idx, it.qt, a.nKV);
  constexpr int kSub = kBlock / kR;
  const int nstep = kSub * tiles.ntot;
  auto step_base = [&](int j) { return tiles.at(j / kSub) * kBlock + (j % kSub) * kR; };

  Stage32<HD> stK, stV;
  KeyCode wkey;
  auto load_step = [&](int j) {
    const int kb = step_base(j);
    stK.load(kp, a.k_ss, kb, a.L - 1);
    stV.load(vp, a.v_ss, kb, a.L - 1);
    if (tid < kR) wkey.load(a.code, kb + tid, a.P, a.L);
  };
  auto store_step = [&](float *dK, float *dV, int *dW) {
    stK.store(dK);
    stV.store(dV);
    if (tid < kR) dW[tid] = wkey.w();
  };

  const float c = a.scale_log2;
  float m_run = kNegInfF32, l_run = 0.f;
  f32x16 oacc[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) oacc[db] = zero16();

  auto run_step = [&](const float *tK, const float *tV, const int *tW, int j) {
    const int kbase = step_base(j);
    if (kbase >= a.L) return;
    // operands of group i + 1 read before the MFMAs of group i (the
    // scheduling barriers stop the compiler from hoisting every read)
    f32x16 s = zero16();
    f32x4 kr = row4<HD>(tK, l32, KH / 4 * hi);
#pragma unroll
    for (int i = 0; i < KH / 4; ++i) {
      f32x4 kn;
      if (i + 1 < KH / 4) kn = row4<HD>(tK, l32, KH / 4 * hi + i + 1);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int e = 0; e < 4; ++e) s = mfma_f32(kr[e], qf[4 * i + e], s);
      __builtin_amdgcn_sched_barrier(0);
      if (i + 1 < KH / 4) kr = kn;
    }
    float mx = kNegInfF32;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int ko = acc_row(r, hi);
      const bool ok = (tW[ko] >= qv) & (kbase + ko <= qlim);
      s[r] = ok ? s[r] * c : kNegInfF32;
      mx = fmaxf(mx, s[r]);
    }
    mx = fmaxf(mx, xor32(mx));
    const float m_new = fmaxf(m_run, mx);
    // nothing visible yet: probabilities 0 and nothing to rescale
    const float m_use = m_new == kNegInfF32 ? 0.f : m_new;
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);   // 0 while m_run = -inf
    m_run = m_new;
    float ps = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      s[r] = __builtin_amdgcn_exp2f(s[r] - m_use);
      ps += s[r];
    }
    l_run = l_run * alpha + ps;
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int r = 0; r < 16; ++r) oacc[db][r] *= alpha;
    float av[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db) av[db] = elem<HD>(tV, acc_row(0, hi), 32 * db + l32);
#pragma unroll
    for (int t = 0; t < 16; ++t) {
      float nv[DB];
      if (t + 1 < 16)
#pragma unroll
        for (int db = 0; db < DB; ++db) nv[db] = elem<HD>(tV, acc_row(t + 1, hi), 32 * db + l32);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int db = 0; db < DB; ++db) oacc[db] = mfma_f32(av[db], s[t], oacc[db]);
      __builtin_amdgcn_sched_barrier(0);
      if (t + 1 < 16)
#pragma unroll
        for (int db = 0; db < DB; ++db) av[db] = nv[db];
    }
  };

  if (nstep > 0) {
    load_step(0);
    store_step(sK0, sV0, sW0);
  }
  __syncthreads();
  // two steps per iteration, one per buffer: both code paths see fixed
  // buffers, and the accumulators stay in place across them
  for (int j = 0; j < nstep; j += 2) {
    if (j + 1 < nstep) load_step(j + 1);
    run_step(sK0, sV0, sW0, j);
    if (j + 1 < nstep) store_step(sK1, sV1, sW1);
    __syncthreads();
    if (j + 1 < nstep) {
      if (j + 2 < nstep) load_step(j + 2);
      run_step(sK1, sV1, sW1, j + 1);
      if (j + 2 < nstep) store_step(sK0, sV0, sW0);
      __syncthreads();
    }
  }

  const float lt = l_run + xor32(l_run);
  if (row < a.S) {
    const float inv = lt > 0.f ? 1.f / lt : 0.f;
    if (hi == 0) a.lse[(int64_t)it.h * a.S + row] = lt > 0.f ? (m_run + __log2f(lt)) * kLn2 : kNegInfF32;
    float *orow = reinterpret_cast<float *>(const_cast<void *>(a.o)) + it.h * a.o_sh + (int64_t)row * a.o_ss;
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        store4(orow + db * 32 + 8 * i + 4 * hi, oacc[db][4 * i] * inv, oacc[db][4 * i + 1] * inv,
               oacc[db][4 * i + 2] * inv, oacc[db][4 * i + 3] * inv);
  }
}

// ---------------------------------------------------------------------------
// Backward, dQ pass (also writes delta)
// ---------------------------------------------------------------------------
template <int HD>
__global__ __launch_bounds__(256, 1) void attn_bwd_dq_f32_kernel(AttnArgs a) {
  constexpr int KH = HD / 2;
  constexpr int DB = HD / 32;
  constexpr int TILE = kR * kStride<HD>;
  __shared__ __attribute__((aligned(16))) float sK0[TILE], sK1[TILE], sV0[TILE], sV1[TILE];
  __shared__ int sW0[kR], sW1[kR];

  const int tid = threadIdx.x, lane = tid & 63, l32 = lane & 31, hi = lane >> 5;
  const QItem it = q_item(a);
  const int row = it.row, qr = min(row, a.S - 1);
  const bool in = row < a.S;
  const float *qp = reinterpret_cast<const float *>(a.q) + it.h * a.q_sh + (int64_t)qr * a.q_ss + KH * hi;
  const float *dop = reinterpret_cast<const float *>(a.dout) + it.h * a.do_sh + (int64_t)qr * a.do_ss + KH * hi;
  const float *op = reinterpret_cast<const float *>(a.o) + it.h * a.o_sh + (int64_t)qr * a.o_ss + KH * hi;
  const float *kp = reinterpret_cast<const float *>(a.k) + it.g * a.k_sh;
  const float *vp = reinterpret_cast<const float *>(a.v) + it.g * a.v_sh;

  float qf[KH], dof[KH];
  float del = 0.f;
#pragma unroll
  for (int i = 0; i < KH / 4; ++i) {
    const f32x4 x = *reinterpret_cast<const f32x4 *>(qp + 4 * i);
    const f32x4 d = *reinterpret_cast<const f32x4 *>(dop + 4 * i);
    const f32x4 o = *reinterpret_cast<const f32x4 *>(op + 4 * i);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      qf[4 * i + e] = x[e];
      dof[4 * i + e] = d[e];
      del += o[e] * d[e];
    }
  }
  del += xor32(del);
  if (!in) del = 0.f;
  if (in && hi == 0) a.delta[(int64_t)it.h * a.S + row] = del;
  const float lse = in ? a.lse[(int64_t)it.h * a.S + row] : kNegInfF32;
  const float lse2 = lse == kNegInfF32 ? 0.f : lse * kLog2e;
  const int qcode = in ? a.code[row] : kCodePad;
  const int qv = query_v(qcode);
  const int qlim = (qcode == kCodePad || lse == kNegInfF32) ? -1 : row + a.P;

  TileList tiles = tile_list(a.kv_num, a.kv_idx, a.fkv_num, a.fkv_idx, it.qt, a.nKV);
  constexpr int kSub = kBlock / kR;
  const int nstep = kSub * tiles.ntot;
  auto step_base = [&](int j) { return tiles.at(j / kSub) * kBlock + (j % kSub) * kR; };

  Stage32<HD> stK, stV;
  KeyCode wkey;
  auto load_step = [&](int j) {
    const int kb = step_base(j);
    stK.load(kp, a.k_ss, kb, a.L - 1);
    stV.load(vp, a.v_ss, kb, a.L - 1);
    if (tid < kR) wkey.load(a.code, kb + tid, a.P, a.L);
  };
  auto store_step = [&](float *dK, float *dV, int *dW) {
    stK.store(dK);
    stV.store(dV);
    if (tid < kR) dW[tid] = wkey.w();
  };

  const float c = a.scale_log2;
  f32x16 dqacc[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) dqacc[db] = zero16();

  auto run_step = [&](const float *tK, const float *tV, const int *tW, int j) {
    const int kbase = step_base(j);
    if (kbase >= a.L) return;
    f32x16 s = zero16(), dp;
#pragma unroll
    for (int r = 0; r < 16; ++r) dp[r] = -del;
    f32x4 kr = row4<HD>(tK, l32, KH / 4 * hi), vr = row4<HD>(tV, l32, KH / 4 * hi);
#pragma unroll
    for (int i = 0; i < KH / 4; ++i) {
      f32x4 kn, vn;
      if (i + 1 < KH / 4) {
        kn = row4<HD>(tK, l32, KH / 4 * hi + i + 1);
        vn = row4<HD>(tV, l32, KH / 4 * hi + i + 1);
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        s = mfma_f32(kr[e], qf[4 * i + e], s);
        dp = mfma_f32(vr[e], dof[4 * i + e], dp);
      }
      __builtin_amdgcn_sched_barrier(0);
      if (i + 1 < KH / 4) {
        kr = kn;
        vr = vn;
      }
    }
    // dS^T = P (dP^T - delta), P = exp2(s c - lse2), 0 where masked
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int ko = acc_row(r, hi);
      const bool ok = (tW[ko] >= qv) & (kbase + ko <= qlim);
      dp[r] = ok ? __builtin_amdgcn_exp2f(__builtin_fmaf(s[r], c, -lse2)) * dp[r] : 0.f;
    }
    float ak[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db) ak[db] = elem<HD>(tK, acc_row(0, hi), 32 * db + l32);
#pragma unroll
    for (int t = 0; t < 16; ++t) {
      float nk[DB];
      if (t + 1 < 16)
#pragma unroll
        for (int db = 0; db < DB; ++db) nk[db] = elem<HD>(tK, acc_row(t + 1, hi), 32 * db + l32);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int db = 0; db < DB; ++db) dqacc[db] = mfma_f32(ak[db], dp[t], dqacc[db]);
      __builtin_amdgcn_sched_barrier(0);
      if (t + 1 < 16)
#pragma unroll
        for (int db = 0; db < DB; ++db) ak[db] = nk[db];
    }
  };

  if (nstep > 0) {
    load_step(0);
    store_step(sK0, sV0, sW0);
  }
  __syncthreads();
  // two steps per iteration, one per buffer: both code paths see fixed
  // buffers, and the accumulators stay in place across them
  for (int j = 0; j < nstep; j += 2) {
    if (j + 1 < nstep) load_step(j + 1);
    run_step(sK0, sV0, sW0, j);
    if (j + 1 < nstep) store_step(sK1, sV1, sW1);
    __syncthreads();
    if (j + 1 < nstep) {
      if (j + 2 < nstep) load_step(j + 2);
      run_step(sK1, sV1, sW1, j + 1);
      if (j + 2 < nstep) store_step(sK0, sV0, sW0);
      __syncthreads();
    }
  }

  if (in) {
    float *out = reinterpret_cast<float *>(a.dq) + it.h * a.dq_sh + (int64_t)row * a.dq_ss;
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        store4(out + db * 32 + 8 * i + 4 * hi, dqacc[db][4 * i] * a.scale, dqacc[db][4 * i + 1] * a.scale,
               dqacc[db][4 * i + 2] * a.scale, dqacc[db][4 * i + 3] * a.scale);
  }
}

// ---------------------------------------------------------------------------
// Backward, dK/dV pass (reads the delta of the dQ pass)
// ---------------------------------------------------------------------------
template <int HD>
__global__ __launch_bounds__(256, 1) void attn_bwd_dkdv_f32_kernel(AttnArgs a, int kt0) {
  constexpr int KH = HD / 2;
  constexpr int DB = HD / 32;
  constexpr int TILE = kR * kStride<HD>;
  __shared__ __attribute__((aligned(16))) float sQ0[TILE], sQ1[TILE], sD0[TILE], sD1[TILE];
  // per query row of a step: lse (log2 units; 0 for a row that sees nothing),
  // delta, ordered-compare value and causal bound (-1: the row sees no key)
  __shared__ __attribute__((aligned(16))) float sL0[kR], sL1[kR], sE0[kR], sE1[kR];
  __shared__ __attribute__((aligned(16))) int sV0[kR], sV1[kR], sM0[kR], sM1[kR];

  const int tid = threadIdx.x, lane = tid & 63, l32 = lane & 31, hi = lane >> 5, wave = tid >> 6;
  const int G = a.Hq / a.Hkv;
  const int nkt = a.nKV - kt0;
  const int li = xcd_swizzle(blockIdx.x, a.Hkv * nkt);
  const int g = li / nkt;
  const int kt = kt0 + li % nkt;
  const int key = kt * kBlock + kR * wave + l32;
  const int kr = min(key, a.L - 1);
  const int kw = key_w(a.code, key, a.P, a.L);

  // this lane's key: K and V dims (KH) hi + s
  float kf[KH], vf[KH];
  {
    const float *kp = reinterpret_cast<const float *>(a.k) + g * a.k_sh + (int64_t)kr * a.k_ss + KH * hi;
    const float *vp = reinterpret_cast<const float *>(a.v) + g * a.v_sh + (int64_t)kr * a.v_ss + KH * hi;
#pragma unroll
    for (int i = 0; i < KH / 4; ++i) {
      const f32x4 x = *reinterpret_cast<const f32x4 *>(kp + 4 * i);
      const f32x4 y = *reinterpret_cast<const f32x4 *>(vp + 4 * i);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        kf[4 * i + e] = x[e];
        vf[4 * i + e] = y[e];
      }
    }
  }

  TileList tiles = tile_list(a.q_num, a.q_idx, a.fq_num, a.fq_idx, kt, a.nQ);
  constexpr int kSub = kBlock / kR;
  const int per_tile = kSub * G;
  const int nstep = per_tile * tiles.ntot;
  // step j: query tile j / per_tile, 32-row block, head of the kv group
  auto step_q0 = [&](int j) { return tiles.at(j / per_tile) * kBlock + ((j % per_tile) / G) * kR; };
  auto step_h = [&](int j) { return g * G + (j % per_tile) % G; };

  Stage32<HD> stQ, stD;
  float rl = 0.f, re = 0.f;
  int rv = 0, rm = -1;
  auto load_step = [&](int j) {
    const int q0 = step_q0(j), h = step_h(j);
    if (q0 >= a.S) return;   // no rows: never computed
    stQ.load(reinterpret_cast<const float *>(a.q) + h * a.q_sh, a.q_ss, q0, a.S - 1);
    stD.load(reinterpret_cast<const float *>(a.dout) + h * a.do_sh, a.do_ss, q0, a.S - 1);
    if (tid < kR) {
      const int q = q0 + tid;
      rl = 0.f; re = 0.f; rv = 0; rm = -1;
      if (q < a.S) {
        const int qc = a.code[q];
        const float lse = a.lse[(int64_t)h * a.S + q];
        re = a.delta[(int64_t)h * a.S + q];
        rv = query_v(qc);
        if (qc != kCodePad && lse != kNegInfF32) {
          rm = q + a.P;
          rl = lse * kLog2e;
        }
      }
    }
  };
  auto store_step = [&](int j, float *dQ, float *dD, float *dL, float *dE, int *dV, int *dM) {
    if (step_q0(j) >= a.S) return;
    stQ.store(dQ);
    stD.store(dD);
    if (tid < kR) {
      dL[tid] = rl; dE[tid] = re; dV[tid] = rv; dM[tid] = rm;
    }
  };

  const float c = a.scale_log2;
  f32x16 dk[DB], dv[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) {
    dk[db] = zero16();
    dv[db] = zero16();
  }

  auto run_step = [&](const float *tQ, const float *tD, const float *tL, const float *tE, const int *tV,
                      const int *tM, int j) {
    if (step_q0(j) >= a.S) return;
    // S = Q K^T and dP = dO V^T: registers are query rows, the lane's column
    // its key. Operands of group i + 1 are read before the MFMAs of group i;
    // the scheduling barriers keep every read from being hoisted further (all
    // of a step's reads in flight at once would exceed the register file).
    f32x16 s = zero16(), dp = zero16();
    f32x4 qr = row4<HD>(tQ, l32, KH / 4 * hi), dr = row4<HD>(tD, l32, KH / 4 * hi);
#pragma unroll
    for (int i = 0; i < KH / 4; ++i) {
      f32x4 qn, dn;
      if (i + 1 < KH / 4) {
        qn = row4<HD>(tQ, l32, KH / 4 * hi + i + 1);
        dn = row4<HD>(tD, l32, KH / 4 * hi + i + 1);
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        s = mfma_f32(qr[e], kf[4 * i + e], s);
        dp = mfma_f32(dr[e], vf[4 * i + e], dp);
      }
      __builtin_amdgcn_sched_barrier(0);
      if (i + 1 < KH / 4) {
        qr = qn;
        dr = dn;
      }
    }
    // P and dS = P (dP - delta); rows r: 8 (r / 4) + 4 hi + r % 4, four at a time
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r0 = 8 * i + 4 * hi;
      const f32x4 l4 = *reinterpret_cast<const f32x4 *>(tL + r0);
      const f32x4 e4 = *reinterpret_cast<const f32x4 *>(tE + r0);
      const i32x4 v4 = *reinterpret_cast<const i32x4 *>(tV + r0);
      const i32x4 m4 = *reinterpret_cast<const i32x4 *>(tM + r0);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int r = 4 * i + e;
        const bool ok = (key <= m4[e]) & (kw >= v4[e]);
        const float p = ok ? __builtin_amdgcn_exp2f(__builtin_fmaf(s[r], c, -l4[e])) : 0.f;
        s[r] = p;
        dp[r] = p * (dp[r] - e4[e]);
      }
    }
    // dV^T += dO^T P, dK^T += Q^T dS (k-index: query row acc_row(t, hi)),
    // operands of t + 1 read before the MFMAs of t
    float ad[DB], aq[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db) {
      ad[db] = elem<HD>(tD, acc_row(0, hi), 32 * db + l32);
      aq[db] = elem<HD>(tQ, acc_row(0, hi), 32 * db + l32);
    }
#pragma unroll
    for (int t = 0; t < 16; ++t) {
      float nd[DB], nq[DB];
      if (t + 1 < 16)
#pragma unroll
        for (int db = 0; db < DB; ++db) {
          nd[db] = elem<HD>(tD, acc_row(t + 1, hi), 32 * db + l32);
          nq[db] = elem<HD>(tQ, acc_row(t + 1, hi), 32 * db + l32);
        }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        dv[db] = mfma_f32(ad[db], s[t], dv[db]);
        dk[db] = mfma_f32(aq[db], dp[t], dk[db]);
      }
      __builtin_amdgcn_sched_barrier(0);
      if (t + 1 < 16)
#pragma unroll
        for (int db = 0; db < DB; ++db) {
          ad[db] = nd[db];
          aq[db] = nq[db];
        }
    }
  };

  if (nstep > 0) {
    load_step(0);
    store_step(0, sQ0, sD0, sL0, sE0, sV0, sM0);
  }
  __syncthreads();
  for (int j = 0; j < nstep; j += 2) {
    if (j + 1 < nstep) load_step(j + 1);
    run_step(sQ0, sD0, sL0, sE0, sV0, sM0, j);
    if (j + 1 < nstep) store_step(j + 1, sQ1, sD1, sL1, sE1, sV1, sM1);
    __syncthreads();
    if (j + 1 < nstep) {
      if (j + 2 < nstep) load_step(j + 2);
      run_step(sQ1, sD1, sL1, sE1, sV1, sM1, j + 1);
      if (j + 2 < nstep) store_step(j + 2, sQ0, sD0, sL0, sE0, sV0, sM0);
      __syncthreads();
    }
  }

  // lane = key, registers = dims 32 db + 8 (r / 4) + 4 hi + r % 4
  if (key >= a.grad_start && key < a.L) {
    const int64_t r = key - a.grad_start;
    float *dko = reinterpret_cast<float *>(a.dk) + g * a.dk_sh + r * a.dk_ss;
    float *dvo = reinterpret_cast<float *>(a.dv) + g * a.dv_sh + r * a.dv_ss;
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        store4(dko + db * 32 + 8 * i + 4 * hi, dk[db][4 * i] * a.scale, dk[db][4 * i + 1] * a.scale,
               dk[db][4 * i + 2] * a.scale, dk[db][4 * i + 3] * a.scale);
        store4(dvo + db * 32 + 8 * i + 4 * hi, dv[db][4 * i], dv[db][4 * i + 1], dv[db][4 * i + 2],
               dv[db][4 * i + 3]);
      }
  }
}

template __global__ void attn_fwd_f32_kernel<128>(AttnArgs);
template __global__ void attn_fwd_f32_kernel<64>(AttnArgs);
template __global__ void attn_bwd_dq_f32_kernel<128>(AttnArgs);
template __global__ void attn_bwd_dq_f32_kernel<64>(AttnArgs);
template __global__ void attn_bwd_dkdv_f32_kernel<128>(AttnArgs, int);
template __global__ void attn_bwd_dkdv_f32_kernel<64>(AttnArgs, int);

namespace {

int q_items(const AttnArgs &a) {
  const int G = a.Hq / a.Hkv;
  const int HPW = heads_per_wg_f32(G);
  const int QR = kR * (4 / HPW);
  return a.Hkv * (G / HPW) * ((a.S + QR - 1) / QR);
}

template <int HD>
void bwd_f32(const AttnArgs &a, int passes, hipStream_t st) {
  if (passes & kBwdDq) hipLaunchKernelGGL((attn_bwd_dq_f32_kernel<HD>), dim3(q_items(a)), dim3(256), 0, st, a);
  if ((passes & kBwdDkDv) && a.grad_start < a.L) {
    const int kt0 = a.grad_start / kBlock;
    hipLaunchKernelGGL((attn_bwd_dkdv_f32_kernel<HD>), dim3(a.Hkv * (a.nKV - kt0)), dim3(256), 0, st, a, kt0);
  }
}

}  // namespace

void launch_attn_fwd_f32(const AttnArgs &a, int head_dim, hipStream_t st) {
  if (head_dim == 128) hipLaunchKernelGGL((attn_fwd_f32_kernel<128>), dim3(q_items(a)), dim3(256), 0, st, a);
  else hipLaunchKernelGGL((attn_fwd_f32_kernel<64>), dim3(q_items(a)), dim3(256), 0, st, a);
}

void launch_attn_bwd_f32(const AttnArgs &a, int head_dim, int passes, hipStream_t st) {
  if (head_dim == 128) bwd_f32<128>(a, passes, st);
  else bwd_f32<64>(a, passes, st);
}

}  // namespace mga
