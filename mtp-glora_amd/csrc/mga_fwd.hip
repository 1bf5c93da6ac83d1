// MTP block-masked GQA attention forward for gfx950.
//
// Work item = (kv head g, slice of the G query heads, block of query rows).
// A wave holds one (query head, 32-row block) pair of one kv head and
// computes
//   S^T = K Q^T  (v_mfma_f32_32x32x16_bf16 / _f16; lane = query column)
// over 64-key steps, keeps the online-softmax state of its queries in the lane
// (plus one exchange with the lane 32 away) and accumulates O^T += V^T P^T,
// feeding the probabilities from registers straight into the B operand. V^T
// comes from the row-major V tile through the LDS transpose read. Each K/V
// tile staged in LDS feeds every wave of the workgroup (with G a multiple of
// 4: 4 heads x the same rows per 4 waves). 2 waves per SIMD. Three forms:
// * pair (G even): 8 waves, two 4-wave row blocks per item. A step is a
//   softmax interval (VALU work only) and a product interval (the O^T update
//   and the next step's scores: MFMAs only), one barrier each; the second
//   block runs one interval behind the first, so each SIMD holds one wave in
//   its softmax and one issuing MFMAs (a SIMD overlaps one wave's VALU work
//   with another's MFMAs far better than the two kinds within one wave).
// * 4-wave (G odd): one row block per workgroup, two workgroups per CU; the
//   scores of step j + 1 are computed while the softmax of step j runs, in
//   one scheduling region whose MFMAs and VALU instructions are interleaved,
//   then O^T takes step j's probabilities (one barrier per step).
// * split: a last round of items that would leave half of an XCD's workgroup
//   slots empty runs each row block as an 8-wave workgroup whose two 4-wave
//   groups split the tile list (as in the 4-wave form) and merge through LDS.
// K runs one step ahead of V: while the K tile of step j + 1 and the V tile of
// step j are read, the K tile of step j + 2 and the V tile of step j + 1 load
// straight into the two other named buffers.
//
// Softmax without a per-step row max: probabilities are exp2(s * c - m) with
// m the row's running offset, and a step is accepted when every lane's partial
// row sum is at most 2^20 (so is every probability; 2^15 for fp16). Otherwise
// (a row's first unmasked scores, or a score more than 20 log2 units above m)
// the step takes the slow path: m moves to the exact running max, O and the
// row sum are rescaled and the probabilities recomputed from the scores still
// held in registers. Row sums add the fp32 probabilities, before they are
// rounded to the operand type for the O update, as the reference's kernel
// does ([torch]_inductor/kernel/flex/templates/common.py.jinja:101, 114).
// Masking runs only on partial tiles: one ordered compare per score (see
// key_w; it also masks pad rows), plus the causal bound only on the steps
// whose keys reach past the wave's first query.
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

// scheduling-group masks (AMDGPU sched_group_barrier)
constexpr int kSgMfma = 0x008;
constexpr int kSgValu = 0x002 | 0x400;   // VALU and transcendental
constexpr int kSgDsRead = 0x100;

__device__ __forceinline__ float exp2f_(float x) { return __builtin_amdgcn_exp2f(x); }

// Heads sharing a workgroup (a divisor of both G and 4).
__host__ __device__ __forceinline__ int heads_per_wg(int G) { return (G % 4 == 0) ? 4 : (G % 2 == 0 ? 2 : 1); }
// Row blocks of 4 waves per item: 2 when the heads split into slices of 2 or
// 4 (an item's rows then still lie in one 128-row query tile), else 1.
__host__ __device__ __forceinline__ int units_per_item(int HPW) { return HPW >= 2 ? 2 : 1; }

enum { kFwd4 = 0, kFwdPair = 1, kFwdSplit = 2 };

}  // namespace

// An item is (kv head, slice of HPW query heads, U consecutive blocks of
// 4 * 32 / HPW rows), U = units_per_item; a wave holds one (query head,
// 32-row block) pair. Forms:
// * kFwdPair (U = 2): 8 waves, one workgroup per CU; each staged K/V tile
//   feeds all 8 waves (half the tile loads and LDS writes per MFMA of two
//   4-wave workgroups sharing the CU). A step runs as two barrier intervals,
//   the softmax (V: VALU work only) and the products (M: the O^T update and
//   the next step's scores), and the second row block (waves 4-7, each
//   sharing a SIMD with one of waves 0-3) runs one interval behind the
//   first: each SIMD holds one wave in its softmax while the other issues
//   MFMAs, instead of two waves held in the same phase.
// * kFwd4 (U = 1): 4 waves, two workgroups per CU.
// * kFwdSplit: each row block of an item as an 8-wave workgroup whose two
//   4-wave groups take the even and the odd entries of the tile list and
//   merge (O, offset, row sum) through LDS at the end, so the block takes
//   about half as long (for a last round of workgroups that would leave half
//   the GPU idle).
// The launch runs items [k1, k1 + kn) of each XCD's share.
template <int HD, typename T, int MODE>
__global__ __launch_bounds__(MODE == kFwd4 ? 256 : 512, 2) void attn_fwd_kernel(AttnArgs a, int k1, int kn) {
  constexpr int NG = MODE == kFwdSplit ? 2 : 1;    // groups splitting the tile list
  constexpr int NWD = 4;                           // waves loading each staged tile
  typedef typename MfmaElem<T>::type E;
  constexpr int KS = HD / 16;          // k-steps of QK^T over head_dim
  constexpr int DB = HD / 32;          // 32-dim blocks of O^T
  constexpr int TILE = kStepKeys * HD; // elements of one K or V step tile
  // [group][TILE]: each 4-wave group stages the K/V tiles of its own keys
  __shared__ __attribute__((aligned(16))) bf16_t sK0[NG * TILE], sK1[NG * TILE];
  __shared__ __attribute__((aligned(16))) bf16_t sV0[NG * TILE], sV1[NG * TILE];
  __shared__ __attribute__((aligned(16))) int sW0[NG * kStepKeys], sW1[NG * kStepKeys];

  const int tid = threadIdx.x, lane = tid & 63;
  const int grp = NG == 2 ? wave_id() >> 2 : 0;                // the group's entries: grp, grp + NG, ...
  const int wave = NG == 2 ? wave_id() & 3 : wave_id();        // wave among those holding the rows
  const int gtid = NG == 2 ? tid & 255 : tid;
  const int l32 = lane & 31, hi = lane >> 5;
  const int G = a.Hq / a.Hkv;
  const int HPW = heads_per_wg(G);
  const int QR4 = 32 * (4 / HPW);         // rows of 4 waves (<= 128)
  const int U = units_per_item(HPW);
  const int QU = U * QR4;                 // rows of an item (<= 128)
  const int nslice = G / HPW;
  const int nqb = (a.S + QU - 1) / QU;

  // logical item: kv head major (one kv head per XCD when Hkv = 8), then query
  // blocks from the last (longest) to the first, then the head slice
  // item: XCD x = blockIdx % 8 runs the contiguous share x0 .. x0 + n_x - 1
  // of the logical items (kv head major, longest first), this launch its
  // entries k1 .. k1 + kn - 1
  // (a kFwdSplit workgroup: entry t / U, row block t % U of it)
  const int n_items = a.Hkv * nslice * nqb;
  const int xcd = blockIdx.x & 7;
  const int t = (int)(blockIdx.x >> 3);
  const int o = k1 + (MODE == kFwdSplit ? t / U : t);
  const int n_x = n_items / 8 + (xcd < n_items % 8 ? 1 : 0);
  if (o >= n_x || o >= k1 + kn) return;
  const int li = xcd * (n_items / 8) + min(xcd, n_items % 8) + o;
  const int g = li / (nslice * nqb);
  const int rem = li % (nslice * nqb);
  const int qb = nqb - 1 - rem / nslice;
  const int slice = rem % nslice;
  const int wg_row0 = qb * QU + (MODE == kFwdSplit ? (t % U) * QR4 : 0);
  const int h = g * G + slice * HPW + wave % HPW;
  const int row0 = wg_row0 + (wave / HPW) * 32;        // first row of this wave
  const int qt = wg_row0 / kBlock;                     // block-mask query tile

  const T *qp = reinterpret_cast<const T *>(a.q) + h * a.q_sh;
  const T *kp = reinterpret_cast<const T *>(a.k) + g * a.k_sh;
  const T *vp = reinterpret_cast<const T *>(a.v) + g * a.v_sh;

  // lane owns query row0 + l32
  const int row = row0 + l32;
  bf16x8 qf[KS];
  {
    const int qr = min(row, a.S - 1);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) qf[ks] = load8(qp + (int64_t)qr * a.q_ss + ks * 16 + hi * 8);
  }
  const int qcode = row < a.S ? a.code[row] : kCodePad;   // a row past S is a pad
  const int qv = query_v(qcode);
  const int qlim = row + a.P;        // causal bound
  const int diag = row0 + a.P;       // keys up to here precede every query of the wave

  TileList tiles = tile_list(a.kv_num, a.kv_idx, a.fkv_num, a.fkv_idx, qt, a.nKV);
  const int npart = tiles.npart;
  const int nstep = kStepsPerTile * ((tiles.ntot - grp + NG - 1) / NG);   // this group's steps
  const int nloop = kStepsPerTile * ((tiles.ntot + NG - 1) / NG);        // group 0's (>= group 1's)
  auto tile_of = [&](int j) { return NG * (j / kStepsPerTile) + grp; };
  auto step_base = [&](int j) { return tiles.at(tile_of(j)) * kBlock + (j % kStepsPerTile) * kStepKeys; };

  // per-lane LDS offsets: K rows (A operand of QK^T) and the V^T transpose reads
  // K operand of k-step ks: row l32 (+ 32 kb), granule (2 ks + hi) ^ swz(l32),
  // i.e. byte offset krow ^ (ks << 5)
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

  BufDma<HD, kStepKeys, NWD> dmaK, dmaV;
  dmaK.init(a.k_ss);
  dmaV.init(a.v_ss);
  KeyCode wkey;
  // rows past L (the last tile's tail) arrive as zeros; a step that starts
  // past L (the second half of the last tile) is never computed: no loads
  auto load_tile = [&](int kb, bf16_t *dst, const T *src, int64_t ss, const BufDma<HD, kStepKeys, NWD> &d) {
    if (kb < a.L) d.issue(dst + grp * TILE, reinterpret_cast<const bf16_t *>(src) + (int64_t)kb * ss, ss, a.L - kb);
  };
  auto load_k = [&](int j, bf16_t *dK) { load_tile(step_base(j), dK, kp, a.k_ss, dmaK); };
  // the keys' raw codes of step j, read before any tile load of the step:
  // the compiler, which does not see the tile loads, waits for every
  // outstanding load before it writes the code register (and converting the
  // code here would wait for the read)
  auto load_w = [&](int j) {
    if (gtid < kStepKeys) wkey.load(a.code, step_base(j) + gtid, a.P, a.L);
  };
  auto load_v = [&](int j, bf16_t *dV) { load_tile(step_base(j), dV, vp, a.v_ss, dmaV); };
  auto store_w = [&](int *dW) {
    if (gtid < kStepKeys)
      *reinterpret_cast<int *>(const_cast<char *>(lds_at(dW + grp * kStepKeys, opaque_u32(gtid * 4u)))) = wkey.w();
  };

  const float c = a.scale_log2;
  float m_run = qcode == kCodePad ? 0.f : kNegInfF;   // a pad row never needs an offset
  float l_run = 0.f;
  f32x16 oacc[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) oacc[db] = zero16();
  // scores of the steps of even / odd parity: register r of sacc[p][kb] is key
  // kb * 32 + 8 (r / 4) + 4 hi + r % 4 of the step
  f32x16 sacc[2][kStepBlocks];

  auto kread = [&](const bf16_t *tK, int ks, int kb) {
    return lds_read8(reinterpret_cast<const bf16_t *>(lds_at(tK + kb * 32 * HD, krow ^ (uint32_t)(ks << 5))));
  };
  // S^T = K Q^T of one step, K operands read one k-step ahead (kept in that
  // order by scheduling barriers)
  auto scores = [&](const bf16_t *tK, f32x16 (&s)[kStepBlocks]) {
#pragma unroll
    for (int kb = 0; kb < kStepBlocks; ++kb) s[kb] = zero16();
    bf16x8 ka[kStepBlocks];
#pragma unroll
    for (int kb = 0; kb < kStepBlocks; ++kb) ka[kb] = kread(tK, 0, kb);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      bf16x8 kn[kStepBlocks];
      if (ks + 1 < KS)
#pragma unroll
        for (int kb = 0; kb < kStepBlocks; ++kb) kn[kb] = kread(tK, ks + 1, kb);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int kb = 0; kb < kStepBlocks; ++kb) s[kb] = mfma32<E>(ka[kb], qf[ks], s[kb]);
      __builtin_amdgcn_sched_barrier(0);
      if (ks + 1 < KS)
#pragma unroll
        for (int kb = 0; kb < kStepBlocks; ++kb) ka[kb] = kn[kb];
    }
  };
  // the same inside a fused region: no read-ahead (the interleaved VALU work
  // covers the LDS latency) and no fences
  auto scores_fused = [&](const bf16_t *tK, f32x16 (&s)[kStepBlocks]) {
#pragma unroll
    for (int kb = 0; kb < kStepBlocks; ++kb) s[kb] = zero16();
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      bf16x8 ka[kStepBlocks];
#pragma unroll
      for (int kb = 0; kb < kStepBlocks; ++kb) ka[kb] = kread(tK, ks, kb);
#pragma unroll
      for (int kb = 0; kb < kStepBlocks; ++kb) s[kb] = mfma32<E>(ka[kb], qf[ks], s[kb]);
    }
  };
  // probs(s, m) = exp2(s * c - m) (one fma per score, inside the exponent's
  // operand) packed as O^T's B operands; returns the lane's partial row sum.
  // The raw scores stay in s: the slow path reads them again.
  bf16x8 pb[2 * kStepBlocks];
  auto probs = [&](const f32x16 (&s)[kStepBlocks], float m) {
    float ps = 0.f;
#pragma unroll
    for (int kb = 0; kb < kStepBlocks; ++kb)
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        i32x4 wv;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float e0 = exp2f_(__builtin_fmaf(s[kb][8 * u + 2 * q], c, -m));
          const float e1 = exp2f_(__builtin_fmaf(s[kb][8 * u + 2 * q + 1], c, -m));
          wv[q] = (int)cvt2<E>(e0, e1);
          ps += e0 + e1;
        }
        pb[2 * kb + u] = __builtin_bit_cast(bf16x8, wv);
      }
    return ps;
  };
  // the interleave of a fused region: K reads, MFMAs and the VALU work of
  // probs (32 fma + 32 exp2 + 16 cvt + 32 adds per step)
  auto interleave = [&]() {
    constexpr int kValuPer = 112 / (KS * kStepBlocks);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      __builtin_amdgcn_sched_group_barrier(kSgDsRead, kStepBlocks, 0);
      __builtin_amdgcn_sched_group_barrier(kSgValu, kValuPer, 0);
#pragma unroll
      for (int kb = 0; kb < kStepBlocks; ++kb) {
        __builtin_amdgcn_sched_group_barrier(kSgMfma, 1, 0);
        if (kb + 1 < kStepBlocks) __builtin_amdgcn_sched_group_barrier(kSgValu, kValuPer, 0);
      }
    }
  };

  // F(j), step j of parity B: the softmax of step j with the scores of step
  // j + 1 (past the group's steps: nothing)
  // O^T += V^T P^T of the step whose V is in tV; operand t = (16-key slice
  // t / DB, output block t % DB), read one ahead. The wave issues at raised
  // priority meanwhile, so the SIMD's other wave, usually in its softmax,
  // yields it the issue slots (about 1 % on the step)
  auto pv = [&](const bf16_t *tV) __attribute__((always_inline)) {
    __builtin_amdgcn_s_setprio(1);
    bf16x8 vcur = tro.operand(tV, 0, 0);
#pragma unroll
    for (int t = 0; t < 2 * kStepBlocks * DB; ++t) {
      bf16x8 vnext;
      if (t + 1 < 2 * kStepBlocks * DB) vnext = tro.operand(tV, ((t + 1) / DB) * 16, (t + 1) % DB);
      __builtin_amdgcn_sched_barrier(0);
      oacc[t % DB] = mfma32<E>(vcur, pb[t / DB], oacc[t % DB]);
      __builtin_amdgcn_sched_barrier(0);
      if (t + 1 < 2 * kStepBlocks * DB) vcur = vnext;
    }
    __builtin_amdgcn_s_setprio(0);
  };
  // (WP: followed by the O^T update of step j, in the same branch; FZ: with
  // the scores of step j + 1, else the softmax alone)
  auto fphase = [&](auto bsel, auto wp_sel, auto fz_sel, int j) __attribute__((always_inline)) {
    constexpr int B = decltype(bsel)::value;
    constexpr bool WP = decltype(wp_sel)::value;
    constexpr bool FZ = decltype(fz_sel)::value;
    const bf16_t *tKn = B ? sK0 : sK1;   // K of step j + 1
    const int *tW = (B ? sW1 : sW0) + grp * kStepKeys;
    f32x16 (&s)[kStepBlocks] = sacc[B];
    f32x16 (&sn)[kStepBlocks] = sacc[1 - B];
    const int kbase = j < nstep ? step_base(j) : a.L;
    const bool act = kbase < a.L;
    const bool act_n = FZ && j + 1 < nstep && step_base(j + 1) < a.L;
    const bool partial = tile_of(j) < npart;
    if (act) {
      if (partial) {
        // a real branch: if-converted, full tiles would pay for the masking
        asm volatile("");
        if (kbase + kStepKeys - 1 > diag) {
          const int lim = qlim - kbase - 4 * hi;   // key offset (without 4 hi) must be <= lim
#pragma unroll
          for (int kb = 0; kb < kStepBlocks; ++kb)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const i32x4 w4 = *reinterpret_cast<const i32x4 *>(&tW[kb * 32 + 8 * i + 4 * hi]);
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                const bool ok = (w4[e] >= qv) & (kb * 32 + 8 * i + e <= lim);
                s[kb][4 * i + e] = ok ? s[kb][4 * i + e] : kNegInfF;
              }
            }
        } else {
#pragma unroll
          for (int kb = 0; kb < kStepBlocks; ++kb)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const i32x4 w4 = *reinterpret_cast<const i32x4 *>(&tW[kb * 32 + 8 * i + 4 * hi]);
#pragma unroll
              for (int e = 0; e < 4; ++e) s[kb][4 * i + e] = w4[e] >= qv ? s[kb][4 * i + e] : kNegInfF;
            }
        }
      }
      const float m_eff = m_run == kNegInfF ? 0.f : m_run;
      float ps;
      if (act_n) {
        // one region: step j + 1's MFMAs interleaved with step j's softmax.
        // The offset passes through an empty asm so that this region's fmas
        // differ from the other branch's and stay here instead of being
        // hoisted above the branch, out of reach of the interleave.
        float mf = m_eff;
        asm volatile("" : "+v"(mf));
        scores_fused(tKn, sn);
        ps = probs(s, mf);
        interleave();
      } else {
        ps = probs(s, m_eff);
      }
      // slow path: no offset yet, or a partial row sum past the bound
      if (__builtin_amdgcn_ballot_w64(!(ps <= kPBound<E>) | (m_run == kNegInfF))) {
        float mx = kNegInfF;
#pragma unroll
        for (int kb = 0; kb < kStepBlocks; ++kb)
#pragma unroll
          for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[kb][r]);
        mx = fmaxf(mx, xor32(mx)) * c;   // the row's max of s * c (c > 0)
        const float m_new = fmaxf(m_run, mx);
        if (m_new > m_run) {
          const float alpha = exp2f_(m_run - m_new);   // 0 when m_run = -inf
          l_run *= alpha;
#pragma unroll
          for (int db = 0; db < DB; ++db)
#pragma unroll
            for (int r = 0; r < 16; ++r) oacc[db][r] *= alpha;
          m_run = m_new;
        }
        ps = probs(s, m_run == kNegInfF ? 0.f : m_run);
      }
      l_run += ps;
      if constexpr (WP) pv(B ? sV1 : sV0);
    } else if (act_n) {
      scores(tKn, sn);
    }
  };
  // step j (parity B): loads, softmax and O^T update, one barrier
  auto run_step = [&](auto bsel, int j) {
    constexpr int B = decltype(bsel)::value;
    if (j + 1 < nstep) load_w(j + 1);
    if (j + 2 < nstep) load_k(j + 2, B ? sK1 : sK0);
    if (j + 1 < nstep) load_v(j + 1, B ? sV0 : sV1);
    fphase(bsel, std::true_type{}, std::true_type{}, j);
    if (j + 1 < nstep) {
      __builtin_amdgcn_s_waitcnt(0);   // this thread's direct loads have landed
      store_w(B ? sW0 : sW1);
    }
    __syncthreads();
  };

  // prologue: K and V of step 0, K of step 1; the scores of step 0
  if (nstep > 0) {
    load_w(0);
    // (in the pair form waves w and w + 4 stage the same quarter of a tile:
    // the first block alone loads)
    if (MODE != kFwdPair || wave < 4) {
      load_k(0, sK0);
      load_v(0, sV0);
      if (nstep > 1) load_k(1, sK1);
    }
    __builtin_amdgcn_s_waitcnt(0);
    store_w(sW0);
    if (MODE == kFwdPair && nstep > 1) {
      // the pair form loads the codes of step j + 2 in V(j): step 1's here
      load_w(1);
      __builtin_amdgcn_s_waitcnt(0);
      store_w(sW1);
    }
  }
  __syncthreads();
  if (nstep > 0) scores(sK0, sacc[0]);   // step 0 always has keys
  __syncthreads();   // every wave is done with sK0 before step 0 loads into it
  if constexpr (MODE == kFwdPair) {
    // Intervals of one barrier each. A step is a softmax interval V(j)
    // (masking, probabilities, row sums: VALU work only) and a product
    // interval M(j) (the O^T update of step j and the scores of step j + 1:
    // MFMAs and their operand reads only). The first row block (waves 0-3)
    // runs V(j) in interval 2j and M(j) in 2j + 1, the second (waves 4-7) one
    // interval later, after a leading idle interval (the first block closes
    // with a trailing one), so each SIMD holds one wave in V and one in M and
    // the matrix core works under the other wave's softmax. Both blocks run
    // this one loop body.
    // Loads: the second block issues K of step j + 2 (into K(j)'s buffer, read
    // last in its own M(j - 1), interval 2j) with the codes of step j + 2 at
    // the start of its V(j), interval 2j + 1, waits for both at the end of
    // its M(j), interval 2j + 2, and then stores the codes into step j's
    // buffer (read last in interval 2j + 1); K is first read in interval
    // 2j + 3, the codes in 2j + 4. The first block issues V of step j + 1
    // (into V(j - 1)'s buffer, read last in the second block's M(j - 1),
    // interval 2j) at the start of its M(j), interval 2j + 1, under its
    // MFMAs, and waits for it at the end of its V(j + 1), interval 2j + 2; it
    // is first read in interval 2j + 3. The prologue stages the codes of
    // steps 0 and 1. Each block keeps a load's issue and its store or wait
    // inside one loop body: a value carried across the loop's back edge was
    // copied between registers right after the tile loads, and the copy
    // waited for them. The tile-list positions are read before the loads are
    // issued (a list refill waits for every load in flight).
    const bool late = wave >= 4;
    const int ltid = tid - 256;   // thread of the second block
    auto step2 = [&](auto bsel, int j) __attribute__((always_inline)) {
      constexpr int B = decltype(bsel)::value;
      const int sb0 = j < nstep ? step_base(j) : a.L;
      const int sb1 = j + 1 < nstep ? step_base(j + 1) : a.L;
      const int sb2 = j + 2 < nstep ? step_base(j + 2) : a.L;
      // V(j). The second block loads the codes and the K tile of step j + 2
      // (the codes first: the compiler waits for every load in flight before
      // it writes their register), stored or waited for at the end of its
      // M(j); the first block's V load of its M(j - 1) (V of step j) lands by
      // the end of it.
      if (late && j + 2 < nstep) {
        if (ltid < kStepKeys) wkey.load(a.code, sb2 + ltid, a.P, a.L);
        load_tile(sb2, B ? sK1 : sK0, kp, a.k_ss, dmaK);
      }
      fphase(bsel, std::false_type{}, std::false_type{}, j);
      if (!late) __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
      // M(j): the first block issues V of step j + 1
      if (!late && j + 1 < nstep) load_tile(sb1, B ? sV0 : sV1, vp, a.v_ss, dmaV);
      if (sb0 < a.L) pv(B ? sV1 : sV0);                      // O^T += V^T P^T of step j
      if (sb1 < a.L) scores(B ? sK0 : sK1, sacc[1 - B]);     // S^T of step j + 1
      if (late && j + 2 < nstep) {
        __builtin_amdgcn_s_waitcnt(0);   // K and the codes of step j + 2 (codes into step j's buffer)
        if (ltid < kStepKeys)
          *reinterpret_cast<int *>(const_cast<char *>(lds_at(B ? sW1 : sW0, opaque_u32(ltid * 4u)))) = wkey.w();
      }
      __syncthreads();
    };
    if (late) __syncthreads();
    for (int j = 0; j < nloop; j += 2) {
      step2(std::integral_constant<int, 0>{}, j);
      if (j + 1 < nloop) step2(std::integral_constant<int, 1>{}, j + 1);
    }
    if (!late) __syncthreads();
  } else {
    for (int j = 0; j < nloop; j += 2) {
      run_step(std::integral_constant<int, 0>{}, j);
      if (j + 1 < nloop) run_step(std::integral_constant<int, 1>{}, j + 1);
    }
  }

  if constexpr (NG == 2) {
    // group 1 hands its (O^T, offset, row sum) to group 0 through LDS (the
    // tile buffers are free after the last barrier); group 0 rescales both
    // to the larger offset and adds them, in a fixed order
    float *xo = reinterpret_cast<float *>(wave < 2 ? sK0 : sV0) + (wave & 1) * (DB * 16 * 64);
    float *xm = reinterpret_cast<float *>(sK1) + wave * 128;
    if (grp == 1) {
#pragma unroll
      for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) xo[(db * 16 + r) * 64 + lane] = oacc[db][r];
      xm[lane] = m_run;
      xm[64 + lane] = l_run;
    }
    __syncthreads();
    if (grp == 1) return;
    const float m1 = xm[lane], l1 = xm[64 + lane];
    const float mm = fmaxf(m_run, m1);
    const bool none = mm == kNegInfF;   // neither group saw an unmasked key
    const float a0 = none ? 0.f : exp2f_(m_run - mm), a1 = none ? 0.f : exp2f_(m1 - mm);
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int r = 0; r < 16; ++r) oacc[db][r] = oacc[db][r] * a0 + xo[(db * 16 + r) * 64 + lane] * a1;
    l_run = l_run * a0 + l1 * a1;
    m_run = mm;
  }

  // ---- epilogue: normalise, write O [S, Hq, D] and the natural-log LSE -------
  const float lt = l_run + xor32(l_run);
  if (row < a.S) {
    const float inv = lt > 0.f ? 1.f / lt : 0.f;
    if (hi == 0)
      a.lse[(int64_t)h * a.S + row] = lt > 0.f ? (m_run + __log2f(lt)) * kLn2 : kNegInfF;
    T *orow = reinterpret_cast<T *>(const_cast<void *>(a.o)) + h * a.o_sh + (int64_t)row * a.o_ss;
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const f32x16 &cc = oacc[db];
        store4(orow + db * 32 + 8 * i + 4 * hi, cc[4 * i] * inv, cc[4 * i + 1] * inv, cc[4 * i + 2] * inv,
               cc[4 * i + 3] * inv);
      }
  }
}

// explicit instantiations: clang otherwise drops some host launch stubs of
// this template (the bf16 ones), leaving undefined symbols
#define MGA_FWD_INST(HD, T)                                                     \
  template __global__ void attn_fwd_kernel<HD, T, kFwd4>(AttnArgs, int, int);    \
  template __global__ void attn_fwd_kernel<HD, T, kFwdPair>(AttnArgs, int, int); \
  template __global__ void attn_fwd_kernel<HD, T, kFwdSplit>(AttnArgs, int, int);
MGA_FWD_INST(128, bf16_t)
MGA_FWD_INST(64, bf16_t)
MGA_FWD_INST(128, f16_t)
MGA_FWD_INST(64, f16_t)
#undef MGA_FWD_INST

// Items per XCD that the first launch runs (the rest go to the split launch):
// each XCD takes a contiguous 1/8 of the items on its m workgroup slots. When
// the last round would fill at most half of them -- a half-empty round takes
// as long as a full one here, a lone workgroup on a CU running no faster --
// that round's items run split (one 8-wave workgroup per row block, each in
// about half the time); when all items fill at most half a round, all of them
// do. Items of fewer than 16 tiles are not split.
int fwd_split_point(int items, int L, int m) {
  const int nmax = (items + 7) / 8;
  if (m < 1) m = 1;
  if (L < 16 * kBlock) return nmax;
  if (nmax <= m / 2) return 0;
  const int r = nmax % m;
  return (nmax > m && r > 0 && r <= m / 2) ? nmax - r : nmax;
}

template <int HD, typename T>
static void fwd_launch(const AttnArgs &a, hipStream_t st) {
  const int G = a.Hq / a.Hkv;
  const int HPW = heads_per_wg(G);
  const int U = units_per_item(HPW);
  const int QU = U * 32 * (4 / HPW);
  const int nqb = (a.S + QU - 1) / QU;
  const int items = a.Hkv * (G / HPW) * nqb;
  const int nmax = (items + 7) / 8;
  const int cx = device_cu_count() / 8;   // CUs per XCD
  const int k1 = fwd_split_point(items, a.L, U == 2 ? cx : 2 * cx);
  if (k1 > 0) {
    if (U == 2) hipLaunchKernelGGL((attn_fwd_kernel<HD, T, kFwdPair>), dim3(8 * k1), dim3(512), 0, st, a, 0, k1);
    else hipLaunchKernelGGL((attn_fwd_kernel<HD, T, kFwd4>), dim3(8 * k1), dim3(256), 0, st, a, 0, k1);
  }
  if (k1 < nmax)
    hipLaunchKernelGGL((attn_fwd_kernel<HD, T, kFwdSplit>), dim3(8 * U * (nmax - k1)), dim3(512), 0, st, a, k1,
                       nmax - k1);
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
