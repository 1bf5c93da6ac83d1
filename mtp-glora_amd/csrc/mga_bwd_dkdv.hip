// MTP block-masked GQA attention backward, dK/dV pass, for gfx950.
//
// Work item = (64-key tile of the keys that receive gradient, kv head g): one
// workgroup of 8 waves, 2 per SIMD. The G query heads of g and the q-major
// block-mask list of the key tile give a list of (query tile, head) pairs;
// the two 4-wave groups of the workgroup take alternate pairs, 32 query rows
// per step. Within a group each 32-key half of the tile belongs to a pair of
// waves that split the four products between them:
//   wave A holds K in registers:  S = Q K^T (accumulator starting at
//       -lse / scale, so P = exp2(scale_log2 * S)), 0 where masked,
//       dV^T += dO^T P                       (A operand dO^T by transpose read)
//   wave B holds V in registers:  dP = dO V^T (starting at -delta),
//       dS = P (dP - delta) from A's fp32 P, rounded once to the operand type,
//       dK^T += Q^T dS                       (A operand Q^T by transpose read)
// B runs its dS / dK part one step behind A, so A's P crosses LDS (as fp32)
// under the one barrier per step. The B waves issue every load of their group:
// the Q tile two steps ahead, the dO tile and the row data one step ahead (dO
// is first read halfway through A's step). Loads go global -> LDS through
// buffer resources whose range ends at the chunk's last row: rows past S, and
// every row of a step past a group's list, arrive as zeros, so they add
// exactly nothing to dK / dV and need no masking. The loads are inline asm
// outside the compiler's wait counting; each B wave waits for exactly its
// loads of the next step (vmcnt) and the per-step barrier carries no memory
// fence. At the end group 1 hands its accumulators to group 0 through LDS and
// group 0 adds them in a fixed order: dK and dV summed over the G heads
// without partial sums in global memory or atomics, bit-for-bit repeatable.
// Row data per (query head, row) is written by the dQ pass: -lse / scale, -delta
// and the row's mask threshold (three planes of the delta workspace).
// Semantics: [torch]_higher_order_ops/flex_attention.py:826-990 (dK/dV summed
// over the query heads of a kv head, :957-966), restricted to keys >=
// grad_start; dS formed from the fp32 P and rounded only before the dK
// product, as [torch]_inductor/kernel/flex/templates/flex_backwards.py.jinja:570-618.
#include <type_traits>

#include "mga_common.hpp"
#include "mga_internal.hpp"

namespace mga {

namespace {

constexpr int kRows = 32;         // query rows per step
constexpr int kKeys = 64;         // keys per workgroup
constexpr int kThreads = 512;
constexpr uint32_t kOob = 0xfffffff0u;   // a buffer offset past every range: the load returns zeros

// 16 per-row values of a 32-row block in accumulator order: register r holds
// row 8 (r / 4) + 4 hi + r % 4, four consecutive rows per 16-byte read; ofs is
// the lane's byte offset of row 4 hi.
template <typename V>
__device__ __forceinline__ V rows16(const void *t, uint32_t ofs) {
  V v;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    typedef __attribute__((__vector_size__(4 * sizeof(v[0])))) __typeof__(v[0] + 0) q4;
    const q4 x = *reinterpret_cast<const q4 *>(lds_at(t, ofs + 32 * i));
    v[4 * i] = x[0]; v[4 * i + 1] = x[1]; v[4 * i + 2] = x[2]; v[4 * i + 3] = x[3];
  }
  return v;
}
typedef __attribute__((__vector_size__(16 * sizeof(uint32_t)))) uint32_t u32x16;

// The group's walk over its (query tile, head) pairs gr, gr + 2, ...: four
// 32-row steps per pair, the step within the pair being the index of the
// four-fold unrolled step loop. Advanced once per pair (no division).
struct PairWalk {
  int k, hh, it;
  __device__ __forceinline__ void init(int gr, int G) {
    k = 0;
    it = gr / G;
    hh = gr - it * G;
  }
  __device__ __forceinline__ void next(int G) {
    ++k;
    hh += 2;
    if (hh >= G) { hh -= G; ++it; }
    if (hh >= G) { hh -= G; ++it; }
  }
};

// One pair: query rows row0 .. row0 + 127 of head h (row0 = S: past the
// group's list); partial: the query tile's block-mask entry is partial.
struct PairInfo {
  int row0;
  int h;
  int partial;
};

}  // namespace

template <int HD, typename T>
__global__ __launch_bounds__(kThreads, 1) void attn_bwd_dkdv_kernel(AttnArgs a, int kh0, int nkh) {
  typedef typename MfmaElem<T>::type E;
  constexpr int KS = HD / 16;
  constexpr int DB = HD / 32;
  constexpr int TILE = kRows * HD;                 // one group's tile (elements)
  constexpr int kGranRow = HD / 8;
  constexpr int kRowsPerInst = 64 / kGranRow;      // tile rows per 1 KB load
  constexpr int kInst = kRows / kRowsPerInst / 2;  // loads per tile per B wave
  // Staging ([group][tile]): Q ring of four step slots (B's dK of step j - 1
  // reads Q(j - 1) while Q(j + 2) loads), dO and row data rings of two. Named
  // objects, the step loop unrolled by four: every buffer base is a constant.
  __shared__ __attribute__((aligned(16))) bf16_t sQ0[2 * TILE], sQ1[2 * TILE], sQ2[2 * TILE], sQ3[2 * TILE];
  __shared__ __attribute__((aligned(16))) bf16_t sD0[2 * TILE], sD1[2 * TILE];
  // row data ([group][-lse / scale x 32, -delta x 32, threshold x 32, unused x 32])
  __shared__ __attribute__((aligned(16))) float sR0[2 * 128], sR1[2 * 128];
  // A's fp32 probabilities for B ([wave pair][4 register quads][64 lanes][4])
  __shared__ __attribute__((aligned(16))) float sP0[4 * 1024], sP1[4 * 1024];

  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const int l32 = lane & 31, hi = lane >> 5;
  const int gr = wave >> 2;                 // group
  const int w4 = wave & 3;                  // wave within the group
  const int half = w4 >> 1;                 // 32-key half of the tile
  // 0: A (S, P, dV), 1: B (dP, dS, dK). Wave w and wave w + 4 share a SIMD
  // (a workgroup's waves are placed round-robin), so the groups swap the
  // roles: every SIMD holds one A and one B.
  const int role = (w4 & 1) ^ gr;
  const int pair = gr * 2 + half;
  const int G = a.Hq / a.Hkv;

  // item: kv head major (its key tiles share an XCD), key tiles in order (the
  // first ones have the longest query lists)
  const int li = xcd_swizzle(blockIdx.x, a.Hkv * nkh);
  const int g = li / nkh;
  const int kh = kh0 + li % nkh;
  const int kt = (kh * kKeys) / kBlock;     // block-mask key tile

  const int key = kh * kKeys + half * 32 + l32;
  const int key_last = kh * kKeys + half * 32 + 31;   // the wave's last key
  const int kr = min(key, a.L - 1);
  // the key's mask threshold: a query row with threshold s sees the key iff
  // s >= kwp (unsigned). Regular key 1, mask key of code c 2^31 - 1 - c, pad
  // key (or past L) above every row's s.
  uint32_t kwp;
  {
    const int c = key < a.P ? kCodeX : (key < a.L ? a.code[key - a.P] : kCodePad);
    kwp = c == kCodeX ? 1u : (c == kCodePad ? 0xffffffffu : 0x7fffffffu - (uint32_t)c);
  }

  // the wave's key operands: K for A, V for B (8 dims of key l32 per k-step)
  bf16x8 kv[KS];
  {
    const T *src = role == 0 ? reinterpret_cast<const T *>(a.k) + g * a.k_sh + (int64_t)kr * a.k_ss
                             : reinterpret_cast<const T *>(a.v) + g * a.v_sh + (int64_t)kr * a.v_ss;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) kv[ks] = load8(src + ks * 16 + hi * 8);
  }

  TileList tiles = tile_list(a.q_num, a.q_idx, a.fq_num, a.fq_idx, kt, a.nQ);
  const int npart = tiles.npart;
  const int npairs = G * tiles.ntot;                   // (query tile, head) pairs
  const int mine = (npairs - gr + 1) / 2;              // pairs gr, gr + 2, ...
  const int nsteps_other = 4 * ((npairs - (1 - gr) + 1) / 2);
  const int niter = (max(4 * mine, nsteps_other) + 1 + 3) / 4 * 4;   // + 1: B's last dK step

  auto pinfo = [&](const PairWalk &w) -> PairInfo {
    PairInfo p;
    p.row0 = w.k < mine ? tiles.at(w.it) * kBlock : a.S;
    p.h = g * G + w.hh;
    p.partial = w.it < npart;
    return p;
  };

  // LDS byte offsets (the group's block folded in, so every buffer base is an
  // immediate): Q / dO operand of k-step ks (row l32, granule (2 ks + hi) ^
  // swz(l32)), the transposed operands, this lane's row data and P words
  const uint32_t gofs = (uint32_t)(gr * TILE * 2);
  const uint32_t qrow = (uint32_t)(l32 * HD + (((uint32_t)hi ^ swz<HD>(l32)) << 3)) * 2u;
  uint32_t qk[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) qk[ks] = opaque_u32(gofs + (qrow ^ (uint32_t)(ks << 5)));
  TrOffsets<HD> tro;
  tro.init(lane);
#pragma unroll
  for (int sx = 0; sx < 2; ++sx)
#pragma unroll
    for (int mb = 0; mb < DB; ++mb) tro.off[sx][mb] = opaque_u32(tro.off[sx][mb] + gofs);
  const uint32_t rofs = opaque_u32((uint32_t)(gr * 128 + 4 * hi) * 4u);
  const uint32_t pofs = opaque_u32((uint32_t)(pair * 4096 + lane * 16));
  const float c = a.scale_log2;

  // Inactive or stale buffer contents must be finite (0 * NaN would not vanish):
  // every buffer starts at zero.
  {
    const i32x4 z = {0, 0, 0, 0};
    for (int i = tid; i < 2 * TILE / 8; i += kThreads) {
      reinterpret_cast<i32x4 *>(sQ0)[i] = z; reinterpret_cast<i32x4 *>(sQ1)[i] = z;
      reinterpret_cast<i32x4 *>(sQ2)[i] = z; reinterpret_cast<i32x4 *>(sQ3)[i] = z;
      reinterpret_cast<i32x4 *>(sD0)[i] = z; reinterpret_cast<i32x4 *>(sD1)[i] = z;
    }
    for (int i = tid; i < 4 * 1024 / 4; i += kThreads) {
      reinterpret_cast<i32x4 *>(sP0)[i] = z; reinterpret_cast<i32x4 *>(sP1)[i] = z;
    }
    if (tid < 2 * 128 / 4) { reinterpret_cast<i32x4 *>(sR0)[tid] = z; reinterpret_cast<i32x4 *>(sR1)[tid] = z; }
  }
  // the key operands landed: a wait the compiler sees, so that it knows no
  // tracked load is in flight in the loops below (their loads are inline asm)
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  auto qslot = [&](int i) -> bf16_t * { return i == 0 ? sQ0 : (i == 1 ? sQ1 : (i == 2 ? sQ2 : sQ3)); };
  auto dslot = [&](int i) -> bf16_t * { return i == 0 ? sD0 : sD1; };
  auto rslot = [&](int i) -> float * { return i == 0 ? sR0 : sR1; };
  auto pslot = [&](int i) -> float * { return i == 0 ? sP0 : sP1; };

  // ---- load set-up of the B waves, and their loads of step 0 ----
  // load lane offsets: tile load i of this wave covers rows
  // (half * kInst + i) * kRowsPerInst + lane / kGranRow; the lane fetches
  // the granule the swizzle places at its LDS slot
  uint32_t voQ[kInst], voD[kInst];
  {
    const int p = lane % kGranRow, lr = lane / kGranRow;
#pragma unroll
    for (int i = 0; i < kInst; ++i) {
      const int r = (half * kInst + i) * kRowsPerInst + lr;
      const uint32_t gran = (uint32_t)((p ^ swz<HD>(r)) << 4);
      voQ[i] = opaque_u32((uint32_t)(r * a.q_ss * 2) + gran);
      voD[i] = opaque_u32((uint32_t)(r * a.do_ss * 2) + gran);
    }
  }
  // row data: B of key half 0 loads -lse / scale (lanes 0-31) and -delta
  // (lanes 32-63), B of half 1 the thresholds (lanes 0-31); plane byte
  // offset of the lane, or none
  const int64_t plane = (int64_t)a.Hq * a.S;
  const bool rlane = half == 0 || hi == 0;
  const uint32_t rplane = (uint32_t)((half == 0 ? hi : 2) * plane * 4);
  const i32x4 rws = buf_rsrc(a.delta, (uint32_t)(3 * plane * 4));
  const uint32_t rdst = (uint32_t)(gr * 128 + half * 64) * 4u;

  // per pair: the Q and dO bases of its first row and its row-data index
  struct PairBase {
    const char *qb, *db;
    int rb, row0;
  };
  auto pbase = [&](const PairInfo &p) -> PairBase {
    PairBase b;
    b.qb = reinterpret_cast<const char *>(a.q) + (p.h * a.q_sh + (int64_t)p.row0 * a.q_ss) * 2;
    b.db = reinterpret_cast<const char *>(a.dout) + (p.h * a.do_sh + (int64_t)p.row0 * a.do_ss) * 2;
    b.rb = p.h * a.S + p.row0;
    b.row0 = p.row0;
    return b;
  };
  const int64_t qstep = (int64_t)kRows * a.q_ss * 2, dstep = (int64_t)kRows * a.do_ss * 2;
  // step sub of pair b: rows row0 + 32 sub ..; rows at or past S read as zeros
  auto issue_rows = [&](const PairBase &b, int sub, float *dst) {
    const int rr = b.row0 + sub * kRows + l32;
    const uint32_t vo = rplane + (uint32_t)((b.rb + sub * kRows + l32) * 4);
    bdma4(rws, (rlane && rr < a.S) ? vo : kOob, reinterpret_cast<const char *>(dst) + rdst);
  };
  auto issue_tile = [&](const char *base, int64_t ss, const uint32_t *vo, int q0, bf16_t *dst) {
    const uint32_t nb = (uint32_t)(min(max(a.S - q0, 0), kRows) * ss * 2);
    const i32x4 r = buf_rsrc(base, nb);
    bf16_t *d = dst + gr * TILE + half * kInst * 512;
#pragma unroll
    for (int i = 0; i < kInst; ++i) bdma16(r, vo[i], d + i * 512);
  };

  PairWalk wkb;   // B: the pair after qp
  PairBase qp, dp_;   // B: pairs of the Q loads (step j + 2) and of the dO and row-data loads (step j + 1)
  if (role == 1) {
    wkb.init(gr, G);
    qp = pbase(pinfo(wkb));
    wkb.next(G);
    dp_ = qp;
    // step 0's dO, rows and Q, then Q(1); wait for all but Q(1)
    issue_tile(dp_.db, a.do_ss, voD, dp_.row0, sD0);
    issue_rows(dp_, 0, sR0);
    issue_tile(qp.qb, a.q_ss, voQ, qp.row0, sQ0);
    issue_tile(qp.qb + qstep, a.q_ss, voQ, qp.row0 + kRows, sQ1);
    asm volatile("s_waitcnt vmcnt(%0)" : : "n"(kInst) : "memory");
  }
  // step 0's tiles and row data are in LDS for every wave (Q(1) may still be
  // in flight: the barrier carries no fence)
  lds_barrier();


  f32x16 acc[DB];                     // A: dV^T, B: dK^T (dims x keys)
#pragma unroll
  for (int db = 0; db < DB; ++db) acc[db] = zero16();

  if (role == 0) {
    // ------------------------------------------------------------------ A
    PairWalk wk;
    wk.init(gr, G);
    PairInfo cur;
    auto stepA = [&](auto jsel) {
      constexpr int J = decltype(jsel)::value;
      if constexpr (J == 0) {
        cur = pinfo(wk);
        wk.next(G);
      }
      const int q0 = min(cur.row0 + J * kRows, a.S);
      const bf16_t *tQ = qslot(J % 4);
      const bf16_t *tD = dslot(J % 2);
      const float *tR = rslot(J % 2);
      // S - lse / scale = Q K^T + (-lse / scale)
      f32x16 sc = rows16<f32x16>(tR, rofs);
      bf16x8 op = lds_read8(reinterpret_cast<const bf16_t *>(lds_at(tQ, qk[0])));
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        bf16x8 nx;
        if (ks + 1 < KS) nx = lds_read8(reinterpret_cast<const bf16_t *>(lds_at(tQ, qk[ks + 1])));
        sc = mfma32<E>(op, kv[ks], sc);
        if (ks + 1 < KS) op = nx;
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) sc[r] = __builtin_amdgcn_exp2f(sc[r] * c);
      if (cur.partial) {
        // real branches (if-converted, full tiles would pay for the masking),
        // each updating P in place
        asm volatile("");
        const u32x16 th = rows16<u32x16>(tR + 64, rofs);
#pragma unroll
        for (int r = 0; r < 16; ++r) sc[r] = th[r] >= kwp ? sc[r] : 0.f;
        if (q0 + a.P < key_last) {   // some row precedes one of the wave's keys: causal bound too
          asm volatile("");
          const int thr = key - q0 - a.P - 4 * hi;   // causal: row offset (without 4 hi) >= thr
#pragma unroll
          for (int r = 0; r < 16; ++r) sc[r] = 8 * (r / 4) + r % 4 >= thr ? sc[r] : 0.f;
        }
      }
      // fp32 P for B's dS
      {
        char *pp = reinterpret_cast<char *>(pslot(J % 2));
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const f32x4 v = {sc[4 * q], sc[4 * q + 1], sc[4 * q + 2], sc[4 * q + 3]};
          *reinterpret_cast<f32x4 *>(pp + pofs + q * 1024) = v;
        }
      }
      // dV^T += dO^T P (16-row slice u, 32-dim block db); the transposed
      // operands are read three MFMAs ahead
      i32x4 pw[2];
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int t = 0; t < 4; ++t) pw[u][t] = (int)cvt2<E>(sc[8 * u + 2 * t], sc[8 * u + 2 * t + 1]);
      {
        constexpr int NT = 2 * DB, AH = 3;
        bf16x8 ow[AH];
#pragma unroll
        for (int t = 0; t < AH; ++t) ow[t] = tro.operand(tD, (t / DB) * 16, t % DB);
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          bf16x8 nx;
          if (t + AH < NT) nx = tro.operand(tD, ((t + AH) / DB) * 16, (t + AH) % DB);
          acc[t % DB] = mfma32<E>(ow[t % AH], __builtin_bit_cast(bf16x8, pw[t / DB]), acc[t % DB]);
          if (t + AH < NT) ow[t % AH] = nx;
        }
      }
      lds_barrier();
    };
    for (int j = 0; j < niter; j += 4) {
      stepA(std::integral_constant<int, 0>{});
      stepA(std::integral_constant<int, 1>{});
      stepA(std::integral_constant<int, 2>{});
      stepA(std::integral_constant<int, 3>{});
    }
  } else {
    // ------------------------------------------------------------------ B
    // B: dP - delta of the current and the previous step, alternating by step parity
    f32x16 dp2[2] = {zero16(), zero16()};
    auto stepB = [&](auto jsel) {
      constexpr int J = decltype(jsel)::value;
      // loads: dO and row data of step j + 1 first (waited for at this step's
      // end), then Q of step j + 2 (still in flight across the barrier); step
      // j + 2 starts a pair at J = 2, step j + 1 at J = 3
      if constexpr (J == 2) {
        qp = pbase(pinfo(wkb));
        wkb.next(G);
      }
      if constexpr (J == 3) dp_ = qp;
      constexpr int s1 = (J + 1) % 4, s2 = (J + 2) % 4;
      issue_tile(dp_.db + s1 * dstep, a.do_ss, voD, dp_.row0 + s1 * kRows, dslot((J + 1) % 2));
      issue_rows(dp_, s1, rslot((J + 1) % 2));
      issue_tile(qp.qb + s2 * qstep, a.q_ss, voQ, qp.row0 + s2 * kRows, qslot((J + 2) % 4));

      f32x16 &dp = dp2[J % 2];
      const f32x16 &dprev = dp2[(J + 1) % 2];
      // dS of the previous step from A's fp32 P: dK^T += Q^T dS
      {
        const char *pp = reinterpret_cast<const char *>(pslot((J + 1) % 2));
        f32x4 pv[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) pv[q] = *reinterpret_cast<const f32x4 *>(pp + pofs + q * 1024);
        i32x4 dsw[2];
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            const int r = 8 * u + 2 * t;
            dsw[u][t] = (int)cvt2<E>(pv[r / 4][r % 4] * dprev[r], pv[(r + 1) / 4][(r + 1) % 4] * dprev[r + 1]);
          }
        const bf16_t *tQprev = qslot((J + 3) % 4);
        // the dK and dP products at raised issue priority: the SIMD's A wave
        // is then in its exponentials or its dV product (about 1 % on the pass)
        __builtin_amdgcn_s_setprio(1);
        constexpr int NT = 2 * DB, AH = 3;
        bf16x8 ow[AH];
#pragma unroll
        for (int t = 0; t < AH; ++t) ow[t] = tro.operand(tQprev, (t / DB) * 16, t % DB);
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          bf16x8 nx;
          if (t + AH < NT) nx = tro.operand(tQprev, ((t + AH) / DB) * 16, (t + AH) % DB);
          acc[t % DB] = mfma32<E>(ow[t % AH], __builtin_bit_cast(bf16x8, dsw[t / DB]), acc[t % DB]);
          if (t + AH < NT) ow[t % AH] = nx;
        }
      }
      // dP - delta = dO V^T + (-delta)
      {
        const bf16_t *tD = dslot(J % 2);
        dp = rows16<f32x16>(rslot(J % 2) + 32, rofs);
        bf16x8 op = lds_read8(reinterpret_cast<const bf16_t *>(lds_at(tD, qk[0])));
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          bf16x8 nx;
          if (ks + 1 < KS) nx = lds_read8(reinterpret_cast<const bf16_t *>(lds_at(tD, qk[ks + 1])));
          dp = mfma32<E>(op, kv[ks], dp);
          if (ks + 1 < KS) op = nx;
        }
      }
      __builtin_amdgcn_s_setprio(0);
      // this wave's loads of step j + 1 landed: all but Q(j + 2) just issued
      asm volatile("s_waitcnt vmcnt(%0)" : : "n"(kInst) : "memory");
      lds_barrier();
    };
    for (int j = 0; j < niter; j += 4) {
      stepB(std::integral_constant<int, 0>{});
      stepB(std::integral_constant<int, 1>{});
      stepB(std::integral_constant<int, 2>{});
      stepB(std::integral_constant<int, 3>{});
    }
  }
  // the last steps' loads (past the end) land before the buffers take the accumulators
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();

  // ---- group 1 hands its accumulators to group 0 (the Q ring is free after
  // the last barrier): wave (half, role) of group 1 writes Q slot [half][role],
  // 16 KB in quads of registers, lane-interleaved ----
  float *x = reinterpret_cast<float *>(qslot(half * 2 + role));
  if (gr == 1) {
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        f32x4 v = {acc[db][4 * q], acc[db][4 * q + 1], acc[db][4 * q + 2], acc[db][4 * q + 3]};
        *reinterpret_cast<f32x4 *>(x + ((db * 4 + q) * 64 + lane) * 4) = v;
      }
  }
  __syncthreads();
  if (gr == 0) {
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const f32x4 v = *reinterpret_cast<const f32x4 *>(x + ((db * 4 + q) * 64 + lane) * 4);
        acc[db][4 * q] += v[0]; acc[db][4 * q + 1] += v[1]; acc[db][4 * q + 2] += v[2]; acc[db][4 * q + 3] += v[3];
      }
    // lane = key, registers = dims 8 (r / 4) + 4 hi + r % 4 of block db
    if (key >= a.grad_start && key < a.L) {
      const int64_t row = key - a.grad_start;
      const float f = role == 0 ? 1.f : a.scale;
      T *out = role == 0 ? reinterpret_cast<T *>(a.dv) + g * a.dv_sh + row * a.dv_ss
                         : reinterpret_cast<T *>(a.dk) + g * a.dk_sh + row * a.dk_ss;
#pragma unroll
      for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          store4(out + db * 32 + 8 * i + 4 * hi, acc[db][4 * i] * f, acc[db][4 * i + 1] * f,
                 acc[db][4 * i + 2] * f, acc[db][4 * i + 3] * f);
    }
  }
}

// explicit instantiations: clang otherwise drops some host launch stubs of
// this template, leaving undefined symbols
template __global__ void attn_bwd_dkdv_kernel<128, bf16_t>(AttnArgs, int, int);
template __global__ void attn_bwd_dkdv_kernel<64, bf16_t>(AttnArgs, int, int);
template __global__ void attn_bwd_dkdv_kernel<128, f16_t>(AttnArgs, int, int);
template __global__ void attn_bwd_dkdv_kernel<64, f16_t>(AttnArgs, int, int);

template <int HD, typename T>
void dkdv_launch(const AttnArgs &a, hipStream_t st) {
  if (a.grad_start >= a.L) return;
  const int kh0 = a.grad_start / kKeys;
  const int nkh = (a.L - kh0 * kKeys + kKeys - 1) / kKeys;
  hipLaunchKernelGGL((attn_bwd_dkdv_kernel<HD, T>), dim3(a.Hkv * nkh), dim3(kThreads), 0, st, a, kh0, nkh);
}

template <int HD, typename T>
void dq_launch(const AttnArgs &a, hipStream_t st);   // mga_bwd_dq.hip

template <int HD, typename T>
static void bwd_launch(const AttnArgs &a, int passes, hipStream_t st) {
  if (passes & kBwdDq) dq_launch<HD, T>(a, st);
  if (passes & kBwdDkDv) dkdv_launch<HD, T>(a, st);
}

template <int HD>
static void bwd_launch_dt(const AttnArgs &a, int dtype, int passes, hipStream_t st) {
  if (dtype == kDtF16) bwd_launch<HD, f16_t>(a, passes, st);
  else bwd_launch<HD, bf16_t>(a, passes, st);
}

void launch_attn_bwd(const AttnArgs &a, int head_dim, int dtype, int passes, hipStream_t st) {
  if (dtype == kDtF32) launch_attn_bwd_f32(a, head_dim, passes, st);
  else if (head_dim == 128) bwd_launch_dt<128>(a, dtype, passes, st);
  else bwd_launch_dt<64>(a, dtype, passes, st);
}

}  // namespace mga
