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
//       dS = P dP with A's P read back from LDS,
//       dK^T += Q^T dS                       (A operand Q^T by transpose read)
// so each wave keeps one 32 x HD accumulator and one operand set (about 200
// registers) and two waves share a SIMD. B runs its dS / dK part one step
// behind A: A's P crosses LDS under the one barrier per step that also
// rotates the staging buffers. The Q / dO tiles of step j + 2 are loaded
// (global -> LDS) while step j computes, their row data one step ahead: four
// step slots of Q and dO tiles (B's dK of step j - 1 reads Q(j - 1)). The
// two B waves of a group issue all of its loads: A's chain (S, exp, the mask,
// P, dV) is the longer one, and B waits for it at the barrier anyway. Those
// loads stay in flight across the step's end: the direct loads and the row
// loads are inline asm that the compiler does not count, B waits for exactly
// the loads of step j + 1 (vmcnt), and the per-step barrier carries no memory
// fence (__syncthreads' release fence would wait for every direct load in
// flight, since they write LDS). At the end group 1 hands its
// accumulators to group 0 through LDS and group 0 adds them in a fixed order:
// dK and dV summed over the G heads without partial sums in global memory or
// atomics, and bit-for-bit repeatable.
// Semantics: [torch]_higher_order_ops/flex_attention.py:826-990 (dK/dV summed
// over the query heads of a kv head, :957-966), restricted to keys >= grad_start.
#include <type_traits>

#include "mga_common.hpp"
#include "mga_internal.hpp"

namespace mga {

namespace {

constexpr float kNegInfK = -__builtin_huge_valf();
constexpr int kRows = 32;         // query rows per step
constexpr int kKeys = 64;         // keys per workgroup
constexpr int kThreads = 512;
// ordered-compare values of this pass: a pad query (or a row past S) sits
// above every key, a regular key and a regular query one below
constexpr int kVRegular = 0x7ffffffe;
constexpr int kVPadQuery = 0x7fffffff;

// Per-step bookkeeping of one group, carried from the load to the compute.
struct StepInfo {
  int q0;       // first query row (chunk index)
  int h;        // query head
  int flags;    // 1: rows exist (step active), 2: partial tile (masking)
};

// 16 per-row values of a 32-row block in accumulator order: register r holds
// row 8 (r / 4) + 4 hi + r % 4, four consecutive rows per 16-byte read; ofs is
// the lane's byte offset of row 4 hi (plus the group's block).
__device__ __forceinline__ f32x16 rows16(const float *t, uint32_t ofs) {
  f32x16 v;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const f32x4 x = *reinterpret_cast<const f32x4 *>(lds_at(t, ofs + 32 * i));
    v[4 * i] = x[0]; v[4 * i + 1] = x[1]; v[4 * i + 2] = x[2]; v[4 * i + 3] = x[3];
  }
  return v;
}

// Global -> LDS staging of a 32 x HD tile (bf16 or fp16) by the two B waves
// of a group (wl: the loading wave, 0 or 1, wave-uniform): direct loads as
// inline asm (dma16), completion on vmcnt waited for by the caller; rows past
// rmax repeat row rmax. Addresses are a scalar
// row base plus a 32-bit lane offset (the lane's row term for the source's
// stride, precomputed, plus its swizzled granule), as in DmaLane.
template <int HD>
struct GroupTile {
  static constexpr int kGranRow = HD / 8;
  static constexpr int kRowsPerInst = 64 / kGranRow;
  static constexpr int kInst = kRows / kRowsPerInst / 2;   // direct loads per loading wave
  uint32_t gran[kInst];   // byte offset of the lane's granule in its row, per load
  int lr;                 // the lane's row within a load's row block

  __device__ __forceinline__ void init(int wl, int lane) {
    const int p = lane % kGranRow;
    lr = lane / kGranRow;
#pragma unroll
    for (int i = 0; i < kInst; ++i) {
      const int r = (wl * kInst + i) * kRowsPerInst + lr;
      gran[i] = opaque_u32((uint32_t)((p ^ swz<HD>(r)) << 4));
    }
  }
  // byte offset of the lane's row for row stride ss
  __device__ __forceinline__ uint32_t lane_row(int64_t ss) const { return opaque_u32((uint32_t)(lr * ss * 2)); }

  __device__ __forceinline__ void load(bf16_t *tile, const bf16_t *src, int64_t ss, uint32_t lrow, int r0,
                                       int rmax, int wl) const {
    if (r0 + kRows - 1 <= rmax) {
      const bf16_t *base = src + (int64_t)r0 * ss;
#pragma unroll
      for (int i = 0; i < kInst; ++i) {
        const int blk = wl * kInst + i;
        const char *b = reinterpret_cast<const char *>(base + (int64_t)(blk * kRowsPerInst) * ss);
        dma16(b, opaque_u32(lrow) + gran[i], tile + blk * 512);
      }
    } else {   // the chunk's last rows: clamp per lane
#pragma unroll
      for (int i = 0; i < kInst; ++i) {
        const int blk = wl * kInst + i;
        const int row = min(r0 + blk * kRowsPerInst + lr, rmax);
        dma16(reinterpret_cast<const char *>(src + (int64_t)row * ss) + gran[i], tile + blk * 512);
      }
    }
  }
};

}  // namespace

template <int HD, typename T>
__global__ __launch_bounds__(kThreads, 1) void attn_bwd_dkdv_kernel(AttnArgs a, int kh0, int nkh) {
  typedef typename MfmaElem<T>::type E;
  constexpr int KS = HD / 16;
  constexpr int DB = HD / 32;
  constexpr int TILE = kRows * HD;          // one group's tile (elements)
  // staging buffers, each holding both groups' tiles ([group][TILE]); named
  // objects so the compiler sees that the direct loads into one never alias
  // the reads of another (the step loop is unrolled to make every index a
  // constant)
  // ([group][Q tile, dO tile]): one object per step slot, so that the
  // compiler's wait tracking of the direct loads (a few LDS objects) tells
  // every slot apart
  __shared__ __attribute__((aligned(16))) bf16_t sT0[4 * TILE], sT1[4 * TILE], sT2[4 * TILE], sT3[4 * TILE];
  // per row of a step ([group][row]): -lse / scale, -delta, ordered-compare value
  __shared__ __attribute__((aligned(16))) float sL0[2 * kRows], sL1[2 * kRows];
  __shared__ __attribute__((aligned(16))) float sE0[2 * kRows], sE1[2 * kRows];
  __shared__ __attribute__((aligned(16))) int sC0[2 * kRows], sC1[2 * kRows];
  // A's packed probabilities for B ([wave pair][512 dwords])
  __shared__ __attribute__((aligned(16))) uint32_t sP0[4 * 512], sP1[4 * 512];

  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const int l32 = lane & 31, hi = lane >> 5;
  const int gr = wave >> 2;                 // group
  const int w4 = wave & 3;                  // wave within the group
  const int half = w4 >> 1;                 // 32-key half of the tile
  // 0: A (S, P, dV), 1: B (dP, dS, dK). Wave w and wave w + 4 share a SIMD
  // (a workgroup's waves are placed round-robin), so the groups swap the
  // roles: every SIMD holds one VALU-heavy A and one lighter B.
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
  const int kw = min(key_w(a.code, key, a.P, a.L), kVRegular);

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
  const int npairs = G * tiles.ntot;                  // (query tile, head) pairs
  const int mine = (npairs - gr + 1) / 2;              // pairs gr, gr + 2, ...
  const int nsteps = 4 * mine;
  const int nsteps_other = 4 * ((npairs - (1 - gr) + 1) / 2);
  const int niter = (max(nsteps, nsteps_other) + 1 + 3) / 4 * 4;   // + 1: B's last dK step

  auto info_of = [&](int j) -> StepInfo {
    StepInfo s{0, 0, 0};
    if (j < nsteps) {
      const int i = gr + 2 * (j >> 2);
      const int it = i / G;
      s.h = g * G + i % G;
      s.q0 = tiles.at(it) * kBlock + (j & 3) * kRows;
      s.flags = (s.q0 < a.S ? 1 : 0) | (it < npart ? 2 : 0);
    }
    return s;
  };

  // Q / dO operand of k-step ks: row l32, granule (2 ks + hi) ^ swz(l32)
  // LDS byte offsets, the group's block folded in so that every buffer base
  // is an immediate: Q / dO operand of k-step ks (row l32, granule
  // (2 ks + hi) ^ swz(l32)), the transposed operands, this lane's row data and
  // its pair's P words
  const uint32_t gofs = (uint32_t)(gr * 2 * TILE * 2);
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
  const uint32_t rofs = opaque_u32((uint32_t)(gr * kRows + 4 * hi) * 4u);
  const uint32_t pofs = opaque_u32((uint32_t)(pair * 2048 + lane * 16));
  const float c = a.scale_log2;
  const float inv_scale = 1.f / a.scale;

  // tiles: global -> LDS two steps ahead; row data: global -> registers at
  // the start of the step before its own, -> LDS at that step's end
  float rl = 0.f, re = 0.f;
  int rc = kCodePad, rq = 0;
  // the B waves (one per key half) stage the group's tiles and row data: A,
  // whose chain S -> P -> dV is the longer one, issues no global loads
  const int wlu = __builtin_amdgcn_readfirstlane(half);
  GroupTile<HD> gtile;
  gtile.init(wlu, lane);
  const uint32_t lrowQ = gtile.lane_row(a.q_ss), lrowD = gtile.lane_row(a.do_ss);
  // Every B wave issues the same loads on every step, inactive ones included
  // (an inactive step's StepInfo is zero: head 0, rows from 0, always in
  // bounds, never read): with a fixed count in flight the compiler's own wait
  // before the row data's first use is the same vmcnt as the explicit one, so
  // the tiles of step j + 2 stay in flight across the step's end.
  auto load_tiles = [&](const StepInfo &s, bf16_t *dQ, bf16_t *dD) {
    const bf16_t *qp = reinterpret_cast<const bf16_t *>(a.q) + s.h * a.q_sh;
    const bf16_t *dop = reinterpret_cast<const bf16_t *>(a.dout) + s.h * a.do_sh;
    gtile.load(dQ, qp, a.q_ss, lrowQ, s.q0, a.S - 1, wlu);
    gtile.load(dD, dop, a.do_ss, lrowD, s.q0, a.S - 1, wlu);
  };
  // row data: loaded by every lane of both B waves (clamped rows), stored by
  // lanes 0 .. 31 of the B wave of key half 0
  const bool row_lane = role == 1 && half == 0 && lane < kRows;
  // The row loads are inline asm, outside the compiler's wait counting (which
  // would wait for every load in flight, the tiles of step j + 2 included,
  // before the values' first use); rows_wait() below is their wait, and it
  // hands the registers back only after it.
  auto load_rows = [&](const StepInfo &s) {
    rq = (s.flags & 1) ? s.q0 + (lane & 31) : a.S;
    const int rr = min(rq, a.S - 1);
    const float *pl = a.lse + ((int64_t)s.h * a.S + rr);
    const float *pe = a.delta + ((int64_t)s.h * a.S + rr);
    const int32_t *pc = a.code + rr;
    asm volatile("global_load_dword %0, %1, off" : "=v"(rl) : "v"(pl) : "memory");
    asm volatile("global_load_dword %0, %1, off" : "=v"(re) : "v"(pe) : "memory");
    asm volatile("global_load_dword %0, %1, off" : "=v"(rc) : "v"(pc) : "memory");
  };
  auto store_rows = [&](const StepInfo &s, float *dL, float *dE, int *dC) {
    if (row_lane) {
      const bool in = rq < a.S;
      const int code = in ? rc : kCodePad;
      const float lse = in ? rl : kNegInfK;
      const bool none = code == kCodePad || lse == kNegInfK;   // the row sees no key
      dL[lane] = none ? 0.f : -lse * inv_scale;
      dE[lane] = in ? -re : 0.f;
      dC[lane] = none ? kVPadQuery : (code == kCodeX ? kVRegular : code);
    }
  };

  f32x16 acc[DB];                     // A: dV^T, B: dK^T (dims x keys)
#pragma unroll
  for (int db = 0; db < DB; ++db) acc[db] = zero16();

  // Inactive steps multiply stale staging contents by zero words: start every
  // buffer at zero so that stale data is always finite (0 * NaN would not vanish).
  {
    const i32x4 z = {0, 0, 0, 0};
    for (int i = tid; i < 2 * TILE / 8; i += kThreads) {
      reinterpret_cast<i32x4 *>(sT0)[i] = z; reinterpret_cast<i32x4 *>(sT1)[i] = z;
      reinterpret_cast<i32x4 *>(sT2)[i] = z; reinterpret_cast<i32x4 *>(sT3)[i] = z;
      reinterpret_cast<i32x4 *>(sT0)[i + 2 * TILE / 8] = z; reinterpret_cast<i32x4 *>(sT1)[i + 2 * TILE / 8] = z;
      reinterpret_cast<i32x4 *>(sT2)[i + 2 * TILE / 8] = z; reinterpret_cast<i32x4 *>(sT3)[i + 2 * TILE / 8] = z;
    }
    for (int i = tid; i < 2 * kRows; i += kThreads) {
      sL0[i] = 0.f; sL1[i] = 0.f; sE0[i] = 0.f; sE1[i] = 0.f; sC0[i] = kVPadQuery; sC1[i] = kVPadQuery;
    }
    for (int i = tid; i < 4 * 512; i += kThreads) { sP0[i] = 0u; sP1[i] = 0u; }
    __syncthreads();
  }

  auto qb = [&](int i) -> bf16_t * { return i == 0 ? sT0 : (i == 1 ? sT1 : (i == 2 ? sT2 : sT3)); };
  auto db_ = [&](int i) -> bf16_t * { return qb(i) + TILE; };
  auto lb = [&](int i) -> float * { return i == 0 ? sL0 : sL1; };
  auto eb = [&](int i) -> float * { return i == 0 ? sE0 : sE1; };
  auto cb = [&](int i) -> int * { return i == 0 ? sC0 : sC1; };
  auto pbuf = [&](int i) -> uint32_t * { return i == 0 ? sP0 : sP1; };

  // step j's information sits in ring[j % 4] from step j - 2 on
  StepInfo ring[4] = {{0, 0, 0}, {0, 0, 0}, {0, 0, 0}, {0, 0, 0}};
  ring[0] = info_of(0);
  ring[1] = info_of(1);
  if (role == 1) {
    load_rows(ring[0]);
    load_tiles(ring[0], qb(0) + gr * 2 * TILE, db_(0) + gr * 2 * TILE);
    asm volatile("s_waitcnt vmcnt(0)" : "+v"(rl), "+v"(re), "+v"(rc) : : "memory");   // step 0's loads landed
    store_rows(ring[0], sL0 + gr * kRows, sE0 + gr * kRows, sC0 + gr * kRows);
    load_tiles(ring[1], qb(1) + gr * 2 * TILE, db_(1) + gr * 2 * TILE);
  }
  // every wave's key operands (and B's step 0 loads) landed: a wait the
  // compiler sees, so that it knows no tracked load is in flight in the loop
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  // B: dP - delta of the current and the previous step, alternating by step parity
  f32x16 dp2[2] = {zero16(), zero16()};

  // One step of role R: compute step j from Q buffer J % 4, dO buffer J % 4
  // and row buffer J % 2; B's dK of step j - 1 reads Q buffer (J + 3) % 4 and
  // P buffer (J + 1) % 2. Step j + 2's tiles load into buffers (J + 2) % 4,
  // step j + 1's row data into row buffer (J + 1) % 2. Both roles pass the
  // same barrier once per step.
  auto run_step = [&](auto rsel, auto jsel, int j) {
    constexpr int R = decltype(rsel)::value;
    constexpr int J = decltype(jsel)::value;
    const bf16_t *tQ = qb(J % 4);
    const bf16_t *tD = db_(J % 4);
    const bf16_t *tQprev = qb((J + 3) % 4);
    const StepInfo cur = ring[J % 4];
    const StepInfo prev = ring[(J + 3) % 4];
    const StepInfo nxt1 = ring[(J + 1) % 4];
    const bool cur_on = j < nsteps && (cur.flags & 1);
    const bool prev_on = j >= 1 && j - 1 < nsteps && (prev.flags & 1);

    // row data of step j + 1 first: vmcnt retires in issue order, and the
    // wait at the end of this step must not cover the tiles of step j + 2
    const StepInfo nxt2 = info_of(j + 2);
    if constexpr (R == 1) {
      load_rows(nxt1);
      __builtin_amdgcn_sched_barrier(0);
      load_tiles(nxt2, qb((J + 2) % 4) + gr * 2 * TILE, db_((J + 2) % 4) + gr * 2 * TILE);
      __builtin_amdgcn_sched_barrier(0);
    }

    // The products run on every step, inactive ones included (the operands are
    // then stale buffer contents, in bounds): a conditional accumulator update
    // makes the compiler copy the accumulators around the branch. An inactive
    // step contributes nothing because its P / dS words are cleared.
    if constexpr (R == 0) {
      const int keep = cur_on ? -1 : 0;
      // S - lse / scale = Q K^T + (-lse / scale); register r is row 8 (r / 4) + 4 hi + r % 4
      f32x16 sc = rows16(lb(J % 2), rofs);
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
      if (cur.flags & 2) {
        // a real branch: if-converted, full tiles would pay for the masking
        asm volatile("");
        const int *tc = cb(J % 2);
        if (cur.q0 + a.P < key_last) {   // some row precedes one of the wave's keys: causal bound too
          const int thr = key - cur.q0 - a.P - 4 * hi;   // causal: row offset (without 4 hi) >= thr
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const i32x4 qv = *reinterpret_cast<const i32x4 *>(lds_at(tc, rofs + 32 * i));
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const bool ok = (8 * i + e >= thr) & (kw >= qv[e]);
              sc[4 * i + e] = ok ? sc[4 * i + e] : 0.f;
            }
          }
        } else {   // the ordered compare alone (a pad row sits above every key)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const i32x4 qv = *reinterpret_cast<const i32x4 *>(lds_at(tc, rofs + 32 * i));
#pragma unroll
            for (int e = 0; e < 4; ++e) sc[4 * i + e] = kw >= qv[e] ? sc[4 * i + e] : 0.f;
          }
        }
      }
      i32x4 pw[2];
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int t = 0; t < 4; ++t) pw[u][t] = (int)cvt2<E>(sc[8 * u + 2 * t], sc[8 * u + 2 * t + 1]) & keep;
      char *pp = reinterpret_cast<char *>(pbuf(J % 2));
      *reinterpret_cast<i32x4 *>(pp + pofs) = pw[0];
      *reinterpret_cast<i32x4 *>(pp + pofs + 1024) = pw[1];
      // dV^T += dO^T P (16-row slice u, 32-dim block db); the transposed
      // operands are read three MFMAs ahead (one ahead left the MFMAs waiting
      // on the LDS latency: 3-5 % slower at config 2)
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
    } else {
      f32x16 &dp = dp2[J % 2];
      const f32x16 &dprev = dp2[(J + 1) % 2];
      const int keep = prev_on ? -1 : 0;
      // dS of the previous step from A's P: dK^T += Q^T dS
      const char *pp = reinterpret_cast<const char *>(pbuf((J + 1) % 2));
      const i32x4 pw0 = *reinterpret_cast<const i32x4 *>(pp + pofs);
      const i32x4 pw1 = *reinterpret_cast<const i32x4 *>(pp + pofs + 1024);
      const i32x4 pws[2] = {pw0, pw1};
      i32x4 dsw[2];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          // bit_cast of the element through a named scalar: bit_cast of a vector
          // subscript reads the vector's first element instead
          const uint32_t wd = (uint32_t)pws[u][t];
          dsw[u][t] = (int)cvt2<E>(pair_lo<E>(wd) * dprev[8 * u + 2 * t], pair_hi<E>(wd) * dprev[8 * u + 2 * t + 1]) &
                      keep;
        }
      }
      {
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
      dp = rows16(eb(J % 2), rofs);
      bf16x8 op = lds_read8(reinterpret_cast<const bf16_t *>(lds_at(tD, qk[0])));
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        bf16x8 nx;
        if (ks + 1 < KS) nx = lds_read8(reinterpret_cast<const bf16_t *>(lds_at(tD, qk[ks + 1])));
        dp = mfma32<E>(op, kv[ks], dp);
        if (ks + 1 < KS) op = nx;
      }
    }

    if constexpr (R == 1) {
      // this thread's loads of step j + 1 landed (issued one step ago): wait
      // for all but the tiles of step j + 2 just issued
      constexpr int n = 2 * GroupTile<HD>::kInst;
      asm volatile("s_waitcnt vmcnt(%3)" : "+v"(rl), "+v"(re), "+v"(rc) : "n"(n) : "memory");
      store_rows(nxt1, lb((J + 1) % 2) + gr * kRows, eb((J + 1) % 2) + gr * kRows, cb((J + 1) % 2) + gr * kRows);
    }
    ring[(J + 2) % 4] = nxt2;
    lds_barrier();
  };

  // four steps per iteration with no exit in between: an exit inside the
  // unrolled body (or a separate tail) makes every accumulator a join of
  // several register sets, which no longer fit. The step count is rounded up
  // to a multiple of four; the extra steps are inactive (their P / dS words
  // are cleared).
  auto main_loop = [&](auto rsel) {
    for (int j = 0; j < niter; j += 4) {
      run_step(rsel, std::integral_constant<int, 0>{}, j);
      run_step(rsel, std::integral_constant<int, 1>{}, j + 1);
      run_step(rsel, std::integral_constant<int, 2>{}, j + 2);
      run_step(rsel, std::integral_constant<int, 3>{}, j + 3);
    }
  };
  if (role == 0) main_loop(std::integral_constant<int, 0>{});
  else main_loop(std::integral_constant<int, 1>{});
  // the last steps' loads (of steps past the end, into buffers 0 and 1) land
  // before those buffers take the accumulators
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();

  // ---- group 1 hands its accumulators to group 0 (the staging buffers are
  // free after the last barrier): wave (half, role) of group 1 writes into
  // buffer [half][role], 16 KB in quads of registers, lane-interleaved ----
  float *x = reinterpret_cast<float *>((half == 0 ? sT0 : sT1) + role * 2 * TILE);
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
