// Shared device types and helpers for the gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

typedef __bf16 bf16_t;
typedef _Float16 f16_t;
// bf16x8 is also the carrier of any 16-byte MFMA operand fragment: fp16
// fragments travel in it as raw bits and are reinterpreted at the MFMA.
typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(4 * sizeof(__bf16)))) __bf16 bf16x4;
typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2;
typedef __attribute__((__vector_size__(8 * sizeof(_Float16)))) _Float16 f16x8;
typedef __attribute__((__vector_size__(4 * sizeof(_Float16)))) _Float16 f16x4;
typedef __attribute__((__vector_size__(2 * sizeof(_Float16)))) _Float16 f16x2;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;
typedef __attribute__((__vector_size__(4 * sizeof(int)))) int i32x4;
typedef __attribute__((__vector_size__(2 * sizeof(int)))) int i32x2;

namespace mga {

constexpr int kBlock = 128;          // BlockMask tile edge
constexpr int kCodePad = -1;
constexpr int kCodeX = -2;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// ---- 16-byte global loads of 8 elements, returned as bf16x8 --------------

__device__ __forceinline__ bf16x8 load8(const bf16_t *p) {
  return __builtin_bit_cast(bf16x8, *reinterpret_cast<const i32x4 *>(p));
}

// fp16 elements: the raw bits (an fp16 MFMA fragment)
__device__ __forceinline__ bf16x8 load8(const f16_t *p) {
  return __builtin_bit_cast(bf16x8, *reinterpret_cast<const i32x4 *>(p));
}

// ---- stores of 4 consecutive output values -------------------------------

__device__ __forceinline__ void store4(bf16_t *p, float a, float b, float c, float d) {
  bf16x4 v;
  v[0] = (bf16_t)a; v[1] = (bf16_t)b; v[2] = (bf16_t)c; v[3] = (bf16_t)d;
  *reinterpret_cast<i32x2 *>(p) = __builtin_bit_cast(i32x2, v);
}

__device__ __forceinline__ void store4(f16_t *p, float a, float b, float c, float d) {
  f16x4 v;
  v[0] = (f16_t)a; v[1] = (f16_t)b; v[2] = (f16_t)c; v[3] = (f16_t)d;
  *reinterpret_cast<i32x2 *>(p) = __builtin_bit_cast(i32x2, v);
}

__device__ __forceinline__ void store4(float *p, float a, float b, float c, float d) {
  f32x4 v = {a, b, c, d};
  *reinterpret_cast<f32x4 *>(p) = v;
}

// ---- LDS fragment reads ---------------------------------------------------

__device__ __forceinline__ bf16x8 lds_read8(const bf16_t *p) {
  return __builtin_bit_cast(bf16x8, *reinterpret_cast<const i32x4 *>(p));
}

// Two runs of 4 consecutive bf16 (8 bytes each) -> one MFMA operand.
__device__ __forceinline__ bf16x8 lds_read4x2(const bf16_t *p0, const bf16_t *p1) {
  const i32x2 a = *reinterpret_cast<const i32x2 *>(p0);
  const i32x2 b = *reinterpret_cast<const i32x2 *>(p1);
  i32x4 r = {a[0], a[1], b[0], b[1]};
  return __builtin_bit_cast(bf16x8, r);
}

// ---- the 16-bit MFMA element E (bf16_t or f16_t) ---------------------------
// Operand fragments are 8 elements of E carried as bf16x8 bits; conversions
// from fp32 round to nearest even.

template <typename E> struct Elem;
template <> struct Elem<bf16_t> { typedef bf16x8 v8; typedef bf16x2 v2; };
template <> struct Elem<f16_t> { typedef f16x8 v8; typedef f16x2 v2; };

// Eight fp32 accumulator values -> one MFMA operand of E.
template <typename E>
__device__ __forceinline__ bf16x8 pack8(float a0, float a1, float a2, float a3,
                                        float a4, float a5, float a6, float a7) {
  typename Elem<E>::v8 r;
  r[0] = (E)a0; r[1] = (E)a1; r[2] = (E)a2; r[3] = (E)a3;
  r[4] = (E)a4; r[5] = (E)a5; r[6] = (E)a6; r[7] = (E)a7;
  return __builtin_bit_cast(bf16x8, r);
}

// Two fp32 values -> one packed pair of E (x in the low half).
template <typename E>
__device__ __forceinline__ uint32_t cvt2(float x, float y) {
  typename Elem<E>::v2 v;
  v[0] = (E)x;
  v[1] = (E)y;
  return __builtin_bit_cast(uint32_t, v);
}

// The two elements of a packed pair, as fp32.
template <typename E>
__device__ __forceinline__ float pair_lo(uint32_t w) { return (float)__builtin_bit_cast(typename Elem<E>::v2, w)[0]; }
template <typename E>
__device__ __forceinline__ float pair_hi(uint32_t w) { return (float)__builtin_bit_cast(typename Elem<E>::v2, w)[1]; }

// acc + both elements of a packed pair (one v_dot2 against (1, 1)).
template <typename E> __device__ __forceinline__ float add_pair(uint32_t p, float acc);
template <>
__device__ __forceinline__ float add_pair<bf16_t>(uint32_t p, float acc) {
  const bf16x2 one = {(bf16_t)1.0f, (bf16_t)1.0f};
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, p), one, acc, false);
}
template <>
__device__ __forceinline__ float add_pair<f16_t>(uint32_t p, float acc) {
  const f16x2 one = {(f16_t)1.0f, (f16_t)1.0f};
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, p), one, acc, false);
}

// One 32x32x16 MFMA of E operands into fp32.
template <typename E> __device__ __forceinline__ f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c);
template <>
__device__ __forceinline__ f32x16 mfma32<bf16_t>(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
template <>
__device__ __forceinline__ f32x16 mfma32<f16_t>(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                0, 0);
}

// The MFMA element of a 16-bit storage type: itself.
template <typename T> struct MfmaElem;
template <> struct MfmaElem<bf16_t> { typedef bf16_t type; };
template <> struct MfmaElem<f16_t> { typedef f16_t type; };

__device__ __forceinline__ f32x16 zero16() {
  f32x16 z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.f;
  return z;
}

// Swap with the lane 32 away (both halves of a wave hold the same MFMA column).
__device__ __forceinline__ float xor32(float x) { return __shfl_xor(x, 32, 64); }

// MTP predicate from codes: key j (global kv index) is visible to chunk query
// row i (global index i + P) iff causal, the query is not a pad, and the key is
// a regular token or a mask token of the query's own block.
__device__ __forceinline__ bool mtp_allowed(int qglob, int qcode, int key, int kcode) {
  return (key <= qglob) & (qcode != kCodePad) & ((kcode == kCodeX) | (kcode == qcode));
}

// Code of a global key index: cached prefix keys are regular tokens.
__device__ __forceinline__ int key_code(const int32_t *code, int key, int P, int L) {
  return key < P ? kCodeX : (key < L ? code[key - P] : kCodePad);
}

// WG id -> logical work index so that consecutive logical indices land on the
// same XCD (the hardware deals WG ids round-robin over the 8 XCDs).
__device__ __forceinline__ int xcd_swizzle(int b, int n) {
  const int x = b & 7, slot = b >> 3;
  const int per = n >> 3, rem = n & 7;
  return x * per + (x < rem ? x : rem) + slot;
}

}  // namespace mga

namespace mga {

// ---- LDS tiles: rows of HD bf16, 16-byte granules XOR-swizzled per row -----
// Granule c of row r sits at slot c ^ swz(r). The map (linear over GF(2) in
// the low four row bits) keeps both access patterns the kernels use free of
// bank conflicts for 32- and 64-bank LDS: 16-byte row reads of one granule
// by 16 consecutive rows, and the 8-byte transpose reads of 4 consecutive rows
// x 16 (or 32) consecutive columns.
template <int HD>
__device__ __forceinline__ int swz(int r) {
  if constexpr (HD == 128)
    return ((r & 1) ? 4 : 0) ^ ((r & 2) ? 10 : 0) ^ ((r & 4) ? 1 : 0) ^ ((r & 8) ? 2 : 0);
  else
    return ((r & 1) ? 2 : 0) ^ ((r & 2) ? 4 : 0) ^ ((r & 4) ? 1 : 0) ^ ((r & 8) ? 2 : 0);
}

// Element offset of granule g (8 elements) of row r in a swizzled tile.
template <int HD>
__device__ __forceinline__ int tile_off(int r, int g) {
  return r * HD + ((g ^ swz<HD>(r)) << 3);
}

typedef __attribute__((__vector_size__(4 * sizeof(short)))) short i16x4;
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

// 8-byte transpose read (ds_read_b64_tr_b16). Within each 16-lane group, lane
// i receives element i % 4 of the 8-byte loads addressed by lanes i / 4 + 4k,
// k = 0..3: pointing lane j at X[k0 + j / 4][m0 + 4 (j % 4)] of a row-major
// tile hands lane i the column m0 + i at rows k0 .. k0 + 3.
__device__ __forceinline__ i16x4 lds_tr4(const bf16_t *p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4 *)(p));
}

__device__ __forceinline__ bf16x8 join8(i16x4 a, i16x4 b) {
  const i32x2 x = __builtin_bit_cast(i32x2, a), y = __builtin_bit_cast(i32x2, b);
  i32x4 r = {x[0], x[1], y[0], y[1]};
  return __builtin_bit_cast(bf16x8, r);
}

// Per-lane constants of a transposed MFMA A-operand read (32 m-rows x 16 k)
// from a k-major swizzled tile: lane (l32, hi) needs column m0 + l32 at rows
// k0 + 4 hi + 0..3 (slots 0..3) and k0 + 8 + 4 hi + 0..3 (slots 4..7), the k
// order of a 32x32 accumulator's registers 8u .. 8u + 7. For k0 a multiple of
// 16 and m0 a multiple of 32 the swizzle term only depends on the lane, so the
// address is rowbase(k0) + lo[s] + ((m0 / 32) ^ hi2[s]) * 32.
struct TrLane {
  int row[2];   // tile row offset (in rows) of the two reads, relative to k0
  int lo[2];    // low column part, elements
  int hi2[2];   // XOR applied to the 32-column block index
};

template <int HD>
__device__ __forceinline__ TrLane tr_lane(int lane) {
  TrLane t;
  const int i = lane & 15, hi = lane >> 5;
  const int m = 16 * ((lane >> 4) & 1) + 4 * (i & 3);   // column within the 32-block
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    const int r = 4 * hi + (i >> 2) + 8 * s;
    const int sw = swz<HD>(r);
    t.row[s] = r;
    t.lo[s] = ((((m >> 3) ^ sw) & 3) << 3) + (m & 7);
    t.hi2[s] = sw >> 2;
  }
  return t;
}

// A lane offset whose bits the compiler may not reason about. Added to an LDS
// buffer's address it stays an add, so the buffer base and constant parts fold
// into the ds_read offset field; with known-disjoint bits the add becomes an
// or, and every (buffer, offset) pair costs a register.
__device__ __forceinline__ uint32_t opaque_u32(uint32_t x) {
  asm volatile("" : "+v"(x));
  return x;
}

__device__ __forceinline__ const char *lds_at(const void *base, uint32_t byte_off) {
  return reinterpret_cast<const char *>(base) + byte_off;
}

// Byte offsets of the transposed operand reads (see TrLane) for every 32-column
// block: the tile base and the k0 row term are added as constants.
template <int HD>
struct TrOffsets {
  uint32_t off[2][HD / 32];
  __device__ __forceinline__ void init(int lane) {
    const TrLane t = tr_lane<HD>(lane);
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int mb = 0; mb < HD / 32; ++mb)
        off[s][mb] = opaque_u32((uint32_t)(t.row[s] * HD + t.lo[s] + ((mb ^ t.hi2[s]) << 5)) * 2u);
  }
  __device__ __forceinline__ bf16x8 operand(const bf16_t *tile, int k0, int mblk) const {
    const char *b = reinterpret_cast<const char *>(tile) + k0 * HD * 2;
    return join8(lds_tr4(reinterpret_cast<const bf16_t *>(b + off[0][mblk])),
                 lds_tr4(reinterpret_cast<const bf16_t *>(b + off[1][mblk])));
  }
};

template <int HD>
__device__ __forceinline__ bf16x8 lds_tr_operand(const bf16_t *tile, const TrLane &t, int k0, int mblk) {
  const bf16_t *p0 = tile + (k0 + t.row[0]) * HD + t.lo[0] + ((mblk ^ t.hi2[0]) << 5);
  const bf16_t *p1 = tile + (k0 + t.row[1]) * HD + t.lo[1] + ((mblk ^ t.hi2[1]) << 5);
  return join8(lds_tr4(p0), lds_tr4(p1));
}

}  // namespace mga

namespace mga {

// ---- direct global -> LDS staging of an NR x HD bf16 tile (4 waves) ---------
// global_load_lds with 16 bytes per lane writes LDS at base + 16 * lane, so
// each wave instruction fills one contiguous 1 KB block (1024 / (2 HD) rows);
// lane picks the global granule that the swizzle places at its slot. Rows
// beyond rmax repeat row rmax. Completion is tracked by vmcnt: wait for it
// (and a barrier) before the tile is read.
typedef __attribute__((address_space(3))) void lds_void;

template <int HD, int NR>
__device__ __forceinline__ void tile_dma(bf16_t *tile, const bf16_t *src, int64_t ss, int r0, int rmax) {
  constexpr int kGranRow = HD / 8;                 // granules per row
  constexpr int kRowsPerInst = 64 / kGranRow;      // rows per 1 KB block
  constexpr int kInst = NR / kRowsPerInst / 4;     // blocks per wave
  const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int p = lane % kGranRow;
#pragma unroll
  for (int i = 0; i < kInst; ++i) {
    const int blk = w * kInst + i;
    const int r = blk * kRowsPerInst + lane / kGranRow;
    const int c = p ^ swz<HD>(r);
    const int row = min(r0 + r, rmax);
    __builtin_amdgcn_global_load_lds(src + (int64_t)row * ss + c * 8, (lds_void *)(tile + blk * 512), 16, 0, 0);
  }
}

}  // namespace mga

namespace mga {

// The block-mask tile list of one query tile (partial tiles, then full ones),
// cached 64 entries at a time in a register (lane l holds entry base + l) and
// read back with readlane, so a step's tile index costs no memory wait.
// Counts and indices come from the caller's BlockMask tensors: both are
// clamped into range (counts to [0, n], indices to [0, n - 1]), so malformed
// metadata gives wrong results but never an access outside the operands.
struct TileList {
  const int32_t *pidx, *fidx;
  int npart, ntot;
  int lim;          // number of tiles along the listed axis (n)
  int base = -64;
  int val = 0;

  __device__ __forceinline__ int at(int it) {   // it: wave-uniform, < ntot
    const int cb = it & ~63;
    if (cb != base) {
      const int e = cb + (threadIdx.x & 63);
      val = e < npart ? pidx[e] : (e < ntot ? fidx[e - npart] : 0);
      val = min(max(val, 0), lim - 1);
      base = cb;
      // wait for the refill here (once per 64 tiles): left to the use, the
      // wait would sit on every call and drain all loads in flight
      __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8));   // vmcnt(0) only
    }
    return __builtin_amdgcn_readlane(val, it & 63);
  }
};

// Tile list of row r of a BlockMask: partial tiles pidx[r * n ..], count
// pnum[r]; full tiles fidx[r * n ..], count fnum[r]; n tiles per row.
__device__ __forceinline__ TileList tile_list(const int32_t *pnum, const int32_t *pidx, const int32_t *fnum,
                                              const int32_t *fidx, int r, int n) {
  const int np = min(max(pnum[r], 0), n);
  const int nf = min(max(fnum[r], 0), n - np);
  return TileList{pidx + (int64_t)r * n, fidx + (int64_t)r * n, np, np + nf, n};
}

}  // namespace mga

namespace mga {

constexpr int kWX = 0x7ffffffe;      // ordered-compare value of a regular key / query
constexpr int kWPad = -0x7fffffff;   // ordered-compare value of a pad key
constexpr int kVPad = 0x7fffffff;    // ordered-compare value of a pad query: above every key

// Ordered-compare form of the MTP predicate: allowed(q, k) = (k <= qlim(q)) &
// (key_w(k) >= query_v(q)). A mask key at or before the query carries a code
// (num_prefix_x) no larger than the query's, equal exactly within the query's
// own block, so one compare replaces "key is regular or in the same block".
// A pad query sits above every key, so the compare alone masks its row.
__device__ __forceinline__ int key_w(const int32_t *code, int key, int P, int L) {
  if (key < P) return kWX;
  if (key >= L) return kWPad;
  const int c = code[key - P];
  return c == kCodeX ? kWX : (c == kCodePad ? kWPad : c);
}

__device__ __forceinline__ int query_v(int qcode) {
  return qcode == kCodeX ? kWX : (qcode == kCodePad ? kVPad : qcode);
}

// Workgroup barrier without the memory fences of __syncthreads(): the
// workgroup-scope release fence there waits for every direct global -> LDS
// load in flight (they write LDS), which would end any prefetch across the
// barrier. The caller has waited (s_waitcnt vmcnt) for the direct loads the
// next step reads; this wave's LDS writes are complete at lgkmcnt(0), and the
// memory clobber keeps the compiler from moving memory accesses across.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Direct global -> LDS loads of 16 bytes per lane (global_load_lds_dwordx4;
// M0 holds the LDS address of the 1 KB block the wave writes) issued as
// inline asm, outside the compiler's wait counting: the caller owns every
// wait (s_waitcnt vmcnt) before the bytes are read or the buffer is reused.
// Scalar base plus a 32-bit lane offset, or a per-lane 64-bit address.
__device__ __forceinline__ uint32_t lds_addr(const void *p) {
  return (uint32_t)(size_t)(const __attribute__((address_space(3))) void *)p;
}
__device__ __forceinline__ void dma16(const void *sbase, uint32_t voff, const void *lds) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
               :
               : "v"(voff), "s"(sbase), "s"(lds_addr(lds))
               : "memory", "m0");
}
__device__ __forceinline__ void dma16(const void *gaddr, const void *lds) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
               :
               : "v"(gaddr), "s"(lds_addr(lds))
               : "memory", "m0");
}

// Raw buffer resource (stride 0) over nbytes from base: a load at a byte
// offset >= nbytes returns zeros. base, nbytes are wave-uniform.
__device__ __forceinline__ i32x4 buf_rsrc(const void *base, uint32_t nbytes) {
  const uint64_t b = reinterpret_cast<uint64_t>(base);
  i32x4 r;
  r[0] = __builtin_amdgcn_readfirstlane((int)(uint32_t)b);
  r[1] = __builtin_amdgcn_readfirstlane((int)((uint32_t)(b >> 32) & 0xffffu));
  r[2] = __builtin_amdgcn_readfirstlane((int)nbytes);
  r[3] = 0x00020000;
  return r;
}

// Buffer -> LDS loads of 16 (or 4) bytes per lane: lane l writes LDS at
// lds + 16 l (4 l), from byte offset voff of the resource. Inline asm outside
// the compiler's wait counting: the caller owns the vmcnt waits.
__device__ __forceinline__ void bdma16(const i32x4 &r, uint32_t voff, const void *lds) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds"
               :
               : "v"(voff), "s"(r), "s"(lds_addr(lds))
               : "memory", "m0");
}
__device__ __forceinline__ void bdma4(const i32x4 &r, uint32_t voff, const void *lds) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tbuffer_load_dword %0, %1, 0 offen lds"
               :
               : "v"(voff), "s"(r), "s"(lds_addr(lds))
               : "memory", "m0");
}

// The wave's index within the workgroup as a scalar (wave-uniform) value, so
// LDS block bases derived from it stay in scalar registers.
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

// Per-lane offsets of the direct loads of an NR x HD tile (see tile_dma). Load
// i of wave w covers tile rows (w * kInst + i) * kRowsPerInst + lane / kGranRow:
// the wave-uniform part of that row goes into the scalar base address, the
// lane's row term (lrow, bytes) and granule term (gran[i], bytes; the swizzle
// is linear in the row bits, so it splits into a lane part and an i part)
// into the 32-bit vector offset. gran does not depend on the row stride, so
// tiles of different sources share it. NW waves share the loads of a tile:
// with more waves in the workgroup, each group of NW consecutive waves stages
// its own tiles.
template <int HD, int NR, int NW = 4>
struct DmaLane {
  static constexpr int kGranRow = HD / 8;
  static constexpr int kRowsPerInst = 64 / kGranRow;
  static constexpr int kInst = NR / kRowsPerInst / NW;
  static_assert(kInst >= 1 && kInst * kRowsPerInst * NW == NR, "tile rows must split evenly over the waves");
  static_assert((NW & (NW - 1)) == 0, "NW must be a power of two");
  // the wave's index within its group of NW
  __device__ __forceinline__ static int gw() { return wave_id() & (NW - 1); }
  uint32_t gran[kInst];
  __device__ __forceinline__ void init() {
    const int lane = threadIdx.x & 63, w = gw();
    const int p = lane % kGranRow;
#pragma unroll
    for (int i = 0; i < kInst; ++i) {
      const int r = (w * kInst + i) * kRowsPerInst + lane / kGranRow;
      gran[i] = opaque_u32((uint32_t)((p ^ swz<HD>(r)) << 4));
    }
  }
  // byte offset of the lane's row within a load's row block, for row stride ss
  __device__ __forceinline__ static uint32_t lane_row(int64_t ss) {
    return opaque_u32((uint32_t)(((threadIdx.x & 63) / kGranRow) * ss * 2));
  }
  // only rows 0 .. nvalid - 1 of the tile exist, 1 <= nvalid < NR (callers
  // issue nothing for a tile with no rows): later rows repeat the last one
  __device__ __forceinline__ void issue_clamped(bf16_t *tile, const bf16_t *rowbase, int64_t ss,
                                                int nvalid) const {
    const int lane = threadIdx.x & 63, w = gw();
    const int p = lane % kGranRow;
    const char *base = reinterpret_cast<const char *>(rowbase);
#pragma unroll
    for (int i = 0; i < kInst; ++i) {
      const int r = (w * kInst + i) * kRowsPerInst + lane / kGranRow;
      const uint32_t o = (uint32_t)(min(r, nvalid - 1) * (int)ss * 2) + (uint32_t)((p ^ swz<HD>(r)) << 4);
      __builtin_amdgcn_global_load_lds(base + o, (lds_void *)(tile + (w * kInst + i) * 512), 16, 0, 0);
    }
  }
  // Scalar byte offsets for row stride ss: the wave's first row block and the
  // step to the next load's block. Formed once per kernel, so a load's scalar
  // address is one 64-bit add instead of a 64-bit multiply.
  struct Rows {
    int64_t wave;
    int64_t inst;
  };
  __device__ __forceinline__ static Rows rows(int64_t ss) {
    return {(int64_t)(gw() * kInst * kRowsPerInst) * ss * 2, (int64_t)kRowsPerInst * ss * 2};
  }
  // rows r0 .. r0 + NR - 1 all exist in the source; rowbase is wave-uniform
  __device__ __forceinline__ void issue(bf16_t *tile, const bf16_t *rowbase, const Rows &rs, uint32_t lrow) const {
    const char *blk = reinterpret_cast<const char *>(rowbase) + rs.wave;
    bf16_t *dst = tile + gw() * kInst * 512;
#pragma unroll
    for (int i = 0; i < kInst; ++i) {
      // formed at the use: hoisted out of a loop, the sums would hold registers
      const uint32_t vo = opaque_u32(lrow) + gran[i];
      __builtin_amdgcn_global_load_lds(blk + vo, (lds_void *)(dst + i * 512), 16, 0, 0);
      blk += rs.inst;
    }
  }
};

// The same tiles through a raw buffer resource whose range ends at the
// source's last row: the lane offsets (row term for the source's stride plus
// the swizzled granule) are formed once per source, the tile's first row goes
// into the resource base, so a load costs no vector instruction, and rows at
// or past the range's end arrive as zeros (no clamped form for a chunk's last
// rows).
template <int HD, int NR, int NW = 4>
struct BufDma {
  static constexpr int kGranRow = HD / 8;
  static constexpr int kRowsPerInst = 64 / kGranRow;
  static constexpr int kInst = NR / kRowsPerInst / NW;
  static_assert(kInst >= 1 && kInst * kRowsPerInst * NW == NR, "tile rows must split evenly over the waves");
  static_assert((NW & (NW - 1)) == 0, "NW must be a power of two");
  __device__ __forceinline__ static int gw() { return wave_id() & (NW - 1); }
  uint32_t vo[kInst];
  __device__ __forceinline__ void init(int64_t ss) {
    const int lane = threadIdx.x & 63, w = gw();
    const int p = lane % kGranRow;
#pragma unroll
    for (int i = 0; i < kInst; ++i) {
      const int r = (w * kInst + i) * kRowsPerInst + lane / kGranRow;
      vo[i] = opaque_u32((uint32_t)(r * ss * 2) + (uint32_t)((p ^ swz<HD>(r)) << 4));
    }
  }
  // rows 0 .. NR - 1 from rowbase (wave-uniform), the first nrows >= 1 of
  // them in the source (the range: nrows rows of ss >= HD elements, so every
  // 16-byte load of a row in range lies wholly inside it)
  __device__ __forceinline__ void issue(bf16_t *tile, const void *rowbase, int64_t ss, int nrows) const {
    const i32x4 r = buf_rsrc(rowbase, (uint32_t)((int64_t)min(nrows, NR) * ss * 2));
    bf16_t *dst = tile + gw() * kInst * 512;
#pragma unroll
    for (int i = 0; i < kInst; ++i) bdma16(r, vo[i], dst + i * 512);
  }
};

}  // namespace mga

namespace mga {

// A key's code fetched one step ahead: load() only issues the read (so it does
// not wait on the tile loads in flight), w() converts at store time.
struct KeyCode {
  int raw = 0;   // the key's code (a cached prefix key reads as regular, a key past the end as pad)
  __device__ __forceinline__ void load(const int32_t *code, int key, int P, int L) {
    raw = kCodeX;
    if (key >= P) raw = key < L ? code[key - P] : kCodePad;
  }
  // selects, not branches: one conversion per step on the load path
  __device__ __forceinline__ int w() const {
    const int v = raw == kCodePad ? kWPad : raw;
    return raw == kCodeX ? kWX : v;
  }
};

}  // namespace mga
