// Shared device types and helpers for the gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

typedef __bf16 bf16_t;
typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(4 * sizeof(__bf16)))) __bf16 bf16x4;
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

__device__ __forceinline__ bf16x8 load8(const float *p) {
  const f32x4 a = *reinterpret_cast<const f32x4 *>(p);
  const f32x4 b = *reinterpret_cast<const f32x4 *>(p + 4);
  bf16x8 r;
  r[0] = (bf16_t)a[0]; r[1] = (bf16_t)a[1]; r[2] = (bf16_t)a[2]; r[3] = (bf16_t)a[3];
  r[4] = (bf16_t)b[0]; r[5] = (bf16_t)b[1]; r[6] = (bf16_t)b[2]; r[7] = (bf16_t)b[3];
  return r;
}

// ---- stores of 4 consecutive output values -------------------------------

__device__ __forceinline__ void store4(bf16_t *p, float a, float b, float c, float d) {
  bf16x4 v;
  v[0] = (bf16_t)a; v[1] = (bf16_t)b; v[2] = (bf16_t)c; v[3] = (bf16_t)d;
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

// Eight fp32 accumulator values -> one bf16 MFMA operand.
__device__ __forceinline__ bf16x8 pack8(float a0, float a1, float a2, float a3,
                                        float a4, float a5, float a6, float a7) {
  bf16x8 r;
  r[0] = (bf16_t)a0; r[1] = (bf16_t)a1; r[2] = (bf16_t)a2; r[3] = (bf16_t)a3;
  r[4] = (bf16_t)a4; r[5] = (bf16_t)a5; r[6] = (bf16_t)a6; r[7] = (bf16_t)a7;
  return r;
}

__device__ __forceinline__ f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

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
