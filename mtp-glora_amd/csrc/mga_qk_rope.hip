// Qwen3 q_norm / k_norm (RMSNorm over head_dim) + rotary embedding of the
// query and key states, fused, for gfx950. HBM-bound elementwise work with one
// reduction per row: each (token, head) row of D elements is read once and its
// embedding written once; the norm weights and the token's cos / sin rows come
// from cache.
//
// Reference (mtp_glora/models/modeling_qwen3.py): Qwen3RMSNorm.forward :61-67
//   y = T(x * rsqrt(mean(x * x) + eps)),  n = T(w * y)   (x, mean in fp32)
// then apply_rotary_pos_emb :125-149 with rotate_half :118-122
//   out = T(T(n * cos) + T(rotate_half(n) * sin)),
//   rotate_half(n) = [-n[D/2:], n[:D/2]],
// T rounding to the model dtype after each op as the reference's torch ops do
// (fp contraction is off in the forward so fp32 models round each op too).
// The forward can also copy the value rows, so one launch writes a layer's
// post-RoPE keys and its values straight into their KV-cache rows (the
// cache update of modeling_qwen3.py:281-284 then has nothing left to copy).
//
// Layout: grid (token, head block), one wave per workgroup. A group of G lanes
// (a power of two, G * V >= D / 2) owns one (token, head) row; a wave's 64 / G
// groups take consecutive query heads or consecutive key heads, so pointers
// and strides are wave-uniform. Lane j holds the V elements d = jV .. jV+V-1
// of the first half and d + D/2 of the second, so rotate_half pairs meet in
// one lane and the row reduction is a log2(G)-step xor shuffle inside the
// group. V is the widest of 8 (bf16) / 4 that D/2 and every address allow
// (16-byte accesses), else 1. Each bf16 rounding is one conversion
// instruction whose result needs no unpacking. Short waves (about five per
// token at Qwen3-8B's 40 heads) keep the waves of a SIMD out of step, so
// loads of one overlap the rounding work of another, which costs about as
// much VALU time as the rows' HBM traffic.
// The row sum of squares is summed in this kernel's order; torch's order
// differs, so the mean can differ in its last fp32 bit and flip the rounding
// of a rare output element.
//
// Backward (fp32 throughout, the roundings taken as identity):
//   dn = g * cos + rotate_half^T(g * sin),  rotate_half^T(u) = [u[D/2:], -u[:D/2]]
//   dy = dn * w,  dx = r dy - (r^3 / D) x sum(dy * x)
// The norm weights get no gradient (the reference trains LoRA parameters only).
#include "mga_common.hpp"
#include "mga_internal.hpp"

namespace mga {

namespace {

// Two fp32 values rounded to bf16 (nearest even) in one register, a in the low
// half. Written as asm: the compiler splits the pair into two conversions.
__device__ __forceinline__ uint32_t pk_bf16(float a, float b) {
  uint32_t u;
  asm("v_cvt_pk_bf16_f32 %0, %1, %2" : "=v"(u) : "v"(a), "v"(b));
  return u;
}


// Rounding to the model dtype, result as fp32 (fp32: identity). For bf16,
// v_cvt_pk_bf16_f32 with a zero low partner leaves the rounded value in the
// high half over zero bits: that register is the rounded value as an fp32,
// one instruction and nothing to unpack.
template <typename T>
struct Rnd {
  __device__ __forceinline__ static float one(float v) { return v; }
};
template <>
struct Rnd<bf16_t> {
  __device__ __forceinline__ static float one(float v) { return __uint_as_float(pk_bf16(0.f, v)); }
};
// fp16: round to nearest even and back, as two instructions the optimiser
// cannot fold (folded into packed fp16 arithmetic, this kernel's fp16 form
// fails instruction selection with packed fp32 disabled)
template <>
struct Rnd<f16_t> {
  __device__ __forceinline__ static float one(float v) {
    uint32_t h;
    float r;
    asm("v_cvt_f16_f32 %0, %1" : "=v"(h) : "v"(v));
    asm("v_cvt_f32_f16 %0, %1" : "=v"(r) : "v"(h));
    return r;
  }
};

// V consecutive elements of T <-> fp32.
template <typename T, int V>
struct Elems {
  __device__ __forceinline__ static void load(const T *p, float (&v)[V]) {
#pragma unroll
    for (int i = 0; i < V; ++i) v[i] = (float)p[i];
  }
  __device__ __forceinline__ static void store(T *p, const float (&v)[V]) {
#pragma unroll
    for (int i = 0; i < V; ++i) p[i] = (T)v[i];
  }
};
// 16-bit elements (bf16, fp16), V = 8 (16 bytes) or 4 (8 bytes)
template <typename T, int V>
struct Elems16 {
  typedef T vt __attribute__((ext_vector_type(V)));
  __device__ __forceinline__ static void load(const T *p, float (&v)[V]) {
    const vt a = *reinterpret_cast<const vt *>(p);
#pragma unroll
    for (int i = 0; i < V; ++i) v[i] = (float)a[i];
  }
  __device__ __forceinline__ static void store(T *p, const float (&v)[V]) {
    vt a;
#pragma unroll
    for (int i = 0; i < V; ++i) a[i] = (T)v[i];
    if constexpr (V == 8)   // non-temporal: the outputs are streamed once and read by a later kernel
      __builtin_nontemporal_store(__builtin_bit_cast(i32x4, a), reinterpret_cast<i32x4 *>(p));
    else
      *reinterpret_cast<vt *>(p) = a;
  }
};
template <> struct Elems<bf16_t, 8> : Elems16<bf16_t, 8> {};
template <> struct Elems<bf16_t, 4> : Elems16<bf16_t, 4> {};
template <> struct Elems<f16_t, 8> : Elems16<f16_t, 8> {};
template <> struct Elems<f16_t, 4> : Elems16<f16_t, 4> {};
template <>
struct Elems<float, 4> {
  __device__ __forceinline__ static void load(const float *p, float (&v)[4]) {
    const f32x4 a = *reinterpret_cast<const f32x4 *>(p);
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = a[i];
  }
  __device__ __forceinline__ static void store(float *p, const float (&v)[4]) {
    __builtin_nontemporal_store(f32x4{v[0], v[1], v[2], v[3]}, reinterpret_cast<f32x4 *>(p));
  }
};

// Both halves of one row: elements d .. d + V - 1 and the same + D/2.
template <typename T, int V>
struct Half2 {
  float lo[V], hi[V];
  __device__ __forceinline__ void load(const T *p, int half) {
    Elems<T, V>::load(p, lo);
    Elems<T, V>::load(p + half, hi);
  }
  __device__ __forceinline__ void store(T *p, int half) const {
    Elems<T, V>::store(p, lo);
    Elems<T, V>::store(p + half, hi);
  }
};

__device__ __forceinline__ float group_sum(float v, int lg) {
  for (int m = (1 << lg) >> 1; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  return v;
}

}  // namespace

// The rows one wave works on: block blockIdx.y of the token's query heads
// (blocks 0 .. nbq - 1), key heads (the next nbk) or, in a forward that
// stages the values too, value heads (the last nbk), one head per lane group.
// Everything here is wave-uniform.
template <typename T>
struct Block {
  bool isq;
  bool isv;          // a value row copy, no normalisation
  int h0;            // first head of the block
  int nh;            // heads of this operand
  int rstd0;         // rstd index of head 0 of this operand within the token
};

template <typename T>
__device__ __forceinline__ Block<T> block_of(const QkRopeArgs &a, int ngrp) {
  const int nbq = a.q ? (a.Hq + ngrp - 1) / ngrp : 0, nbk = (a.Hkv + ngrp - 1) / ngrp;
  const int b = blockIdx.y;
  Block<T> k;
  k.isq = b < nbq;
  k.isv = b >= nbq + nbk;   // the forward's value-copy blocks (a.v set)
  k.h0 = (k.isq ? b : (k.isv ? b - nbq - nbk : b - nbq)) * ngrp;
  k.nh = k.isq ? a.Hq : a.Hkv;
  k.rstd0 = k.isq ? 0 : a.Hq;
  return k;
}

// Grid (token, head block), one wave per workgroup: many short waves, so the
// waves on a SIMD fall out of step and one's loads overlap another's math.
template <typename T, int V>
__global__ __launch_bounds__(64) void qk_norm_rope_fwd_kernel(QkRopeArgs a, int lg, float inv_d) {
#pragma clang fp contract(off)
  const int so = blockIdx.x;   // output row
  const int lane = threadIdx.x;
  const int j = lane & ((1 << lg) - 1), ngrp = 64 >> lg;
  const Block<T> b = block_of<T>(a, ngrp);
  const int h = b.h0 + (lane >> lg);
  if (h >= b.nh) return;   // whole groups leave together
  const int s = a.rows ? a.rows[so] : so;   // input row (and cos / sin row)
  if (a.rows && (s < 0 || s >= a.src_rows)) return;
  const int half = a.D >> 1;
  const bool on = j * V < half;
  const int d = on ? j * V : 0;
  if (b.isv) {   // stage the value row (e.g. into its cache row), unchanged
    Half2<T, V> v;
    v.load(reinterpret_cast<const T *>(a.v) + (int64_t)s * a.v_ss + (int64_t)h * a.v_hs + d, half);
    if (on) v.store(reinterpret_cast<T *>(a.vo) + (int64_t)so * a.vo_ss + (int64_t)h * a.vo_hs + d, half);
    return;
  }
  const T *x0 = reinterpret_cast<const T *>(b.isq ? a.q : a.k) + (int64_t)s * (b.isq ? a.q_ss : a.k_ss);
  Half2<T, V> x, w, c, sn;
  x.load(x0 + (int64_t)h * (b.isq ? a.q_hs : a.k_hs) + d, half);
  w.load(reinterpret_cast<const T *>(b.isq ? a.qw : a.kw) + d, half);
  c.load(reinterpret_cast<const T *>(a.cos) + (int64_t)s * a.cs_ss + d, half);
  sn.load(reinterpret_cast<const T *>(a.sin) + (int64_t)s * a.cs_ss + d, half);
  // x * x is exact in fp32 for bf16 x, so a fused multiply-add rounds each
  // partial sum once, as torch's pow(2) then sum does
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < V; ++i) ss = __builtin_fmaf(x.hi[i], x.hi[i], __builtin_fmaf(x.lo[i], x.lo[i], ss));
  // torch's mean multiplies the sum by 1 / D
  const float var = group_sum(on ? ss : 0.f, lg) * inv_d;
  const float r = rsqrtf(var + a.eps);
  Half2<T, V> o;
#pragma unroll
  for (int i = 0; i < V; ++i) {
    const float n0 = Rnd<T>::one(w.lo[i] * Rnd<T>::one(x.lo[i] * r));
    const float n1 = Rnd<T>::one(w.hi[i] * Rnd<T>::one(x.hi[i] * r));
    o.lo[i] = Rnd<T>::one(n0 * c.lo[i]) + Rnd<T>::one(-n1 * sn.lo[i]);   // rounded by the store
    o.hi[i] = Rnd<T>::one(n1 * c.hi[i]) + Rnd<T>::one(n0 * sn.hi[i]);
  }
  T *out = reinterpret_cast<T *>(b.isq ? a.qo : a.ko) + (int64_t)so * (b.isq ? a.qo_ss : a.ko_ss) +
           (int64_t)h * (b.isq ? a.qo_hs : a.ko_hs) + d;
  if (on) o.store(out, half);
  if (j == 0 && a.rstd) a.rstd[(int64_t)so * (a.Hq + a.Hkv) + b.rstd0 + h] = r;
}

template <typename T, int V>
__global__ __launch_bounds__(64) void qk_norm_rope_bwd_kernel(QkRopeArgs a, int lg, float inv_d) {
  // The token index is formed per lane (threadIdx.x >> 6 is 0 in a one-wave
  // workgroup) and bounds-checked: the same rows, but the compiler's code for
  // this form measured 24.6 us against 27.1 us at [5120, 32 + 8, 128] bf16
  // (the forward measured slower with it and keeps the plain form).
  const int s = blockIdx.x + (int)(threadIdx.x >> 6);
  if (s >= a.S) return;
  const int lane = threadIdx.x & 63;
  const int j = lane & ((1 << lg) - 1), ngrp = 64 >> lg;
  const Block<T> b = block_of<T>(a, ngrp);
  const int h = b.h0 + (lane >> lg);
  if (h >= b.nh) return;   // whole groups leave together
  const int half = a.D >> 1;
  const bool on = j * V < half;
  const int d = on ? j * V : 0;
  Half2<T, V> x, g, w, c, sn;
  x.load(reinterpret_cast<const T *>(b.isq ? a.q : a.k) + (int64_t)s * (b.isq ? a.q_ss : a.k_ss) +
             (int64_t)h * (b.isq ? a.q_hs : a.k_hs) + d, half);
  g.load(reinterpret_cast<const T *>(b.isq ? a.dqo : a.dko) + (int64_t)s * (b.isq ? a.dqo_ss : a.dko_ss) +
             (int64_t)h * (b.isq ? a.dqo_hs : a.dko_hs) + d, half);
  w.load(reinterpret_cast<const T *>(b.isq ? a.qw : a.kw) + d, half);
  c.load(reinterpret_cast<const T *>(a.cos) + (int64_t)s * a.cs_ss + d, half);
  sn.load(reinterpret_cast<const T *>(a.sin) + (int64_t)s * a.cs_ss + d, half);
  const float r = a.rstd[(int64_t)s * (a.Hq + a.Hkv) + b.rstd0 + h];
  float dy0[V], dy1[V], dot = 0.f;
#pragma unroll
  for (int i = 0; i < V; ++i) {
    // out0 = n0 c0 - n1 s0, out1 = n1 c1 + n0 s1
    dy0[i] = (g.lo[i] * c.lo[i] + g.hi[i] * sn.hi[i]) * w.lo[i];
    dy1[i] = (g.hi[i] * c.hi[i] - g.lo[i] * sn.lo[i]) * w.hi[i];
    dot += dy0[i] * x.lo[i] + dy1[i] * x.hi[i];
  }
  dot = group_sum(on ? dot : 0.f, lg);
  const float k3 = r * r * r * dot * inv_d;
  Half2<T, V> dx;
#pragma unroll
  for (int i = 0; i < V; ++i) {
    dx.lo[i] = r * dy0[i] - k3 * x.lo[i];
    dx.hi[i] = r * dy1[i] - k3 * x.hi[i];
  }
  T *out = reinterpret_cast<T *>(b.isq ? a.dq : a.dk) + (int64_t)s * (b.isq ? a.dq_ss : a.dk_ss) +
           (int64_t)h * (b.isq ? a.dq_hs : a.dk_hs) + d;
  if (on) dx.store(out, half);
}

namespace {

bool aligned(const void *p, int bytes) { return p == nullptr || ((uintptr_t)p % (uintptr_t)bytes) == 0; }

// Can every lane access V elements at once? Each row start (pointer plus any
// multiple of the strides) must sit on a V-element boundary.
bool vec_ok(const QkRopeArgs &a, bool backward, int V, int eb) {
  if ((a.D / 2) % V != 0) return false;
  const int vb = V * eb;
  for (const void *p : {a.q, a.k, a.qw, a.kw, a.cos, a.sin, (const void *)a.qo, (const void *)a.ko, a.dqo, a.dko,
                        (const void *)a.dq, (const void *)a.dk, a.v, (const void *)a.vo})
    if (!aligned(p, vb)) return false;
  for (int64_t s : {a.q_ss, a.q_hs, a.k_ss, a.k_hs, a.cs_ss})
    if (s % V) return false;
  if (backward) {
    for (int64_t s : {a.dqo_ss, a.dqo_hs, a.dko_ss, a.dko_hs, a.dq_ss, a.dq_hs, a.dk_ss, a.dk_hs})
      if (s % V) return false;
  } else {
    for (int64_t s : {a.qo_ss, a.qo_hs, a.ko_ss, a.ko_hs, a.v_ss, a.v_hs, a.vo_ss, a.vo_hs})
      if (s % V) return false;
  }
  return true;
}

template <typename T, int V>
void launch_v(const QkRopeArgs &a, bool backward, hipStream_t st) {
  const int half = a.D / 2;
  int lg = 0;
  while ((1 << lg) * V < half) ++lg;   // half <= 64, so G = 1 << lg <= 64
  const int ngrp = 64 >> lg;
  const int nbk = (a.Hkv + ngrp - 1) / ngrp;
  const int nblk = (a.q ? (a.Hq + ngrp - 1) / ngrp : 0) + nbk + (!backward && a.v ? nbk : 0);
  const dim3 grid((unsigned)a.S, (unsigned)nblk), block(64);
  const float inv_d = 1.f / (float)a.D;
  if (backward) hipLaunchKernelGGL((qk_norm_rope_bwd_kernel<T, V>), grid, block, 0, st, a, lg, inv_d);
  else hipLaunchKernelGGL((qk_norm_rope_fwd_kernel<T, V>), grid, block, 0, st, a, lg, inv_d);
}

template <typename T>
void launch_typed(const QkRopeArgs &a, bool backward, hipStream_t st) {
  constexpr int kWide = 16 / (int)sizeof(T);   // 8 bf16 / fp16 or 4 fp32 per 16-byte access
  if (vec_ok(a, backward, kWide, (int)sizeof(T))) launch_v<T, kWide>(a, backward, st);
  else if (sizeof(T) == 2 && vec_ok(a, backward, 4, 2)) launch_v<T, 4>(a, backward, st);
  else launch_v<T, 1>(a, backward, st);
}

}  // namespace

void launch_qk_norm_rope(const QkRopeArgs &a, int dtype, bool backward, hipStream_t st) {
  if (dtype == kDtF32) launch_typed<float>(a, backward, st);
  else if (dtype == kDtF16) launch_typed<f16_t>(a, backward, st);
  else launch_typed<bf16_t>(a, backward, st);
}

}  // namespace mga
