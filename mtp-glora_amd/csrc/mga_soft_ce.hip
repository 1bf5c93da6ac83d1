// Stable soft cross-entropy of the MTP sampler loss (student logits x, teacher
// logits t, one row per drafted position) for gfx950. HBM-bound: each kernel
// streams its rows once.
//
// Forward, two launches:
//   soft_ce_partial_kernel  - grid (row, column split): one pass over a column
//       range of x and t keeps the online statistics of both rows at once,
//       (mx, dx) of x and (mt, dt, S = sum e^{t - mt} x) of t, and writes
//       them per split;
//   soft_ce_combine_kernel  - one thread per row merges the splits in a fixed
//       order and writes ce = -S / dt + mx + log dx and (mx, dx, mt, dt).
// The reference reads x twice (an x pass, then a fused t + x pass,
// mtp_glora/core/loss.py:63-124); here both rows are read once.
// Backward: grad_x = go * (e^{x - mx} / dx - e^{t - mt} / dt), written in the
// student's dtype (loss.py:188-222, 307-330).
// Exponentials are exp2 of log2(e)-scaled arguments; the clamps of dx and dt
// at 1e-20 follow loss.py:85, 112, 203-205.
#include "mga_common.hpp"
#include "mga_internal.hpp"

namespace mga {

namespace {

constexpr int kThreads = 256;
constexpr float kL2E = 1.4426950408889634f;
constexpr float kClamp = 1e-20f;
constexpr float kNegInf = -__builtin_huge_valf();
constexpr int kChunkQuantum = 2048;   // column split granularity (a multiple of every vector width)

__device__ __forceinline__ float ex2(float v) { return __builtin_amdgcn_exp2f(v); }

// Online statistics of one row segment: x: (mx, dx); t: (mt, dt, s).
struct Stats {
  float mx = kNegInf, dx = 0.f, mt = kNegInf, dt = 0.f, s = 0.f;

  // a group of n consecutive (x, t) values
  template <int N>
  __device__ __forceinline__ void add(const float (&x)[N], const float (&t)[N]) {
    float gx = x[0], gt = t[0];
#pragma unroll
    for (int i = 1; i < N; ++i) {
      gx = fmaxf(gx, x[i]);
      gt = fmaxf(gt, t[i]);
    }
    if (gx > mx) {   // never true for an all -inf group
      dx *= ex2((mx - gx) * kL2E);   // 0 while mx = -inf
      mx = gx;
    }
    if (gt > mt) {
      const float sc = ex2((mt - gt) * kL2E);
      dt *= sc;
      s *= sc;
      mt = gt;
    }
    const float mxl = mx * kL2E, mtl = mt * kL2E;
#pragma unroll
    for (int i = 0; i < N; ++i) {
      dx += ex2(__builtin_fmaf(x[i], kL2E, -mxl));
      const float e = ex2(__builtin_fmaf(t[i], kL2E, -mtl));
      dt += e;
      s = __builtin_fmaf(e, x[i], s);
    }
  }

  __device__ __forceinline__ void merge(const Stats &o) {
    const float nx = fmaxf(mx, o.mx);
    if (nx != kNegInf) {
      dx = dx * ex2((mx - nx) * kL2E) + o.dx * ex2((o.mx - nx) * kL2E);
      mx = nx;
    }
    const float nt = fmaxf(mt, o.mt);
    if (nt != kNegInf) {
      const float a = ex2((mt - nt) * kL2E), b = ex2((o.mt - nt) * kL2E);
      dt = dt * a + o.dt * b;
      s = s * a + o.s * b;
      mt = nt;
    }
  }

  __device__ __forceinline__ Stats shfl_xor(int m) const {
    Stats o;
    o.mx = __shfl_xor(mx, m, 64);
    o.dx = __shfl_xor(dx, m, 64);
    o.mt = __shfl_xor(mt, m, 64);
    o.dt = __shfl_xor(dt, m, 64);
    o.s = __shfl_xor(s, m, 64);
    return o;
  }
};

// 16-byte vectors of the element type <-> fp32.
template <typename T>
struct Vec {   // bf16 and fp16
  static constexpr int W = 8;
  __device__ __forceinline__ static void load(const T *p, float (&v)[W]) {
    const auto a = __builtin_bit_cast(typename Elem<T>::v8, load8(p));
#pragma unroll
    for (int i = 0; i < W; ++i) v[i] = (float)a[i];
  }
  __device__ __forceinline__ static void store(T *p, const float (&v)[W]) {
    typename Elem<T>::v8 a;
#pragma unroll
    for (int i = 0; i < W; ++i) a[i] = (T)v[i];
    *reinterpret_cast<i32x4 *>(p) = __builtin_bit_cast(i32x4, a);
  }
};
template <>
struct Vec<float> {
  static constexpr int W = 4;
  __device__ __forceinline__ static void load(const float *p, float (&v)[W]) {
    const f32x4 a = *reinterpret_cast<const f32x4 *>(p);
#pragma unroll
    for (int i = 0; i < W; ++i) v[i] = a[i];
  }
  __device__ __forceinline__ static void store(float *p, const float (&v)[W]) {
    f32x4 a = {v[0], v[1], v[2], v[3]};
    *reinterpret_cast<f32x4 *>(p) = a;
  }
};

}  // namespace

// VEC: 16-byte vector loads (row starts 16-byte aligned); else element loads.
template <typename T, bool VEC>
__global__ __launch_bounds__(kThreads) void soft_ce_partial_kernel(const T *__restrict__ x, int64_t xs,
                                                                 const T *__restrict__ t, int64_t ts,
                                                                 int32_t V, int32_t chunk, int32_t nsplit,
                                                                 float *__restrict__ part) {
  const int tid = threadIdx.x;
  const int row = blockIdx.x / nsplit, sp = blockIdx.x - row * nsplit;
  const int c0 = sp * chunk, c1 = min(V, c0 + chunk);
  const T *xr = x + (int64_t)row * xs;
  const T *tr = t + (int64_t)row * ts;
  Stats st;
  int cs = c0;   // first column left for the element loop
  if constexpr (VEC) {
    constexpr int W = Vec<T>::W;
    const int nvec = (c1 - c0) / W;
    for (int i = tid; i < nvec; i += kThreads) {
      float xv[W], tv[W];
      Vec<T>::load(xr + c0 + i * W, xv);
      Vec<T>::load(tr + c0 + i * W, tv);
      st.add(xv, tv);
    }
    cs = c0 + nvec * W;
  }
  for (int c = cs + tid; c < c1; c += kThreads) {
    const float xv[1] = {(float)xr[c]}, tv[1] = {(float)tr[c]};
    st.add(xv, tv);
  }
  // wave, then workgroup (fixed order)
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) st.merge(st.shfl_xor(m));
  __shared__ float wst[kThreads / 64][5];
  if ((tid & 63) == 0) {
    float *o = wst[tid >> 6];
    o[0] = st.mx;
    o[1] = st.dx;
    o[2] = st.mt;
    o[3] = st.dt;
    o[4] = st.s;
  }
  __syncthreads();
  if (tid == 0) {
    Stats acc;
#pragma unroll
    for (int w = 0; w < kThreads / 64; ++w) {
      Stats o;
      o.mx = wst[w][0];
      o.dx = wst[w][1];
      o.mt = wst[w][2];
      o.dt = wst[w][3];
      o.s = wst[w][4];
      acc.merge(o);
    }
    float *o = part + (int64_t)blockIdx.x * 5;
    o[0] = acc.mx;
    o[1] = acc.dx;
    o[2] = acc.mt;
    o[3] = acc.dt;
    o[4] = acc.s;
  }
}

__global__ __launch_bounds__(kThreads) void soft_ce_combine_kernel(const float *__restrict__ part, int32_t N,
                                                                 int32_t nsplit, float *__restrict__ loss,
                                                                 float *__restrict__ stats) {
  const int row = blockIdx.x * kThreads + threadIdx.x;
  if (row >= N) return;
  Stats acc;
  for (int sp = 0; sp < nsplit; ++sp) {
    const float *p = part + ((int64_t)row * nsplit + sp) * 5;
    Stats o;
    o.mx = p[0];
    o.dx = p[1];
    o.mt = p[2];
    o.dt = p[3];
    o.s = p[4];
    acc.merge(o);
  }
  const float dx = fmaxf(acc.dx, kClamp), dt = fmaxf(acc.dt, kClamp);
  loss[row] = -(acc.s / dt) + acc.mx + logf(dx);
  stats[row] = acc.mx;
  stats[N + row] = dx;
  stats[2 * N + row] = acc.mt;
  stats[3 * N + row] = dt;
}

template <typename T, bool VEC>
__global__ __launch_bounds__(kThreads) void soft_ce_bwd_kernel(const T *__restrict__ x, int64_t xs,
                                                             const T *__restrict__ t, int64_t ts, int32_t V,
                                                             int32_t chunk, int32_t nsplit, int32_t N,
                                                             const float *__restrict__ grad_out,
                                                             const float *__restrict__ stats,
                                                             T *__restrict__ g, int64_t gs) {
  const int tid = threadIdx.x;
  const int row = blockIdx.x / nsplit, sp = blockIdx.x - row * nsplit;
  const int c0 = sp * chunk, c1 = min(V, c0 + chunk);
  const T *xr = x + (int64_t)row * xs;
  const T *tr = t + (int64_t)row * ts;
  T *gr = g + (int64_t)row * gs;
  const float go = *grad_out;
  const float mxl = stats[row] * kL2E, mtl = stats[2 * N + row] * kL2E;
  // saved values are clamped already; clamping again matches loss.py:203-205
  const float ax = go / fmaxf(stats[N + row], kClamp), at = go / fmaxf(stats[3 * N + row], kClamp);
  int cs = c0;
  if constexpr (VEC) {
    constexpr int W = Vec<T>::W;
    const int nvec = (c1 - c0) / W;
    for (int i = tid; i < nvec; i += kThreads) {
      float xv[W], tv[W], gv[W];
      Vec<T>::load(xr + c0 + i * W, xv);
      Vec<T>::load(tr + c0 + i * W, tv);
#pragma unroll
      for (int e = 0; e < W; ++e)
        gv[e] = ax * ex2(__builtin_fmaf(xv[e], kL2E, -mxl)) - at * ex2(__builtin_fmaf(tv[e], kL2E, -mtl));
      Vec<T>::store(gr + c0 + i * W, gv);
    }
    cs = c0 + nvec * W;
  }
  for (int c = cs + tid; c < c1; c += kThreads) {
    const float xv = (float)xr[c], tv = (float)tr[c];
    gr[c] = (T)(ax * ex2(__builtin_fmaf(xv, kL2E, -mxl)) - at * ex2(__builtin_fmaf(tv, kL2E, -mtl)));
  }
}

// Column split of the rows: enough workgroups to fill the chip (about 1024),
// each over a multiple of kChunkQuantum columns.
void soft_ce_plan(int32_t N, int32_t V, int32_t *nsplit, int32_t *chunk) {
  const int64_t want = (1024 + N - 1) / N;
  const int64_t maxs = (V + 4095) / 4096;
  int64_t s = want < maxs ? want : maxs;
  if (s < 1) s = 1;
  int64_t c = (V + s - 1) / s;
  c = (c + kChunkQuantum - 1) / kChunkQuantum * kChunkQuantum;
  *chunk = (int32_t)c;
  *nsplit = (int32_t)((V + c - 1) / c);
}

int64_t soft_ce_workspace_floats(int32_t N, int32_t V) {
  int32_t ns, ch;
  soft_ce_plan(N, V, &ns, &ch);
  return (int64_t)N * ns * 5;
}

template <typename T>
static void fwd_typed(const void *x, int64_t xs, const void *t, int64_t ts, int32_t N, int32_t V, bool vec,
                      float *loss, float *stats, float *ws, hipStream_t st) {
  int32_t ns, ch;
  soft_ce_plan(N, V, &ns, &ch);
  const dim3 grid((unsigned)((int64_t)N * ns));
  if (vec)
    hipLaunchKernelGGL((soft_ce_partial_kernel<T, true>), grid, dim3(kThreads), 0, st, (const T *)x, xs,
                       (const T *)t, ts, V, ch, ns, ws);
  else
    hipLaunchKernelGGL((soft_ce_partial_kernel<T, false>), grid, dim3(kThreads), 0, st, (const T *)x, xs,
                       (const T *)t, ts, V, ch, ns, ws);
  hipLaunchKernelGGL(soft_ce_combine_kernel, dim3((N + kThreads - 1) / kThreads), dim3(kThreads), 0, st, ws, N,
                     ns, loss, stats);
}

template <typename T>
static void bwd_typed(const void *x, int64_t xs, const void *t, int64_t ts, int32_t N, int32_t V, bool vec,
                      const float *go, const float *stats, void *g, int64_t gs, hipStream_t st) {
  int32_t ns, ch;
  soft_ce_plan(N, V, &ns, &ch);
  const dim3 grid((unsigned)((int64_t)N * ns));
  if (vec)
    hipLaunchKernelGGL((soft_ce_bwd_kernel<T, true>), grid, dim3(kThreads), 0, st, (const T *)x, xs, (const T *)t,
                       ts, V, ch, ns, N, go, stats, (T *)g, gs);
  else
    hipLaunchKernelGGL((soft_ce_bwd_kernel<T, false>), grid, dim3(kThreads), 0, st, (const T *)x, xs,
                       (const T *)t, ts, V, ch, ns, N, go, stats, (T *)g, gs);
}

void launch_soft_ce_fwd(const void *x, int64_t xs, const void *t, int64_t ts, int32_t N, int32_t V, int dtype,
                        bool vec, float *loss, float *stats, float *ws, hipStream_t st) {
  if (dtype == kDtF32) fwd_typed<float>(x, xs, t, ts, N, V, vec, loss, stats, ws, st);
  else if (dtype == kDtF16) fwd_typed<f16_t>(x, xs, t, ts, N, V, vec, loss, stats, ws, st);
  else fwd_typed<bf16_t>(x, xs, t, ts, N, V, vec, loss, stats, ws, st);
}

void launch_soft_ce_bwd(const void *x, int64_t xs, const void *t, int64_t ts, int32_t N, int32_t V, int dtype,
                        bool vec, const float *go, const float *stats, void *g, int64_t gs, hipStream_t st) {
  if (dtype == kDtF32) bwd_typed<float>(x, xs, t, ts, N, V, vec, go, stats, g, gs, st);
  else if (dtype == kDtF16) bwd_typed<f16_t>(x, xs, t, ts, N, V, vec, go, stats, g, gs, st);
  else bwd_typed<bf16_t>(x, xs, t, ts, N, V, vec, go, stats, g, gs, st);
}

}  // namespace mga
