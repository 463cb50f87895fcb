// Row-wise kernels: fused softmax, three-pass softmax, RMSNorm, SwiGLU.
//
// These are HBM-bound: every input byte is read once and every output byte
// written once (the three-pass softmax deliberately round-trips its fp32
// intermediates through HBM, as the reference's unfused kernel does).
//
// Outputs are written with non-temporal (streaming) stores, which reach HBM
// faster than write-back stores for data the kernel never reads again.
//
// Layout: one 64-lane wavefront owns one row; a 256-thread workgroup owns 4
// rows.  Each lane keeps NV 16-byte vectors of its row in registers, so a row
// is read from HBM exactly once and the reductions are wavefront shuffles.
// Rows too long for the register cache, or not 16-byte aligned, take the
// looped kernels, which re-read the row (from L2) once per pass.
#include <math.h>

#include "common.h"

namespace nkl {

constexpr int kRowsPerBlock = 4;

// ------------------------------------------------------------- softmax --
// nkilab/kernels/norm.py:65-89: neg_max = -max(x); e = exp(x + neg_max) with
// the row sum in fp32; rinv = 1 / sum; y = e * rinv rounded once.
template <typename T, int NV>
__global__ __launch_bounds__(256) void softmax_vec_kernel(const T* __restrict__ x, T* __restrict__ y,
                                                          int rows, int cols, long ldx, long ldy) {
  constexpr int E = VecE<T>::value;
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= rows) return;
  const T* xr = x + (long)row * ldx;
  T* yr = y + (long)row * ldy;
  const int nvec = cols / E;
  float v[NV][E];
  float mx = -INFINITY;
#pragma unroll
  for (int n = 0; n < NV; ++n) {
    const int vi = n * kWave + lane;
    if (vi < nvec) {
      load16(xr + (long)vi * E, v[n]);
    } else {
#pragma unroll
      for (int e = 0; e < E; ++e) v[n][e] = -INFINITY;
    }
#pragma unroll
    for (int e = 0; e < E; ++e) mx = fmaxf(mx, v[n][e]);
  }
  mx = wave_max(mx);
  const float mx2 = mx * kLog2e;
  float sum = 0.f;
#pragma unroll
  for (int n = 0; n < NV; ++n)
#pragma unroll
    for (int e = 0; e < E; ++e) {
      v[n][e] = fast_exp2(fmaf(v[n][e], kLog2e, -mx2));
      sum += v[n][e];
    }
  sum = wave_sum(sum);
  const float rinv = 1.0f / sum;
#pragma unroll
  for (int n = 0; n < NV; ++n) {
    const int vi = n * kWave + lane;
    if (vi < nvec) {
      float o[E];
#pragma unroll
      for (int e = 0; e < E; ++e) o[e] = v[n][e] * rinv;
      store_vec_nt<E>(yr + (long)vi * E, o);
    }
  }
}

// Any length / alignment: one wavefront per row, three sweeps over the row.
template <typename T>
__global__ __launch_bounds__(256) void softmax_loop_kernel(const T* __restrict__ x, T* __restrict__ y,
                                                           int rows, int cols, long ldx, long ldy) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= rows) return;
  const T* xr = x + (long)row * ldx;
  T* yr = y + (long)row * ldy;
  float mx = -INFINITY;
  for (int c = lane; c < cols; c += kWave) mx = fmaxf(mx, to_f32(xr[c]));
  mx = wave_max(mx);
  const float mx2 = mx * kLog2e;
  float sum = 0.f;
  for (int c = lane; c < cols; c += kWave) sum += fast_exp2(fmaf(to_f32(xr[c]), kLog2e, -mx2));
  sum = wave_sum(sum);
  const float rinv = 1.0f / sum;
  for (int c = lane; c < cols; c += kWave)
    yr[c] = from_f32<T>(fast_exp2(fmaf(to_f32(xr[c]), kLog2e, -mx2)) * rinv);
}

// ---------------------------------------------------- three-pass softmax --
// nkilab/kernels/norm.py:22-62.  Pass 1: m = max(x) -> HBM.  Pass 2:
// e = exp(x - m) (fp32, -> HBM) and s = sum(e) -> HBM.  Pass 3: y = e / s.
template <typename T>
__global__ __launch_bounds__(256) void softmax_pass1_kernel(const T* __restrict__ x, float* __restrict__ m,
                                                            int rows, int cols, long ldx) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= rows) return;
  const T* xr = x + (long)row * ldx;
  float mx = -INFINITY;
  for (int c = lane; c < cols; c += kWave) mx = fmaxf(mx, to_f32(xr[c]));
  mx = wave_max(mx);
  if (lane == 0) m[row] = mx;
}

template <typename T>
__global__ __launch_bounds__(256) void softmax_pass2_kernel(const T* __restrict__ x, const float* __restrict__ m,
                                                            float* __restrict__ e, float* __restrict__ s,
                                                            int rows, int cols, long ldx) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= rows) return;
  const T* xr = x + (long)row * ldx;
  float* er = e + (long)row * cols;
  const float mr = m[row];
  float sum = 0.f;
  for (int c = lane; c < cols; c += kWave) {
    const float t = fast_exp2((to_f32(xr[c]) - mr) * kLog2e);
    er[c] = t;
    sum += t;
  }
  sum = wave_sum(sum);
  if (lane == 0) s[row] = sum;
}

template <typename T>
__global__ __launch_bounds__(256) void softmax_pass3_kernel(const float* __restrict__ e, const float* __restrict__ s,
                                                            T* __restrict__ y, int rows, int cols, long ldy) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= rows) return;
  const float* er = e + (long)row * cols;
  T* yr = y + (long)row * ldy;
  const float sr = s[row];
  for (int c = lane; c < cols; c += kWave) yr[c] = from_f32<T>(er[c] / sr);
}

// ------------------------------------------------------------- RMSNorm --
// nkilab/kernels/norm.py:92-118: ssq = sum(x^2) (fp32); ms = ssq * (1/D) + eps;
// rstd = rsqrt(ms); xn = x * rstd (fp32); y = xn * w rounded once.
// E weight elements of type TW (16-byte aligned) as fp32 values.
template <int E>
__device__ __forceinline__ void load_w(const float* p, float (&v)[E]) {
#pragma unroll
  for (int i = 0; i < E; i += 4) {
    float t[4];
    load16(p + i, t);
#pragma unroll
    for (int k = 0; k < 4; ++k) v[i + k] = t[k];
  }
}
template <int E>
__device__ __forceinline__ void load_w(const bf16* p, float (&v)[E]) {
  if constexpr (E == 8) {
    load16(p, v);
  } else {
    static_assert(E == 4, "4 or 8 weights per vector");
    const uint2 t = *reinterpret_cast<const uint2*>(p);
    v[0] = bf16lo(t.x), v[1] = bf16hi(t.x), v[2] = bf16lo(t.y), v[3] = bf16hi(t.y);
  }
}

template <typename TI, typename TW, typename TO, int NV>
__global__ __launch_bounds__(256) void rmsnorm_vec_kernel(const TI* __restrict__ x, const TW* __restrict__ w,
                                                          TO* __restrict__ y, int rows, int cols, long ldx,
                                                          long ldy, float inv_d, float eps) {
  constexpr int E = VecE<TI>::value;
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= rows) return;
  const TI* xr = x + (long)row * ldx;
  TO* yr = y + (long)row * ldy;
  const int nvec = cols / E;
  float v[NV][E];
  float ssq = 0.f;
#pragma unroll
  for (int n = 0; n < NV; ++n) {
    const int vi = n * kWave + lane;
    if (vi < nvec) {
      load16(xr + (long)vi * E, v[n]);
    } else {
#pragma unroll
      for (int e = 0; e < E; ++e) v[n][e] = 0.f;
    }
#pragma unroll
    for (int e = 0; e < E; ++e) ssq = fmaf(v[n][e], v[n][e], ssq);
  }
  ssq = wave_sum(ssq);
  const float rstd = __frsqrt_rn(fmaf(ssq, inv_d, eps));
#pragma unroll
  for (int n = 0; n < NV; ++n) {
    const int vi = n * kWave + lane;
    if (vi < nvec) {
      float wv[E];
      load_w<E>(w + (long)vi * E, wv);
      float o[E];
#pragma unroll
      for (int e = 0; e < E; ++e) o[e] = (v[n][e] * rstd) * wv[e];
      store_vec_nt<E>(yr + (long)vi * E, o);
    }
  }
}

template <typename TI, typename TW, typename TO>
__global__ __launch_bounds__(256) void rmsnorm_loop_kernel(const TI* __restrict__ x, const TW* __restrict__ w,
                                                           TO* __restrict__ y, int rows, int cols, long ldx,
                                                           long ldy, float inv_d, float eps) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= rows) return;
  const TI* xr = x + (long)row * ldx;
  TO* yr = y + (long)row * ldy;
  float ssq = 0.f;
  for (int c = lane; c < cols; c += kWave) {
    const float t = to_f32(xr[c]);
    ssq = fmaf(t, t, ssq);
  }
  ssq = wave_sum(ssq);
  const float rstd = __frsqrt_rn(fmaf(ssq, inv_d, eps));
  for (int c = lane; c < cols; c += kWave) yr[c] = from_f32<TO>((to_f32(xr[c]) * rstd) * to_f32(w[c]));
}

// -------------------------------------------------------------- SwiGLU --
// nkilab/kernels/norm.py:121-136: a = silu(g) in fp32; y = a * u rounded once
// (silu is in common.h, shared with the GEMM's gate/up epilogue).

// Each thread handles UNROLL 16-byte vectors spaced a grid-width apart.
template <typename T, int UNROLL>
__global__ __launch_bounds__(256) void swiglu_vec_kernel(const T* __restrict__ g, const T* __restrict__ u,
                                                         T* __restrict__ y, long nvec) {
  constexpr int E = VecE<T>::value;
  const long stride = (long)gridDim.x * blockDim.x;
  const long base = (long)blockIdx.x * blockDim.x + threadIdx.x;
  float gv[UNROLL][E], uv[UNROLL][E];
#pragma unroll
  for (int r = 0; r < UNROLL; ++r) {
    const long vi = base + r * stride;
    if (vi < nvec) {
      load16(g + vi * E, gv[r]);
      load16(u + vi * E, uv[r]);
    }
  }
#pragma unroll
  for (int r = 0; r < UNROLL; ++r) {
    const long vi = base + r * stride;
    if (vi < nvec) {
      float o[E];
#pragma unroll
      for (int e = 0; e < E; ++e) o[e] = silu(gv[r][e]) * uv[r][e];
      store_vec_nt<E>(y + vi * E, o);
    }
  }
}

template <typename T>
__global__ __launch_bounds__(256) void swiglu_tail_kernel(const T* __restrict__ g, const T* __restrict__ u,
                                                          T* __restrict__ y, long start, long n) {
  const long i = start + (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) y[i] = from_f32<T>(silu(to_f32(g[i])) * to_f32(u[i]));
}

// ------------------------------------------------------------ dispatch --
static bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// Smallest register-cache depth (vectors per lane) that holds a row of nvec
// 16-byte vectors; 0 when the row is longer than the deepest variant.
static int pick_nv(int nvec) {
  for (int nv = 1; nv <= 16; nv *= 2)
    if (nvec <= nv * kWave) return nv;
  return 0;
}

template <typename T>
static int softmax_launch(const void* x, void* y, int rows, int cols, long ldx, long ldy, hipStream_t st) {
  constexpr int E = VecE<T>::value;
  const dim3 grid((rows + kRowsPerBlock - 1) / kRowsPerBlock), block(256);
  const T* xp = static_cast<const T*>(x);
  T* yp = static_cast<T*>(y);
  const bool vec = cols % E == 0 && ldx % E == 0 && ldy % E == 0 && aligned16(x) && aligned16(y);
  const int nv = vec ? pick_nv(cols / E) : 0;
  switch (nv) {
    case 1: softmax_vec_kernel<T, 1><<<grid, block, 0, st>>>(xp, yp, rows, cols, ldx, ldy); break;
    case 2: softmax_vec_kernel<T, 2><<<grid, block, 0, st>>>(xp, yp, rows, cols, ldx, ldy); break;
    case 4: softmax_vec_kernel<T, 4><<<grid, block, 0, st>>>(xp, yp, rows, cols, ldx, ldy); break;
    case 8: softmax_vec_kernel<T, 8><<<grid, block, 0, st>>>(xp, yp, rows, cols, ldx, ldy); break;
    case 16: softmax_vec_kernel<T, 16><<<grid, block, 0, st>>>(xp, yp, rows, cols, ldx, ldy); break;
    default: softmax_loop_kernel<T><<<grid, block, 0, st>>>(xp, yp, rows, cols, ldx, ldy); break;
  }
  return check_launch("nkl_softmax");
}

template <typename TI, typename TW, typename TO>
static int rmsnorm_launch(const void* x, const void* w, void* y, int rows, int cols, long ldx, long ldy,
                          float eps, hipStream_t st) {
  constexpr int E = VecE<TI>::value;
  const dim3 grid((rows + kRowsPerBlock - 1) / kRowsPerBlock), block(256);
  const TI* xp = static_cast<const TI*>(x);
  const TW* wp = static_cast<const TW*>(w);
  TO* yp = static_cast<TO*>(y);
  // The multiplier 1/D is the fp32 value nearest the exact quotient.
  const float inv_d = (float)(1.0 / (double)cols);
  const bool out_vec = (E * sizeof(TO)) % 8 == 0;
  const bool vec = out_vec && cols % E == 0 && ldx % E == 0 && ldy % E == 0 && aligned16(x) &&
                   aligned16(w) && aligned16(y);
  const int nv = vec ? pick_nv(cols / E) : 0;
  switch (nv) {
    case 1: rmsnorm_vec_kernel<TI, TW, TO, 1><<<grid, block, 0, st>>>(xp, wp, yp, rows, cols, ldx, ldy, inv_d, eps); break;
    case 2: rmsnorm_vec_kernel<TI, TW, TO, 2><<<grid, block, 0, st>>>(xp, wp, yp, rows, cols, ldx, ldy, inv_d, eps); break;
    case 4: rmsnorm_vec_kernel<TI, TW, TO, 4><<<grid, block, 0, st>>>(xp, wp, yp, rows, cols, ldx, ldy, inv_d, eps); break;
    case 8: rmsnorm_vec_kernel<TI, TW, TO, 8><<<grid, block, 0, st>>>(xp, wp, yp, rows, cols, ldx, ldy, inv_d, eps); break;
    case 16: rmsnorm_vec_kernel<TI, TW, TO, 16><<<grid, block, 0, st>>>(xp, wp, yp, rows, cols, ldx, ldy, inv_d, eps); break;
    default: rmsnorm_loop_kernel<TI, TW, TO><<<grid, block, 0, st>>>(xp, wp, yp, rows, cols, ldx, ldy, inv_d, eps); break;
  }
  return check_launch("nkl_rmsnorm");
}

template <typename T>
static int swiglu_launch(const void* g, const void* u, void* y, long n, hipStream_t st) {
  constexpr int E = VecE<T>::value;
  // Two vectors of each input per thread.  In bench.py's harness at 4096 x
  // 2048 bf16 one per thread was no faster (10.8 against 10.7 us), four
  // slower, and per-workgroup contiguous chunks (with or without an
  // XCD-aware order) slower still.
  constexpr int UNROLL = 2;
  const T* gp = static_cast<const T*>(g);
  const T* up = static_cast<const T*>(u);
  T* yp = static_cast<T*>(y);
  long done = 0;
  if (aligned16(g) && aligned16(u) && aligned16(y)) {
    const long nvec = n / E;
    if (nvec > 0) {
      const long threads = (nvec + UNROLL - 1) / UNROLL;
      const long blocks = (threads + 255) / 256;
      swiglu_vec_kernel<T, UNROLL><<<dim3((unsigned)blocks), dim3(256), 0, st>>>(gp, up, yp, nvec);
    }
    done = nvec * E;
  }
  if (done < n) {
    const long rem = n - done;
    swiglu_tail_kernel<T><<<dim3((unsigned)((rem + 255) / 256)), dim3(256), 0, st>>>(gp, up, yp, done, n);
  }
  return check_launch("nkl_swiglu");
}

// Streaming copy with the row kernels' loads and non-temporal stores and none
// of their arithmetic: each lane reads kCopyUnroll 16-byte chunks one grid
// span apart, then writes them.  Two per lane is the fastest of 1, 2, 4 and 8
// (and of per-workgroup contiguous chunks) at 16 - 128 MiB on MI355X.  It
// measures the HBM ceiling the row kernels' roofline is read against at the
// same size.
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
constexpr int kCopyUnroll = 2;
__global__ __launch_bounds__(256) void stream_copy_kernel(const u32x4* __restrict__ x, u32x4* __restrict__ y, long n) {
  const long base = (long)blockIdx.x * 256 + threadIdx.x, span = (long)gridDim.x * 256;
  u32x4 v[kCopyUnroll];
#pragma unroll
  for (int k = 0; k < kCopyUnroll; ++k) {
    const long i = base + k * span;
    v[k] = i < n ? x[i] : u32x4{0u, 0u, 0u, 0u};
  }
#pragma unroll
  for (int k = 0; k < kCopyUnroll; ++k) {
    const long i = base + k * span;
    if (i < n) __builtin_nontemporal_store(v[k], y + i);
  }
}

// ------------------------------------------------------ hi/lo bf16 split --
// y[r, c] = bf16(x[r, c]) and y[r, cols + c] = bf16(x[r, c] - bf16(x[r, c])):
// an fp32 activation as two bf16 values whose sum carries 16 significand
// bits.  A GEMM over [hi | lo] (K doubled) against a bf16 weight stacked
// twice along K then accumulates x . w in fp32 to about 2^-17 of x: the
// decoder block runs its projections on bf16 MFMA at fp32 accuracy.
// One thread per 4 consecutive columns of a row (cols % 4 == 0, aligned rows).
__global__ __launch_bounds__(256) void split_bf16_kernel(const float* __restrict__ x, bf16* __restrict__ y, int rows,
                                                         int cols, long ldx, long ldy) {
  const int q = cols / 4;
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= (long)rows * q) return;
  const int r = (int)(i / q), c = 4 * (int)(i % q);
  float v[4];
  load16(x + (long)r * ldx + c, v);
  float hi[4], lo[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    hi[e] = (float)(bf16)v[e];
    lo[e] = v[e] - hi[e];  // exact in fp32
  }
  store_vec<4>(y + (long)r * ldy + c, hi);
  store_vec<4>(y + (long)r * ldy + cols + c, lo);
}

}  // namespace nkl

using namespace nkl;

static int check_rows(const char* fn, int rows, int cols, long ldx, long ldy) {
  if (rows < 0 || cols < 0) return set_error(NKL_EINVAL, "%s: negative shape (%d, %d)", fn, rows, cols);
  if (rows > 0 && cols > 0 && (ldx < cols || ldy < cols))
    return set_error(NKL_EINVAL, "%s: leading dimension (%ld, %ld) smaller than cols %d", fn, ldx, ldy, cols);
  return NKL_OK;
}

extern "C" int nkl_softmax(const void* x, void* y, int rows, int cols, long ldx, long ldy, int dtype,
                           void* stream) {
  int rc = check_rows("nkl_softmax", rows, cols, ldx, ldy);
  if (rc) return rc;
  if (rows == 0 || cols == 0) return NKL_OK;
  hipStream_t st = (hipStream_t)stream;
  if (dtype == NKL_F32) return softmax_launch<float>(x, y, rows, cols, ldx, ldy, st);
  if (dtype == NKL_BF16) return softmax_launch<bf16>(x, y, rows, cols, ldx, ldy, st);
  return set_error(NKL_EDTYPE, "nkl_softmax: unsupported dtype %d", dtype);
}

extern "C" size_t nkl_softmax_unfused_workspace_bytes(int rows, int cols) {
  if (rows <= 0 || cols <= 0) return 0;
  const size_t r = ((size_t)rows * 4 + 255) / 256 * 256;
  return 2 * r + (size_t)rows * (size_t)cols * 4;
}

extern "C" int nkl_softmax_unfused(const void* x, void* y, void* workspace, size_t workspace_bytes, int rows,
                                   int cols, long ldx, long ldy, int dtype, void* stream) {
  int rc = check_rows("nkl_softmax_unfused", rows, cols, ldx, ldy);
  if (rc) return rc;
  if (rows == 0 || cols == 0) return NKL_OK;
  const size_t need = nkl_softmax_unfused_workspace_bytes(rows, cols);
  if (!workspace || workspace_bytes < need)
    return set_error(NKL_EWORKSPACE, "nkl_softmax_unfused: workspace of %zu bytes needed, %zu given", need,
                     workspace_bytes);
  const size_t r = ((size_t)rows * 4 + 255) / 256 * 256;
  float* m = static_cast<float*>(workspace);
  float* s = reinterpret_cast<float*>(static_cast<char*>(workspace) + r);
  float* e = reinterpret_cast<float*>(static_cast<char*>(workspace) + 2 * r);
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid((rows + kRowsPerBlock - 1) / kRowsPerBlock), block(256);
  if (dtype == NKL_F32) {
    softmax_pass1_kernel<float><<<grid, block, 0, st>>>(static_cast<const float*>(x), m, rows, cols, ldx);
    softmax_pass2_kernel<float><<<grid, block, 0, st>>>(static_cast<const float*>(x), m, e, s, rows, cols, ldx);
    softmax_pass3_kernel<float><<<grid, block, 0, st>>>(e, s, static_cast<float*>(y), rows, cols, ldy);
  } else if (dtype == NKL_BF16) {
    softmax_pass1_kernel<bf16><<<grid, block, 0, st>>>(static_cast<const bf16*>(x), m, rows, cols, ldx);
    softmax_pass2_kernel<bf16><<<grid, block, 0, st>>>(static_cast<const bf16*>(x), m, e, s, rows, cols, ldx);
    softmax_pass3_kernel<bf16><<<grid, block, 0, st>>>(e, s, static_cast<bf16*>(y), rows, cols, ldy);
  } else {
    return set_error(NKL_EDTYPE, "nkl_softmax_unfused: unsupported dtype %d", dtype);
  }
  return check_launch("nkl_softmax_unfused");
}

extern "C" int nkl_rmsnorm_ex(const void* x, const void* w, void* y, int rows, int cols, long ldx, long ldy,
                              float eps, int dtype_in, int dtype_w, int dtype_out, void* stream) {
  int rc = check_rows("nkl_rmsnorm", rows, cols, ldx, ldy);
  if (rc) return rc;
  if (rows == 0 || cols == 0) return NKL_OK;
  if (dtype_w != NKL_F32 && dtype_w != NKL_BF16)
    return set_error(NKL_EDTYPE, "nkl_rmsnorm: unsupported weight dtype %d", dtype_w);
  hipStream_t st = (hipStream_t)stream;
  const bool wf = dtype_w == NKL_F32;
  if (dtype_in == NKL_F32 && dtype_out == NKL_F32)
    return wf ? rmsnorm_launch<float, float, float>(x, w, y, rows, cols, ldx, ldy, eps, st)
              : rmsnorm_launch<float, bf16, float>(x, w, y, rows, cols, ldx, ldy, eps, st);
  if (dtype_in == NKL_BF16 && dtype_out == NKL_BF16)
    return wf ? rmsnorm_launch<bf16, float, bf16>(x, w, y, rows, cols, ldx, ldy, eps, st)
              : rmsnorm_launch<bf16, bf16, bf16>(x, w, y, rows, cols, ldx, ldy, eps, st);
  if (dtype_in == NKL_F32 && dtype_out == NKL_BF16)
    return wf ? rmsnorm_launch<float, float, bf16>(x, w, y, rows, cols, ldx, ldy, eps, st)
              : rmsnorm_launch<float, bf16, bf16>(x, w, y, rows, cols, ldx, ldy, eps, st);
  if (dtype_in == NKL_F32 && dtype_out == NKL_F16)
    return wf ? rmsnorm_launch<float, float, f16>(x, w, y, rows, cols, ldx, ldy, eps, st)
              : rmsnorm_launch<float, bf16, f16>(x, w, y, rows, cols, ldx, ldy, eps, st);
  return set_error(NKL_EDTYPE, "nkl_rmsnorm: unsupported dtype pair (%d -> %d)", dtype_in, dtype_out);
}

extern "C" int nkl_rmsnorm(const void* x, const void* w, void* y, int rows, int cols, long ldx, long ldy,
                           float eps, int dtype_in, int dtype_out, void* stream) {
  return nkl_rmsnorm_ex(x, w, y, rows, cols, ldx, ldy, eps, dtype_in, dtype_in, dtype_out, stream);
}

extern "C" int nkl_swiglu(const void* g, const void* u, void* y, long n, int dtype, void* stream) {
  if (n < 0) return set_error(NKL_EINVAL, "nkl_swiglu: negative length %ld", n);
  if (n == 0) return NKL_OK;
  hipStream_t st = (hipStream_t)stream;
  if (dtype == NKL_F32) return swiglu_launch<float>(g, u, y, n, st);
  if (dtype == NKL_BF16) return swiglu_launch<bf16>(g, u, y, n, st);
  if (dtype == NKL_F16) return swiglu_launch<f16>(g, u, y, n, st);
  return set_error(NKL_EDTYPE, "nkl_swiglu: unsupported dtype %d", dtype);
}

extern "C" int nkl_stream_copy(const void* x, void* y, long nbytes, void* stream) {
  if (nbytes < 0 || nbytes % 16 != 0)
    return set_error(NKL_EINVAL, "nkl_stream_copy: %ld bytes is not a non-negative multiple of 16", nbytes);
  if (nbytes == 0) return NKL_OK;
  if (!x || !y || ((uintptr_t)x & 15u) || ((uintptr_t)y & 15u))
    return set_error(NKL_EINVAL, "nkl_stream_copy: null or non-16-byte-aligned pointer");
  const long n = nbytes / 16;
  const long grid = (n + kCopyUnroll * 256 - 1) / (kCopyUnroll * 256);
  if (grid > 0x7fffffffL) return set_error(NKL_EINVAL, "nkl_stream_copy: %ld bytes is too large", nbytes);
  stream_copy_kernel<<<dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream>>>(static_cast<const u32x4*>(x),
                                                                                   static_cast<u32x4*>(y), n);
  return check_launch("nkl_stream_copy");
}

extern "C" int nkl_split_bf16(const void* x, void* y, int rows, int cols, long ldx, long ldy, void* stream) {
  if (rows < 0 || cols < 0) return set_error(NKL_EINVAL, "nkl_split_bf16: negative shape (%d, %d)", rows, cols);
  if (rows == 0 || cols == 0) return NKL_OK;
  if (cols % 4 || ldx % 4 || ldy % 4 || ldx < cols || ldy < 2L * cols || ((uintptr_t)x & 15u) || ((uintptr_t)y & 7u))
    return set_error(NKL_EINVAL,
                     "nkl_split_bf16: cols %d and leading dimensions (%ld, %ld) must be multiples of 4 with "
                     "ldx >= cols, ldy >= 2 cols; x 16-byte and y 8-byte aligned", cols, ldx, ldy);
  const long n = (long)rows * (cols / 4);
  split_bf16_kernel<<<dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream>>>(
      static_cast<const float*>(x), static_cast<bf16*>(y), rows, cols, ldx, ldy);
  return check_launch("nkl_split_bf16");
}
