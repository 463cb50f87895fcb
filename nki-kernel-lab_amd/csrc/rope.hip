// Rotary position embedding (RoPE), rotate-half layout.
//
// Not in the reference: its README lists rotary embeddings among the features
// it does not implement (README.md:89).  This is the published method (Su et
// al., "RoFormer", 2021) in the layout GPT-NeoX and Llama use: the head dim
// splits into halves, and element i < d/2 rotates with element i + d/2 by the
// angle (pos0 + s) * base^(-2 i / d) of row s:
//
//   y[i]       = x[i] cos(a) - x[i + d/2] sin(a)
//   y[i + d/2] = x[i + d/2] cos(a) + x[i] sin(a)
//
// The angle, its sine and cosine and both products are fp32; each output is
// rounded once.  HBM-bound: every element is read and written once; one
// thread rotates one pair, consecutive threads take consecutive i, so each
// half-row is read and written as contiguous bytes.  y may alias x.
#include <math.h>

#include "common.h"

namespace nkl {

template <typename T>
__global__ __launch_bounds__(256) void rope_kernel(const T* x, T* y, int H, int S, int half, long x_sh, long x_ss,
                                                   long y_sh, long y_ss, int pos0, float neg_log2_base_over_half) {
  const long t = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const long pairs = (long)H * S * half;
  if (t >= pairs) return;
  const int i = (int)(t % half);
  const long rs = t / half;
  const int s = (int)(rs % S), h = (int)(rs / S);
  // base^(-2 i / d) = 2^(-(i / (d / 2)) log2(base))
  const float inv_freq = exp2f((float)i * neg_log2_base_over_half);
  const float a = (float)(pos0 + s) * inv_freq;
  float sn, cs;
  sincosf(a, &sn, &cs);
  const T* xr = x + (long)h * x_sh + (long)s * x_ss;
  T* yr = y + (long)h * y_sh + (long)s * y_ss;
  const float x1 = to_f32(xr[i]), x2 = to_f32(xr[i + half]);
  yr[i] = from_f32<T>(x1 * cs - x2 * sn);
  yr[i + half] = from_f32<T>(x2 * cs + x1 * sn);
}

template <typename T>
static int rope_launch(const void* x, void* y, int H, int S, int d, long x_sh, long x_ss, long y_sh, long y_ss,
                       int pos0, float base, hipStream_t st) {
  const int half = d / 2;
  const long pairs = (long)H * S * half;
  const float k = -log2f(base) / (float)half;
  rope_kernel<T><<<dim3((unsigned)((pairs + 255) / 256)), dim3(256), 0, st>>>(
      static_cast<const T*>(x), static_cast<T*>(y), H, S, half, x_sh, x_ss, y_sh, y_ss, pos0, k);
  return check_launch("nkl_rope");
}

}  // namespace nkl

using namespace nkl;

extern "C" int nkl_rope(const void* x, void* y, int H, int S, int d, long x_sh, long x_ss, long y_sh, long y_ss,
                        int pos0, float base, int dtype, void* stream) {
  if (H < 0 || S < 0 || d < 0) return set_error(NKL_EINVAL, "nkl_rope: negative shape H=%d S=%d d=%d", H, S, d);
  if (d % 2 != 0) return set_error(NKL_EINVAL, "nkl_rope: head dim d=%d must be even", d);
  if (pos0 < 0 || (long)pos0 + S > (1L << 24))
    return set_error(NKL_EINVAL, "nkl_rope: positions [%d, %ld) outside [0, 2^24)", pos0, (long)pos0 + S);
  if (!(base > 1.0f) || !isfinite(base)) return set_error(NKL_EINVAL, "nkl_rope: base %g must be finite and > 1", base);
  if (dtype != NKL_F32 && dtype != NKL_BF16 && dtype != NKL_F16)
    return set_error(NKL_EDTYPE, "nkl_rope: unsupported dtype %d", dtype);
  if (x_ss < d || y_ss < d) return set_error(NKL_EINVAL, "nkl_rope: row stride below d");
  if ((long)H * S * (d / 2) >= (1L << 31) * 256L) return set_error(NKL_EINVAL, "nkl_rope: tensor too large");
  if (H == 0 || S == 0 || d == 0) return NKL_OK;
  if (!x || !y) return set_error(NKL_EINVAL, "nkl_rope: null pointer");
  hipStream_t st = (hipStream_t)stream;
  if (dtype == NKL_F32) return rope_launch<float>(x, y, H, S, d, x_sh, x_ss, y_sh, y_ss, pos0, base, st);
  if (dtype == NKL_F16) return rope_launch<f16>(x, y, H, S, d, x_sh, x_ss, y_sh, y_ss, pos0, base, st);
  return rope_launch<bf16>(x, y, H, S, d, x_sh, x_ss, y_sh, y_ss, pos0, base, st);
}
