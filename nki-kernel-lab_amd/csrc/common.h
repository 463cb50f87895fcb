// Shared device helpers for the gfx950 kernels: element types, 16-byte
// vector loads/stores, bf16 rounding, wavefront reductions and the MFMA
// operand traits used by the GEMM and attention kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "nkilab_hip.h"

namespace nkl {

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16;
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kWave = 64;

// ---------------------------------------------------------------- scalars --

template <typename T>
__device__ __forceinline__ float to_f32(T v);
template <>
__device__ __forceinline__ float to_f32<float>(float v) { return v; }
template <>
__device__ __forceinline__ float to_f32<bf16>(bf16 v) { return (float)v; }
template <>
__device__ __forceinline__ float to_f32<f16>(f16 v) { return (float)v; }

// fp32 -> T, round-to-nearest-even (v_cvt_pk_bf16_f32 on gfx950).
template <typename T>
__device__ __forceinline__ T from_f32(float v);
template <>
__device__ __forceinline__ float from_f32<float>(float v) { return v; }
template <>
__device__ __forceinline__ bf16 from_f32<bf16>(float v) { return (bf16)v; }
template <>
__device__ __forceinline__ f16 from_f32<f16>(float v) { return (f16)v; }

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  bf16x2 r;
  r[0] = (bf16)lo;
  r[1] = (bf16)hi;
  return __builtin_bit_cast(uint32_t, r);
}

__device__ __forceinline__ uint32_t pack_f16x2(float lo, float hi) {
  f16x2 r;
  r[0] = (f16)lo;
  r[1] = (f16)hi;
  return __builtin_bit_cast(uint32_t, r);
}

__device__ __forceinline__ float bf16lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// max / sum of x and x of lane l ^ 32, without the LDS: v_permlane32_swap
// (gfx950) exchanges lanes 32-63 of its first operand with lanes 0-31 of its
// second; with x in both, every lane ends up holding x of lanes l % 32 and
// l % 32 + 32 in the two results.  (A ds_bpermute would also wait for every
// LDS access of the wavefront still in flight.)
__device__ __forceinline__ float max_xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// ------------------------------------------------------- 16-byte vectors --
// VecE<T> = number of T elements in one 16-byte load.
template <typename T>
struct VecE { static constexpr int value = 16 / sizeof(T); };

// Load one 16-byte vector of T as fp32 values.
__device__ __forceinline__ void load16(const float* p, float (&v)[4]) {
  float4 t = *reinterpret_cast<const float4*>(p);
  v[0] = t.x; v[1] = t.y; v[2] = t.z; v[3] = t.w;
}
__device__ __forceinline__ void load16(const bf16* p, float (&v)[8]) {
  uint4 t = *reinterpret_cast<const uint4*>(p);
  v[0] = bf16lo(t.x); v[1] = bf16hi(t.x);
  v[2] = bf16lo(t.y); v[3] = bf16hi(t.y);
  v[4] = bf16lo(t.z); v[5] = bf16hi(t.z);
  v[6] = bf16lo(t.w); v[7] = bf16hi(t.w);
}

__device__ __forceinline__ void load16(const f16* p, float (&v)[8]) {
  const f16x8 t = *reinterpret_cast<const f16x8*>(p);
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = (float)t[i];
}

// Store E fp32 values as E elements of T (E * sizeof(T) bytes, aligned).
template <int E>
__device__ __forceinline__ void store_vec(float* p, const float (&v)[E]) {
#pragma unroll
  for (int i = 0; i < E; i += 4)
    *reinterpret_cast<float4*>(p + i) = make_float4(v[i], v[i + 1], v[i + 2], v[i + 3]);
}
template <int E>
__device__ __forceinline__ void store_vec(bf16* p, const float (&v)[E]) {
  static_assert(E == 4 || E == 8, "bf16 vector store of 4 or 8 elements");
  if constexpr (E == 8) {
    uint4 t;
    t.x = pack_bf16x2(v[0], v[1]);
    t.y = pack_bf16x2(v[2], v[3]);
    t.z = pack_bf16x2(v[4], v[5]);
    t.w = pack_bf16x2(v[6], v[7]);
    *reinterpret_cast<uint4*>(p) = t;
  } else {
    uint2 t;
    t.x = pack_bf16x2(v[0], v[1]);
    t.y = pack_bf16x2(v[2], v[3]);
    *reinterpret_cast<uint2*>(p) = t;
  }
}

template <int E>
__device__ __forceinline__ void store_vec(f16* p, const float (&v)[E]) {
  static_assert(E == 4 || E == 8, "fp16 vector store of 4 or 8 elements");
  if constexpr (E == 8) {
    uint4 t;
    t.x = pack_f16x2(v[0], v[1]);
    t.y = pack_f16x2(v[2], v[3]);
    t.z = pack_f16x2(v[4], v[5]);
    t.w = pack_f16x2(v[6], v[7]);
    *reinterpret_cast<uint4*>(p) = t;
  } else {
    uint2 t;
    t.x = pack_f16x2(v[0], v[1]);
    t.y = pack_f16x2(v[2], v[3]);
    *reinterpret_cast<uint2*>(p) = t;
  }
}

// Streaming (non-temporal) variant for outputs that are written once and not
// read back by the kernel: on MI355X these stores reach HBM markedly faster
// than ordinary write-back stores (4096 x 2048 bf16 softmax: 9.0 -> 6.6 us).
template <int E>
__device__ __forceinline__ void store_vec_nt(float* p, const float (&v)[E]) {
  typedef float f4 __attribute__((ext_vector_type(4)));
#pragma unroll
  for (int i = 0; i < E; i += 4) {
    const f4 t = {v[i], v[i + 1], v[i + 2], v[i + 3]};
    __builtin_nontemporal_store(t, reinterpret_cast<f4*>(p + i));
  }
}
template <int E>
__device__ __forceinline__ void store_vec_nt(bf16* p, const float (&v)[E]) {
  static_assert(E == 4 || E == 8, "bf16 vector store of 4 or 8 elements");
  typedef unsigned u4 __attribute__((ext_vector_type(4)));
  typedef unsigned u2 __attribute__((ext_vector_type(2)));
  if constexpr (E == 8) {
    const u4 t = {pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]), pack_bf16x2(v[4], v[5]), pack_bf16x2(v[6], v[7])};
    __builtin_nontemporal_store(t, reinterpret_cast<u4*>(p));
  } else {
    const u2 t = {pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
    __builtin_nontemporal_store(t, reinterpret_cast<u2*>(p));
  }
}

template <int E>
__device__ __forceinline__ void store_vec_nt(f16* p, const float (&v)[E]) {
  static_assert(E == 4 || E == 8, "fp16 vector store of 4 or 8 elements");
  typedef unsigned u4 __attribute__((ext_vector_type(4)));
  typedef unsigned u2 __attribute__((ext_vector_type(2)));
  if constexpr (E == 8) {
    const u4 t = {pack_f16x2(v[0], v[1]), pack_f16x2(v[2], v[3]), pack_f16x2(v[4], v[5]), pack_f16x2(v[6], v[7])};
    __builtin_nontemporal_store(t, reinterpret_cast<u4*>(p));
  } else {
    const u2 t = {pack_f16x2(v[0], v[1]), pack_f16x2(v[2], v[3])};
    __builtin_nontemporal_store(t, reinterpret_cast<u2*>(p));
  }
}

// ------------------------------------------------------ wave reductions --
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

// ------------------------------------------------------- MFMA operands --
// A 16x16 (M x N) MFMA with K = 4 * KPER: lane l holds
//   A[m = l % 16][k = KPER * (l / 16) + j], B[k = KPER * (l / 16) + j][n = l % 16]
// for j < KPER, and the accumulator C[4 * (l / 16) + i][l % 16], i < 4.
template <typename T>
struct Mfma16;
template <>
struct Mfma16<bf16> {
  static constexpr int KPER = 8;
  static constexpr int MK = 32;
  typedef bf16x8 frag;
  static __device__ __forceinline__ floatx4 mma(frag a, frag b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};
template <>
struct Mfma16<float> {
  static constexpr int KPER = 1;
  static constexpr int MK = 4;
  typedef float frag;
  static __device__ __forceinline__ floatx4 mma(frag a, frag b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
  }
};

// A 32x32 MFMA with K = 2 * KPER: lane l holds
//   A[m = l % 32][k = KPER * (l / 32) + j], B[k = KPER * (l / 32) + j][n = l % 32]
// and the accumulator C[8 * (i / 4) + 4 * (l / 32) + i % 4][l % 32], i < 16.
template <typename T>
struct Mfma32;
template <>
struct Mfma32<bf16> {
  static constexpr int KPER = 8;
  static constexpr int MK = 16;
  typedef bf16x8 frag;
  static __device__ __forceinline__ floatx16 mma(frag a, frag b, floatx16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};
template <>
struct Mfma32<f16> {
  static constexpr int KPER = 8;
  static constexpr int MK = 16;
  typedef f16x8 frag;
  static __device__ __forceinline__ floatx16 mma(frag a, frag b, floatx16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};
template <>
struct Mfma32<float> {
  static constexpr int KPER = 1;
  static constexpr int MK = 2;
  typedef float frag;
  static __device__ __forceinline__ floatx16 mma(frag a, frag b, floatx16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
  }
};

// A 32x32x16 MFMA on 16-bit operands held as 16-byte vectors (the bf16x8
// register type carries either format's bits): fp16 when H, else bf16.  The
// kernels that take both formats move operands as raw 16-bit values and only
// pick the instruction (and the rounding of what they produce) by H.
template <bool H>
__device__ __forceinline__ floatx16 mma32_16b(bf16x8 a, bf16x8 b, floatx16 c) {
  if constexpr (H)
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                   0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
// fp32 -> the 16-bit format (round to nearest even), as a bf16-typed value
// holding its bits.
template <bool H>
__device__ __forceinline__ bf16 round16(float x) {
  if constexpr (H)
    return __builtin_bit_cast(bf16, (f16)x);
  else
    return (bf16)x;
}

// 16-byte load of base[off] when `ok`, zeros otherwise.  The load itself is
// unconditional (from base[0] when !ok) so that the compiler never turns the
// choice into a load through a pointer to a private zero vector.
template <typename T>
__device__ __forceinline__ uint4 ld16_or_zero(const T* base, long off, bool ok) {
  const uint4 v = *reinterpret_cast<const uint4*>(base + (ok ? off : 0));
  return ok ? v : make_uint4(0, 0, 0, 0);
}

// Load KPER consecutive elements as one MFMA operand fragment.
// silu(g) = g / (1 + e^-g) in fp32 (nkilab/kernels/norm.py:121-136).
__device__ __forceinline__ float silu(float g) {
  return g * __builtin_amdgcn_rcpf(1.0f + fast_exp2(-g * kLog2e));
}

// ds_read_b64_tr_b16 through inline assembly, for kernels whose LDS is also
// filled by LDS-DMA copies.  The compiler's builtin form of this read makes it
// wait for every outstanding copy (vmcnt(0)) first, as it cannot tell the
// copies' LDS ranges from the one read, which leaves only one stage of copies
// in flight; the callers' protocols (each wavefront's vmcnt wait for its own
// copies of a stage, then a barrier) already order the two.  The compiler does
// not track this read's completion: its result goes through lds_wait_tie()
// before any use.
typedef short shortx4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ shortx4 ds_read_tr16_b64_async(const void* lds_ptr) {
  shortx4 r;
  const unsigned a = (unsigned)(size_t)(const __attribute__((address_space(3))) void*)lds_ptr;
  asm volatile("ds_read_b64_tr_b16 %0, %1" : "=v"(r) : "v"(a));
  return r;
}
// ds_read_b128 in the same untracked form (so that the compiler's lgkmcnt
// waits for its own reads do not count across untracked ones).
__device__ __forceinline__ bf16x8 ds_read_b128_async(const void* lds_ptr) {
  bf16x8 r;
  const unsigned a = (unsigned)(size_t)(const __attribute__((address_space(3))) void*)lds_ptr;
  asm volatile("ds_read_b128 %0, %1" : "=v"(r) : "v"(a));
  return r;
}
// The LDS byte address of p (a pointer into a __shared__ array), passed
// through an empty asm: the compiler loses what it was computed from (a
// wavefront-uniform value, kept in an SGPR).  Conversions between LDS
// pointers and integers stay in device functions (a kernel body with them
// lost its host launch stub).
__device__ __forceinline__ unsigned opaque_lds_addr(const void* p) {
  unsigned x = (unsigned)(size_t)(const __attribute__((address_space(3))) void*)p;
  asm volatile("" : "+s"(x));
  return x;
}
__device__ __forceinline__ __attribute__((address_space(3))) void* lds_ptr(unsigned a) {
  return (__attribute__((address_space(3))) void*)(size_t)a;
}
// Waits for every outstanding LDS read of this wavefront (lgkmcnt(0)) and
// hands x on as the wait's output, so that no use of x precedes the wait.
__device__ __forceinline__ void lds_wait_tie(bf16x8& x) { asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(x)); }

// Brings the kernel's argument block into the scalar cache at the kernel's
// start: one scalar load per 64-byte line, issued together, then one wait.
// The compiler fetches a large argument block lazily, in many dependent
// batches each waited for at once (and mostly spilled to VGPR lanes under
// register pressure); every batch that touches a new line of the block waits
// a scalar-cache miss.  Warm, those batches hit.  BYTES: the size of the
// kernel's arguments.  (Loads only; the values are discarded.)
template <int BYTES>
__device__ __forceinline__ void prefetch_kernargs() {
  static_assert(BYTES > 0 && BYTES <= 8 * 64, "argument block of 1 to 8 lines");
  constexpr int LINES = (BYTES + 63) / 64;
  const auto kp = __builtin_amdgcn_kernarg_segment_ptr();
  int a[8];
#pragma unroll
  for (int l = 0; l < LINES; ++l) asm volatile("s_load_dword %0, %1, %2" : "=s"(a[l]) : "s"(kp), "i"(64 * l));
  // The loaded values are inputs of the wait, so that each load has a
  // register of its own.
  constexpr int L1 = LINES > 1 ? 1 : 0, L2 = LINES > 2 ? 2 : 0, L3 = LINES > 3 ? 3 : 0, L4 = LINES > 4 ? 4 : 0,
                L5 = LINES > 5 ? 5 : 0, L6 = LINES > 6 ? 6 : 0, L7 = LINES > 7 ? 7 : 0;
  asm volatile("s_waitcnt lgkmcnt(0)" ::"s"(a[0]), "s"(a[L1]), "s"(a[L2]), "s"(a[L3]), "s"(a[L4]), "s"(a[L5]),
               "s"(a[L6]), "s"(a[L7])
               : "memory");
}

__device__ __forceinline__ bf16x8 load_frag(const bf16* p) {
  return *reinterpret_cast<const bf16x8*>(p);
}
__device__ __forceinline__ float load_frag(const float* p) { return *p; }

}  // namespace nkl

// ----------------------------------------------------- host-side helpers --
namespace nkl {
// Records `msg` as this thread's last error and returns `code`.
int set_error(int code, const char* fmt, ...);
// Checks hipGetLastError() after a launch; returns NKL_OK or NKL_ELAUNCH.
int check_launch(const char* what);
}  // namespace nkl
