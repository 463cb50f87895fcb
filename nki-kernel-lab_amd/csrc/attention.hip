// Causal attention on gfx950.
//
// flash_fwd_kernel -- the hot path.  One 256-thread workgroup owns BM = 64
// consecutive queries of one head; each of its four wavefronts owns 16 of
// them.  Key/value tiles of BN keys stream through double-buffered LDS and
// the running softmax state (max, sum, output) stays in registers, so
// scores never leave the chip.  Key tiles entirely above the diagonal are
// never visited; the tiles that straddle it are masked element-wise.
//
// Everything is computed transposed so that each lane always works on a
// single query:
//     S^T = K . Q^T      (A = K rows from LDS, B = Q^T fragments in VGPRs)
//     O^T = V^T . P^T    (A = V^T from LDS,    B = P^T straight from S^T)
// With 16x16 MFMAs, lane l holds query l % 16 of its wavefront in both the
// S^T and O^T accumulators, so the running max / sum / correction factor are
// per-lane scalars, and the probabilities produced by the exp are already in
// the B-operand layout of the P.V MFMA (no shuffle, no LDS round trip).
// For bf16 the V tile is written to LDS transposed and key-permuted so that
// the V^T operand is one 16-byte read per MFMA.
//
// attention_naive -- the reference's unfused variant: scores and
// probabilities are materialised in a caller-provided workspace, using the
// GEMM kernels for Q.K^T and P.V and a masked row softmax in between.
#include <math.h>

#include "attention.h"

namespace nkl {


template <typename T>
struct FlashCfg;
template <>
struct FlashCfg<bf16> { static constexpr int BN = 64; };
template <>
struct FlashCfg<float> { static constexpr int BN = 32; };

// bf16 V^T layout: within a tile of 64 keys, key kk = 16 * kb + 4 * g + i
// (kb < 4, g < 4, i < 4) is stored at column 32 * (kb / 2) + 8 * g +
// 4 * (kb % 2) + i, so that lane group g's eight keys of MFMA t = kb / 2 are
// contiguous -- the same order in which the lane holds their probabilities.
__device__ __forceinline__ int vt_col(int kk) {
  const int kb = kk >> 4, g = (kk >> 2) & 3, i = kk & 3;
  return 32 * (kb >> 1) + 8 * g + 4 * (kb & 1) + i;
}

template <typename T, int D>
__global__ __launch_bounds__(256) void flash_fwd_kernel(AttnArgs p) {
  using MF = Mfma16<T>;
  constexpr bool BF = sizeof(T) == 2;
  constexpr int BM = 64;
  constexpr int BN = FlashCfg<T>::BN;
  constexpr int E = VecE<T>::value;      // elements per 16-byte chunk
  constexpr int CPR = D / E;             // 16-byte chunks per K/V row
  constexpr int LDK = D + E;             // K (and f32 V) LDS row stride, padded
  constexpr int LDV = BN + 8;            // bf16 V^T LDS row stride, padded
  constexpr int K_CH = BN * CPR / 256;   // K chunks per thread
  constexpr int NKB = BN / 16;           // 16-key sub-blocks per tile
  constexpr int ND = D / 16;             // 16-wide d blocks of O^T
  constexpr int NQF = D / MF::MK;        // Q fragments per lane
  static_assert(K_CH >= 1 && (BN * CPR) % 256 == 0, "tile does not split over 256 threads");

  constexpr int V_ELEMS = BF ? D * LDV : BN * LDK;
  __shared__ T Ks[2][BN * LDK];
  __shared__ T Vs[2][V_ELEMS];

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int g = lane >> 4, r = lane & 15;
  const int S = p.S, dlim = p.d;

  // Heavy-first: the first workgroups dispatched take the query blocks with
  // the most key tiles; consecutive ids walk the heads, so with 8 heads head
  // h always lands on XCD h and its K/V stay in one L2.
  const int nqb = (S + BM - 1) / BM;
  const int h = blockIdx.x % p.H;
  const int qb = nqb - 1 - blockIdx.x / p.H;
  const int q0 = qb * BM;
  const int qw = q0 + 16 * w;   // first query of this wavefront
  const int myq = qw + r;       // this lane's query

  const T* Q = static_cast<const T*>(p.q) + (long)h * p.q_sh;
  const T* K = static_cast<const T*>(p.k) + (long)(h / p.group) * p.k_sh;  // shared K/V head (GQA)
  const T* V = static_cast<const T*>(p.v) + (long)(h / p.group) * p.v_sh;
  T* O = static_cast<T*>(p.o) + (long)h * p.o_sh;

  // Q^T fragments: lane (r, g) holds Q[myq][MK * f + KPER * g + j].
  typename MF::frag qf[NQF];
#pragma unroll
  for (int f = 0; f < NQF; ++f) {
    const int dd = f * MF::MK + g * MF::KPER;
    if constexpr (BF) {
      if (myq < S && dd < dlim)
        qf[f] = load_frag(Q + (long)myq * p.q_ss + dd);
      else
#pragma unroll
        for (int j = 0; j < 8; ++j) qf[f][j] = (bf16)0.f;
    } else {
      qf[f] = (myq < S && dd < dlim) ? Q[(long)myq * p.q_ss + dd] : 0.f;
    }
  }

  // ---- K/V staging: global -> registers -> LDS.
  uint4 rk[K_CH];
  // bf16 V: a thread moves 4 consecutive keys x 8 d values.
  constexpr int V_GRP = BF ? (BN / 4) * (D / 8) : 0;
  constexpr int V_IT = BF ? (V_GRP + 255) / 256 : K_CH;
  uint4 rv[BF ? V_IT * 4 : K_CH];
  auto gload = [&](int k0) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < K_CH; ++i) {
      const int c = tid + 256 * i, row = c / CPR, cc = (c % CPR) * E;
      const int key = k0 + row;
      rk[i] = ld16_or_zero(K, (long)key * p.k_ss + cc, key < S && cc < dlim);
      if constexpr (!BF)
        rv[i] = ld16_or_zero(V, (long)key * p.v_ss + cc, key < S && cc < dlim);
    }
    if constexpr (BF) {
#pragma unroll
      for (int it = 0; it < V_IT; ++it) {
        const int grp = tid + 256 * it;
        const int kg = grp % (BN / 4), dc = (grp / (BN / 4)) * 8;
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
          const int key = k0 + 4 * kg + rr;
          rv[it * 4 + rr] = ld16_or_zero(V, (long)key * p.v_ss + dc, grp < V_GRP && key < S && dc < dlim);
        }
      }
    }
  };

  auto lstore = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < K_CH; ++i) {
      const int c = tid + 256 * i, row = c / CPR, cc = (c % CPR) * E;
      *reinterpret_cast<uint4*>(&Ks[buf][row * LDK + cc]) = rk[i];
      if constexpr (!BF) *reinterpret_cast<uint4*>(&Vs[buf][row * LDK + cc]) = rv[i];
    }
    if constexpr (BF) {
#pragma unroll
      for (int it = 0; it < V_IT; ++it) {
        const int grp = tid + 256 * it;
        if (grp < V_GRP) {
          const int kg = grp % (BN / 4), dc = (grp / (BN / 4)) * 8;
          const int col = vt_col(4 * kg);
          const uint32_t* a0 = reinterpret_cast<const uint32_t*>(&rv[it * 4 + 0]);
          const uint32_t* a1 = reinterpret_cast<const uint32_t*>(&rv[it * 4 + 1]);
          const uint32_t* a2 = reinterpret_cast<const uint32_t*>(&rv[it * 4 + 2]);
          const uint32_t* a3 = reinterpret_cast<const uint32_t*>(&rv[it * 4 + 3]);
#pragma unroll
          for (int jj = 0; jj < 8; ++jj) {
            const int wd = jj >> 1;
            uint2 t;
            if (jj & 1) {
              t.x = (a0[wd] >> 16) | (a1[wd] & 0xffff0000u);
              t.y = (a2[wd] >> 16) | (a3[wd] & 0xffff0000u);
            } else {
              t.x = (a0[wd] & 0xffffu) | (a1[wd] << 16);
              t.y = (a2[wd] & 0xffffu) | (a3[wd] << 16);
            }
            *reinterpret_cast<uint2*>(&Vs[buf][(dc + jj) * LDV + col]) = t;
          }
        }
      }
    }
  };

  // ---- running state for query myq
  float m_run = -INFINITY;  // running max of s * c
  float l_run = 0.f;        // this lane's share of the running sum
  floatx4 oacc[ND];
#pragma unroll
  for (int db = 0; db < ND; ++db) oacc[db] = floatx4{0.f, 0.f, 0.f, 0.f};

  const int q_last = min(q0 + BM, S) - 1;
  const int nkt = q_last / BN + 1;  // key tiles 0 .. nkt-1 (the rest are above the diagonal)
  const int wq_last = qw + 15;

  gload(0);
  lstore(0);
  __syncthreads();

  for (int jt = 0; jt < nkt; ++jt) {
    const int buf = jt & 1;
    const int k0 = jt * BN;
    if (jt + 1 < nkt) gload(k0 + BN);

    // S^T = K . Q^T for this wavefront's 16 queries.
    floatx4 sacc[NKB];
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
      sacc[kb] = floatx4{0.f, 0.f, 0.f, 0.f};
      if (k0 + 16 * kb <= wq_last) {
#pragma unroll
        for (int f = 0; f < NQF; ++f) {
          const typename MF::frag a = load_frag(&Ks[buf][(16 * kb + r) * LDK + f * MF::MK + g * MF::KPER]);
          sacc[kb] = MF::mma(a, qf[f], sacc[kb]);
        }
      }
    }

    // Online softmax.  Element i of sacc[kb] is key k0 + 16 kb + 4 g + i.
    const bool diag = k0 + BN - 1 > qw;
    float mloc = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float s = sacc[kb][i] * p.c;
        if (diag && k0 + 16 * kb + 4 * g + i > myq) s = -INFINITY;
        sacc[kb][i] = s;
        mloc = fmaxf(mloc, s);
      }
    mloc = fmaxf(mloc, __shfl_xor(mloc, 16, kWave));
    mloc = fmaxf(mloc, __shfl_xor(mloc, 32, kWave));
    const float m_new = fmaxf(m_run, mloc);
    const float corr = fast_exp2(m_run - m_new);
    m_run = m_new;
    float rsum = 0.f;
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float e = fast_exp2(sacc[kb][i] - m_new);
        sacc[kb][i] = e;
        rsum += e;
      }
    l_run = fmaf(l_run, corr, rsum);
#pragma unroll
    for (int db = 0; db < ND; ++db)
#pragma unroll
      for (int i = 0; i < 4; ++i) oacc[db][i] *= corr;

    // O^T += V^T . P^T
    if constexpr (BF) {
#pragma unroll
      for (int t = 0; t < BN / 32; ++t) {
        if (k0 + 32 * t > wq_last) continue;
        bf16x8 pf;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          pf[i] = (bf16)sacc[2 * t][i];
          pf[4 + i] = (bf16)sacc[2 * t + 1][i];
        }
#pragma unroll
        for (int db = 0; db < ND; ++db) {
          const bf16x8 a = load_frag(&Vs[buf][(16 * db + r) * LDV + 32 * t + 8 * g]);
          oacc[db] = MF::mma(a, pf, oacc[db]);
        }
      }
    } else {
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) {
        if (k0 + 16 * kb > wq_last) continue;
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int db = 0; db < ND; ++db) {
            const float a = Vs[buf][(16 * kb + 4 * g + i) * LDK + 16 * db + r];
            oacc[db] = MF::mma(a, sacc[kb][i], oacc[db]);
          }
      }
    }

    if (jt + 1 < nkt) lstore(buf ^ 1);
    __syncthreads();
  }

  // Finish: l = sum over the four lane groups; O = O^T / l rounded once.
  float l = l_run + __shfl_xor(l_run, 16, kWave);
  l += __shfl_xor(l, 32, kWave);
  const float linv = 1.0f / l;
  if (myq < S) {
    T* orow = O + (long)myq * p.o_ss;
#pragma unroll
    for (int db = 0; db < ND; ++db) {
      const int dd = 16 * db + 4 * g;
      if (dd < dlim) {
        float ov[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) ov[i] = oacc[db][i] * linv;
        store_vec<4>(orow + dd, ov);
      }
    }
  }
}

// ------------------------------------------------ naive (unfused) path --
// nkilab/kernels/attention.py:35-89, pass 2: scores (already Q.K^T) are
// scaled and causally masked, then a row softmax writes P in the input dtype.
template <typename T>
__global__ __launch_bounds__(256) void masked_softmax_kernel(float* __restrict__ sc, T* __restrict__ pr, int H,
                                                             int S, float scale) {
  const int lane = threadIdx.x & 63;
  const long row = (long)blockIdx.x * 4 + (threadIdx.x >> 6);  // (h, q) flattened
  if (row >= (long)H * S) return;
  const int q = (int)(row % S);
  float* srow = sc + row * S;
  T* prow = pr + row * S;
  float mx = -INFINITY;
  for (int c = lane; c < S; c += kWave) {
    const float s = c > q ? -INFINITY : srow[c] * scale;
    srow[c] = s;
    mx = fmaxf(mx, s);
  }
  mx = wave_max(mx);
  float sum = 0.f;
  for (int c = lane; c < S; c += kWave) sum += fast_exp2((srow[c] - mx) * kLog2e);
  sum = wave_sum(sum);
  const float rinv = 1.0f / sum;
  for (int c = lane; c < S; c += kWave) prow[c] = from_f32<T>(fast_exp2((srow[c] - mx) * kLog2e) * rinv);
}

static bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

template <int D>
static void flash_f32_launch(const AttnArgs& a, hipStream_t st) {
  const int nqb = (a.S + 63) / 64;
  flash_fwd_kernel<float, D><<<dim3((unsigned)(nqb * a.H)), dim3(256), 0, st>>>(a);
}

static int flash_f32_dispatch(const AttnArgs& a, hipStream_t st) {
  if (a.d <= 32)
    flash_f32_launch<32>(a, st);
  else if (a.d <= 64)
    flash_f32_launch<64>(a, st);
  else
    flash_f32_launch<128>(a, st);
  return check_launch("nkl_flash_attn_causal");
}

}  // namespace nkl

using namespace nkl;

constexpr long kMaxRowStride = 1L << 21;

static int check_attn(const char* fn, const void* q, const void* k, const void* v, const void* o, int H, int S,
                      int d, int dtype, const long* strides) {
  if (H < 0 || S < 0) return set_error(NKL_EINVAL, "%s: negative shape H=%d S=%d", fn, H, S);
  if (d < 1 || d > 128) return set_error(NKL_EINVAL, "%s: head dim d=%d outside [1, 128]", fn, d);
  if (dtype != NKL_F32 && dtype != NKL_BF16 && dtype != NKL_F16)
    return set_error(NKL_EDTYPE, "%s: unsupported dtype %d", fn, dtype);
  const int E = dtype == NKL_F32 ? 4 : 8;
  if (d % E != 0)
    return set_error(NKL_EINVAL, "%s: d=%d must be a multiple of %d (pad the head dim on the host)", fn, d, E);
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(o))
    return set_error(NKL_EINVAL, "%s: q/k/v/o must be 16-byte aligned", fn);
  if (H > 0 && S > 0 && (!q || !k || !v || !o)) return set_error(NKL_EINVAL, "%s: null q/k/v/o", fn);
  // Head strides (even entries) up to 2^24 elements; row strides (odd) up to
  // 2^21, so that the kernels' 32-bit byte offsets within a block of up to 256
  // rows stay below 2^30 -- the offset at which a copy of a chunk past d reads
  // zeros from outside every buffer.
  for (int i = 0; i < 8; ++i) {
    const long lim = i % 2 ? kMaxRowStride : 1L << 24;
    if (strides[i] % E != 0)
      return set_error(NKL_EINVAL, "%s: stride %ld is not a multiple of %d elements", fn, strides[i], E);
    if (strides[i] < 0 || strides[i] > lim)
      return set_error(NKL_EINVAL, "%s: %s stride %ld outside [0, %ld]", fn, i % 2 ? "row" : "head", strides[i], lim);
  }
  return NKL_OK;
}

static int flash_entry(const char* fn, const void* q, const void* k, const void* v, void* o, void* workspace,
                       size_t workspace_bytes, int* counters, size_t counter_bytes, bool ws_entry, int H, int Hkv,
                       int S, int d, const long* st8, float scale, int dtype, void* stream) {
  int rc = check_attn(fn, q, k, v, o, H, S, d, dtype, st8);
  if (rc) return rc;
  if (Hkv < 1 || H % Hkv != 0)
    return set_error(NKL_EINVAL, "%s: H=%d query heads do not divide into Hkv=%d K/V heads", fn, H, Hkv);
  if (H == 0 || S == 0) return NKL_OK;
  AttnArgs a{q, k, v, o, H, S, d, st8[0], st8[1], st8[2], st8[3], st8[4], st8[5], st8[6], st8[7], scale * kLog2e,
             H / Hkv, dtype == NKL_F16 ? 1 : 0};
  hipStream_t st = (hipStream_t)stream;
  if (dtype == NKL_BF16 || dtype == NKL_F16) {
    if (!ws_entry) return flash_bf16_launch(a, nullptr, 0, nullptr, 0, st);
    // Shapes that need no scratch (size 0) accept a null workspace.
    if (!workspace && flash_bf16_workspace_bytes(H, S, d, dtype == NKL_F16) > 0)
      return set_error(NKL_EWORKSPACE, "%s: null workspace", fn);
    return flash_bf16_launch(a, workspace, workspace_bytes, counters, counter_bytes, st);
  }
  return flash_f32_dispatch(a, st);
}

extern "C" int nkl_flash_attn_causal(const void* q, const void* k, const void* v, void* o, int H, int S, int d,
                                     long q_sh, long q_ss, long k_sh, long k_ss, long v_sh, long v_ss, long o_sh,
                                     long o_ss, float scale, int dtype, void* stream) {
  const long strides[8] = {q_sh, q_ss, k_sh, k_ss, v_sh, v_ss, o_sh, o_ss};
  return flash_entry("nkl_flash_attn_causal", q, k, v, o, nullptr, 0, nullptr, 0, false, H, H > 0 ? H : 1, S, d,
                     strides, scale, dtype, stream);
}

extern "C" size_t nkl_flash_attn_causal_workspace_bytes(int H, int S, int d, int dtype) {
  if (dtype != NKL_BF16 && dtype != NKL_F16) return 0;
  return flash_bf16_workspace_bytes(H, S, d, dtype == NKL_F16);
}

extern "C" size_t nkl_flash_attn_causal_counter_bytes(int H, int S, int dtype) {
  if (dtype != NKL_BF16 && dtype != NKL_F16) return 0;
  return flash_bf16_counter_bytes(H, S);
}

extern "C" int nkl_flash_attn_causal_ws(const void* q, const void* k, const void* v, void* o, void* workspace,
                                        size_t workspace_bytes, int* counters, size_t counter_bytes, int H, int S,
                                        int d, long q_sh, long q_ss, long k_sh, long k_ss, long v_sh, long v_ss,
                                        long o_sh, long o_ss, float scale, int dtype, void* stream) {
  const long strides[8] = {q_sh, q_ss, k_sh, k_ss, v_sh, v_ss, o_sh, o_ss};
  return flash_entry("nkl_flash_attn_causal_ws", q, k, v, o, workspace, workspace_bytes, counters, counter_bytes,
                     true, H, H > 0 ? H : 1, S, d, strides, scale, dtype, stream);
}

extern "C" int nkl_flash_attn_causal_gqa(const void* q, const void* k, const void* v, void* o, void* workspace,
                                         size_t workspace_bytes, int* counters, size_t counter_bytes, int H, int Hkv,
                                         int S, int d, long q_sh, long q_ss, long k_sh, long k_ss, long v_sh,
                                         long v_ss, long o_sh, long o_ss, float scale, int dtype, void* stream) {
  const long strides[8] = {q_sh, q_ss, k_sh, k_ss, v_sh, v_ss, o_sh, o_ss};
  return flash_entry("nkl_flash_attn_causal_gqa", q, k, v, o, workspace, workspace_bytes, counters, counter_bytes,
                     true, H, Hkv, S, d, strides, scale, dtype, stream);
}

// Scratch of the allocation-free entry point: kNoAllocPartBytes of partial
// states, then kNoAllocCounterBytes of arrival counters.  Each GPU the library
// runs on holds its own copy from the first call until the process ends.  In
// host code the array's name is not a device address: kernels and fills get
// the per-device address hipGetSymbolAddress returns.
constexpr size_t kNoAllocPartBytes = (size_t)64 << 20;
constexpr size_t kNoAllocCounterBytes = (size_t)1 << 20;
constexpr int kNoAllocMaxDevices = 64;
static __device__ __align__(256) unsigned char scratch[kNoAllocPartBytes + kNoAllocCounterBytes];
static void* scratch_addr[kNoAllocMaxDevices];

static __global__ void zero_words_kernel(int* p, long n) {
  for (long i = blockIdx.x * (long)blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x) p[i] = 0;
}

// The current device's copy of `scratch`, looked up once per device.  Two
// threads racing on a device's first call both store the same address.
static int scratch_of_current_device(const char* fn, unsigned char** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kNoAllocMaxDevices)
    return set_error(NKL_ELAUNCH, "%s: no usable current device (%d)", fn, dev);
  void* p = __atomic_load_n(&scratch_addr[dev], __ATOMIC_ACQUIRE);
  if (!p) {
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return set_error(NKL_ELAUNCH, "%s: hipGetSymbolAddress(scratch) failed on device %d: %s", fn, dev,
                       hipGetErrorString(e));
    __atomic_store_n(&scratch_addr[dev], p, __ATOMIC_RELEASE);
  }
  *out = static_cast<unsigned char*>(p);
  return NKL_OK;
}

extern "C" int nkl_flash_attn_causal_noalloc(const void* q, const void* k, const void* v, void* o, int H, int Hkv,
                                             int S, int d, long q_sh, long q_ss, long k_sh, long k_ss, long v_sh,
                                             long v_ss, long o_sh, long o_ss, float scale, int dtype, void* stream) {
  const char* fn = "nkl_flash_attn_causal_noalloc";
  const long strides[8] = {q_sh, q_ss, k_sh, k_ss, v_sh, v_ss, o_sh, o_ss};
  int rc = check_attn(fn, q, k, v, o, H, S, d, dtype, strides);
  if (rc) return rc;
  if ((dtype != NKL_BF16 && dtype != NKL_F16) || H == 0 || S == 0)  // no scratch on these paths
    return flash_entry(fn, q, k, v, o, nullptr, 0, nullptr, 0, true, H, Hkv, S, d, strides, scale, dtype, stream);
  const size_t need = flash_bf16_workspace_bytes(H, S, d, dtype == NKL_F16);
  // One counter per 64-query block (the smallest block) covers every schedule.
  const size_t need_c = need ? (size_t)H * ((S + 63) / 64) * 4 : 0;
  if (need > kNoAllocPartBytes || need_c > kNoAllocCounterBytes)
    return set_error(NKL_EWORKSPACE,
                     "%s: H=%d S=%d d=%d needs %zu bytes of partial states and %zu of counters; the static scratch "
                     "holds %zu and %zu (use nkl_flash_attn_causal_gqa with a workspace)",
                     fn, H, S, d, need, need_c, kNoAllocPartBytes, kNoAllocCounterBytes);
  unsigned char* base = nullptr;
  if ((rc = scratch_of_current_device(fn, &base))) return rc;
  int* counters = reinterpret_cast<int*>(base + kNoAllocPartBytes);
  if (need_c > 0) {
    // The kernels leave the counters zero; clear them anyway, with a kernel
    // (not a memset node) so that the call can be captured in a graph.
    const long n = (long)(need_c / 4);
    zero_words_kernel<<<dim3((unsigned)((n + 255) / 256 < 64 ? (n + 255) / 256 : 64)), dim3(256), 0,
                        (hipStream_t)stream>>>(counters, n);
    if ((rc = check_launch(fn))) return rc;
  }
  return flash_entry(fn, q, k, v, o, need ? base : nullptr, need, counters, need_c, true, H, Hkv, S, d, strides,
                     scale, dtype, stream);
}

extern "C" int nkl_flash_attn_configure(int kernel, int schedule, int qb, int cpb) {
  return flash_bf16_configure(kernel, schedule, qb, cpb);
}

extern "C" int nkl_flash_attn_configure_polls(int polls) { return flash_bf16_configure_polls(polls); }

extern "C" int nkl_flash_attn_plan_check(int H, int S, int d, int dtype, long* info) {
  if (dtype != NKL_BF16 && dtype != NKL_F16)
    return set_error(NKL_EDTYPE, "nkl_flash_attn_plan_check: the 16-bit kernels only (dtype %d)", dtype);
  return flash_bf16_plan_check(H, S, d, dtype == NKL_F16, info);
}

extern "C" size_t nkl_attention_naive_workspace_bytes(int H, int S, int dtype) {
  if (H <= 0 || S <= 0) return 0;
  const size_t n = (size_t)H * S * S;
  const size_t sc = (n * 4 + 255) / 256 * 256;
  return sc + n * (dtype == NKL_F32 ? 4 : 2);
}

static int naive_entry(const char* fn, const void* q, const void* k, const void* v, void* o, void* workspace,
                       size_t workspace_bytes, int H, int Hkv, int S, int d, const long* st8, float scale, int dtype,
                       void* stream) {
  int rc = check_attn(fn, q, k, v, o, H, S, d, dtype, st8);
  if (rc) return rc;
  if (Hkv < 1 || H % Hkv != 0)
    return set_error(NKL_EINVAL, "%s: H=%d query heads do not divide into Hkv=%d K/V heads", fn, H, Hkv);
  if (H == 0 || S == 0) return NKL_OK;
  const size_t need = nkl_attention_naive_workspace_bytes(H, S, dtype);
  if (!workspace || workspace_bytes < need)
    return set_error(NKL_EWORKSPACE, "%s: workspace of %zu bytes needed, %zu given", fn, need, workspace_bytes);
  const long q_sh = st8[0], q_ss = st8[1], k_sh = st8[2], k_ss = st8[3], v_sh = st8[4], v_ss = st8[5],
             o_sh = st8[6], o_ss = st8[7];
  const size_t n = (size_t)H * S * S;
  float* sc = static_cast<float*>(workspace);
  char* pr = static_cast<char*>(workspace) + (n * 4 + 255) / 256 * 256;
  const size_t esz = dtype == NKL_F32 ? 4 : 2;
  hipStream_t st = (hipStream_t)stream;
  const long SS = (long)S * S;
  const int G = H / Hkv;
  // Query head h = kvh * G + g uses K/V head kvh.  For each g, the heads
  // g, G + g, ... form one batched GEMM over the K/V heads (batch strides
  // G times the query / score / output strides).
  // pass 1: scores[h] = Q[h] . K[h / G]^T (fp32)
  for (int g = 0; g < G; ++g) {
    rc = nkl_gemm(static_cast<const char*>(q) + g * q_sh * esz, k, sc + g * SS, nullptr, S, S, d, q_ss, k_ss, S, 0, 1,
                  Hkv, G * q_sh, k_sh, G * SS, 0, dtype, NKL_F32, NKL_GEMM_BLOCKED, stream);
    if (rc) return rc;
  }
  // pass 2: scale, mask, row softmax -> P
  const dim3 grid((unsigned)(((long)H * S + 3) / 4)), block(256);
  if (dtype == NKL_BF16)
    masked_softmax_kernel<bf16><<<grid, block, 0, st>>>(sc, reinterpret_cast<bf16*>(pr), H, S, scale);
  else if (dtype == NKL_F16)
    masked_softmax_kernel<f16><<<grid, block, 0, st>>>(sc, reinterpret_cast<f16*>(pr), H, S, scale);
  else
    masked_softmax_kernel<float><<<grid, block, 0, st>>>(sc, reinterpret_cast<float*>(pr), H, S, scale);
  rc = check_launch(fn);
  if (rc) return rc;
  // pass 3: O[h] = P[h] . V[h / G]
  for (int g = 0; g < G; ++g) {
    rc = nkl_gemm(pr + g * SS * esz, v, static_cast<char*>(o) + g * o_sh * esz, nullptr, S, d, S, S, v_ss, o_ss, 0,
                  0, Hkv, G * SS, v_sh, G * o_sh, 0, dtype, dtype, NKL_GEMM_BLOCKED, stream);
    if (rc) return rc;
  }
  return NKL_OK;
}

extern "C" int nkl_attention_naive(const void* q, const void* k, const void* v, void* o, void* workspace,
                                   size_t workspace_bytes, int H, int S, int d, long q_sh, long q_ss, long k_sh,
                                   long k_ss, long v_sh, long v_ss, long o_sh, long o_ss, float scale, int dtype,
                                   void* stream) {
  const long strides[8] = {q_sh, q_ss, k_sh, k_ss, v_sh, v_ss, o_sh, o_ss};
  return naive_entry("nkl_attention_naive", q, k, v, o, workspace, workspace_bytes, H, H > 0 ? H : 1, S, d, strides,
                     scale, dtype, stream);
}

extern "C" int nkl_attention_naive_gqa(const void* q, const void* k, const void* v, void* o, void* workspace,
                                       size_t workspace_bytes, int H, int Hkv, int S, int d, long q_sh, long q_ss,
                                       long k_sh, long k_ss, long v_sh, long v_ss, long o_sh, long o_ss, float scale,
                                       int dtype, void* stream) {
  const long strides[8] = {q_sh, q_ss, k_sh, k_ss, v_sh, v_ss, o_sh, o_ss};
  return naive_entry("nkl_attention_naive_gqa", q, k, v, o, workspace, workspace_bytes, H, Hkv, S, d, strides, scale,
                     dtype, stream);
}
