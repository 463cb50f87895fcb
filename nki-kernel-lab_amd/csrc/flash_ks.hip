// bf16 / fp16 causal flash attention for gfx950, 64 < d <= 128: the key-split
// kernel.
//
// Work decomposition.  Queries are grouped in blocks of 64, keys in tiles of
// 32; units, schedules and balanced ranges are those of flash_sched.h with
// QB = 64.  A workgroup of four wavefronts (one per SIMD) walks its range as
// segments, one per query block it touches.  Every wavefront holds all 64
// queries of the segment's block (two 32-query halves, Q^T in registers) and
// takes every fourth key tile of the segment: wavefront w the tiles
// t0 + w, t0 + w + 4, ...  So the four wavefronts share no tile: each copies
// its own tiles global -> LDS with the buffer unit (buffer_load ... lds, lane
// l's 16 bytes at the instruction's LDS base + 16 l) into its own two K and
// two V buffers, waits only for its own copies, and the loop holds no
// workgroup barrier.  Each K and V byte is copied once per workgroup, and
// every fragment read from LDS feeds two MFMAs (one per query half).
//
// Per wavefront and tile, with 32x32x16 MFMAs (H: the fp16 form):
//     S^T[32 keys x 32 queries] = K . Q^T       8 MFMAs per half
//     O^T[128 d x 32 queries]  += V^T . P^T     8 MFMAs per half
// Lane l holds query l % 32 of each half; its 16 scores are keys
// 8 (i / 4) + 4 (l / 32) + i % 4, so elements 8 u .. 8 u + 7 are the B operand
// of the P V MFMA over keys 16 u .. 16 u + 15.  The V^T operand comes from
// ds_read_b64_tr_b16 transposed reads.  K, V and Q rows are 256 bytes in LDS,
// their 16-byte chunks swizzled (logical chunk c of row r at c ^ row_swz(r)),
// which keeps the fragment reads free of bank conflicts.
//
// Software pipeline of a wavefront, per tile i of its own (three regions,
// each a fixed MFMA/VALU interleave):
//     region 1: S(i+1) = K(i+1) Q^T      x  exp and bf16 P of S(i), half 0
//                                           and the first 8 keys of half 1
//     region 2: O(half 0) += P(i) V(i)   x  the rest of half 1
//     region 3: O(half 1) += P(i) V(i)   x  mask and row max of S(i+1)
// K fragments are read one tile ahead (K(i+2) during region 2), V fragments
// at the start of their tile, and each buffer is refilled as soon as its
// fragments are in registers: copies run two tiles ahead of use with two
// buffers per tensor.  The running max is raised lazily (fsched::kRescaleSlack).
//
// At the end of a segment the four states (max, sum, O) are combined through
// LDS in a fixed order, wavefront w finishing d-block w (32 columns).  A block
// whose units span several ranges is finished by the workgroup that arrives
// last, with no waiting: each part stores its state to the workspace (unless
// it already sees every other part arrived) and counts itself in on the
// block's arrival counter; the part that completes the count folds all parts
// in range order and writes O.  The fold order does not depend on which part
// merges, so results are bitwise reproducible.
#include <math.h>

#include "attention.h"
#include "flash_sched.h"

namespace nkl {

namespace {

using namespace fsched;

constexpr int KS_BN = 32;                          // keys per tile
constexpr int KS_QB = 64;                          // queries per block
constexpr int KS_NW = 4;                           // wavefronts (one per SIMD)
constexpr int KS_ROWB = 256;                       // bytes of a 128-element 16-bit row
constexpr int KS_TILEB = KS_BN * KS_ROWB;          // bytes of a K (or V) tile
constexpr int KS_VOFF = 2 * KS_TILEB;              // V buffers after the two K buffers
constexpr int KS_WAVEB = 4 * KS_TILEB;             // one wavefront's K and V buffers
constexpr int KS_QOFF = KS_NW * KS_WAVEB;          // the block's Q rows
constexpr int KS_LDS = KS_QOFF + KS_QB * KS_ROWB;  // 144 KB
// End-of-segment exchange (over the K/V buffers): (m, l) of every wavefront,
// half and query, then 12 slots of 8 KB -- the d-blocks a wavefront does not
// finish, as 8 float4 chunks per lane.
constexpr int KS_XML = 0;
constexpr int KS_XO = 2048;
constexpr int KS_XSLOT = 8 * 64 * 16;
static_assert(KS_XO + 12 * KS_XSLOT <= KS_QOFF, "exchange area overlaps Q");
// Parts of a split block a wavefront stages per round trip of the merge:
// ten 1 KB chunks each, in its 32 KB of K/V buffers.
constexpr int KS_MB = 3;
static_assert(KS_MB * 10 * 1024 <= KS_WAVEB, "merge staging fits a wavefront's buffers");
// A part's state in the workspace (floats): per d-block 8 float4 chunks per
// lane (the wavefront finishing it stores them), then (m, l, 0, 0) per lane
// and half.
constexpr int KS_PDB = 8 * 64 * 4;
constexpr int KS_PARTF = 4 * KS_PDB + 2 * 64 * 4;

// LDS reads through inline assembly with an immediate offset: the compiler
// does not track them (their results go through lds_wait_tie() before use),
// so that its own waits never hold them behind the outstanding copies.
// The read at (base ^ X) + OFF: the XOR is part of the statement, so that the
// compiler neither hoists the per-fragment addresses into registers of their
// own nor reorders the reads.
template <int X, int OFF>
__device__ __forceinline__ bf16x8 ds_b128(unsigned base) {
  bf16x8 r;
  unsigned t;
  asm volatile("v_xor_b32 %1, %3, %2\n\tds_read_b128 %0, %1 offset:%4"
               : "=v"(r), "=&v"(t)
               : "v"(base), "i"(X), "i"(OFF));
  return r;
}
template <int X, int OFF>
__device__ __forceinline__ shortx4 ds_tr64(unsigned base) {
  shortx4 r;
  unsigned t;
  asm volatile("v_xor_b32 %1, %3, %2\n\tds_read_b64_tr_b16 %0, %1 offset:%4"
               : "=v"(r), "=&v"(t)
               : "v"(base), "i"(X), "i"(OFF));
  return r;
}

// Fragment f (a compile-time constant once unrolled) at base ^ (32 f).
template <int OFF>
__device__ __forceinline__ bf16x8 ds_b128_f(unsigned base, int f) {
  switch (f) {
    case 0: return ds_b128<0, OFF>(base);
    case 1: return ds_b128<32, OFF>(base);
    case 2: return ds_b128<64, OFF>(base);
    case 3: return ds_b128<96, OFF>(base);
    case 4: return ds_b128<128, OFF>(base);
    case 5: return ds_b128<160, OFF>(base);
    case 6: return ds_b128<192, OFF>(base);
    default: return ds_b128<224, OFF>(base);
  }
}
// V^T fragment halves of d-block db at base ^ (64 db).
template <int OFF>
__device__ __forceinline__ shortx4 ds_tr64_db(unsigned base, int db) {
  switch (db) {
    case 0: return ds_tr64<0, OFF>(base);
    case 1: return ds_tr64<64, OFF>(base);
    case 2: return ds_tr64<128, OFF>(base);
    default: return ds_tr64<192, OFF>(base);
  }
}
// Q fragments live in AGPRs, read there straight from LDS.
template <int X, int OFF>
__device__ __forceinline__ bf16x8 ds_b128_acc(unsigned base) {
  bf16x8 r;
  unsigned t;
  asm volatile("v_xor_b32 %1, %3, %2\n\tds_read_b128 %0, %1 offset:%4"
               : "=a"(r), "=&v"(t)
               : "v"(base), "i"(X), "i"(OFF));
  return r;
}
template <int OFF>
__device__ __forceinline__ bf16x8 ds_b128_acc_f(unsigned base, int f) {
  switch (f) {
    case 0: return ds_b128_acc<0, OFF>(base);
    case 1: return ds_b128_acc<32, OFF>(base);
    case 2: return ds_b128_acc<64, OFF>(base);
    case 3: return ds_b128_acc<96, OFF>(base);
    case 4: return ds_b128_acc<128, OFF>(base);
    case 5: return ds_b128_acc<160, OFF>(base);
    case 6: return ds_b128_acc<192, OFF>(base);
    default: return ds_b128_acc<224, OFF>(base);
  }
}
__device__ __forceinline__ void lds_wait_tie_acc(bf16x8& x) { asm volatile("s_waitcnt lgkmcnt(0)" : "+a"(x)); }

// S^T (+)= K . Q^T as one 32x32x16 MFMA with K in VGPRs, Q in AGPRs and the
// accumulator in VGPRs, where the softmax reads it.  (With the compiler's
// MFMA, every MFMA of a kernel takes one accumulator form: O in AGPRs would
// put S there too, and Q would be copied into VGPRs before every MFMA.)  The
// leading s_nop covers the two wait states a VALU write of an operand needs
// before an MFMA reads it; an MFMA result is not read by VALU code until
// another region's MFMAs have issued, or after qk_settle().
// The result is early-clobber: an MFMA's destination may not overlap its A
// or B operand (the K fragment is often dead after it, and free to reuse).
template <bool H>
__device__ __forceinline__ void qk_first(floatx16& d, const bf16x8& k, const bf16x8& q) {
  if constexpr (H)
    asm volatile("s_nop 1\n\tv_mfma_f32_32x32x16_f16 %0, %1, %2, 0" : "=&v"(d) : "v"(k), "a"(q));
  else
    asm volatile("s_nop 1\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %2, 0" : "=&v"(d) : "v"(k), "a"(q));
}
template <bool H>
__device__ __forceinline__ void qk_acc(floatx16& d, const bf16x8& k, const bf16x8& q) {
  if constexpr (H)
    asm volatile("s_nop 1\n\tv_mfma_f32_32x32x16_f16 %0, %1, %2, %0" : "+v"(d) : "v"(k), "a"(q));
  else
    asm volatile("s_nop 1\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(d) : "v"(k), "a"(q));
}
// O^T += V^T . P^T with the accumulator in AGPRs (P written by VALU code just
// before: the s_nop).
template <bool H>
__device__ __forceinline__ void pv_acc(floatx16& o, const bf16x8& v, const bf16x8& p) {
  if constexpr (H)
    asm volatile("s_nop 1\n\tv_mfma_f32_32x32x16_f16 %0, %1, %2, %0" : "+a"(o) : "v"(v), "v"(p));
  else
    asm volatile("s_nop 1\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(o) : "v"(v), "v"(p));
}
// O = 0 as MFMAs of zero operands: O is made in the AGPRs that hold it.  The
// s_nop is the two wait states between the VALU write of the zero operand
// (often just before) and an MFMA read of it; the compiler adds none in front
// of an asm statement.
template <bool H>
__device__ __forceinline__ void o_zero(floatx16 (&o)[2][4]) {
  const bf16x8 z = {};
#pragma unroll
  for (int hq = 0; hq < 2; ++hq)
#pragma unroll
    for (int db = 0; db < 4; ++db) {
      if constexpr (H)
        asm volatile("s_nop 1\n\tv_mfma_f32_32x32x16_f16 %0, %1, %1, 0" : "=a"(o[hq][db]) : "v"(z));
      else
        asm volatile("s_nop 1\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %1, 0" : "=a"(o[hq][db]) : "v"(z));
    }
}
// Wait states for MFMA results to be read or written by other instructions
// (more than an 8-pass MFMA needs), tied to the results.
__device__ __forceinline__ void qk_settle(floatx16 (&s)[2]) {
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" : "+v"(s[0]), "+v"(s[1]));
}
__device__ __forceinline__ void o_settle(floatx16 (&o)[2][4]) {
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7"
               : "+a"(o[0][0]), "+a"(o[0][1]), "+a"(o[0][2]), "+a"(o[0][3]), "+a"(o[1][0]), "+a"(o[1][1]),
                 "+a"(o[1][2]), "+a"(o[1][3]));
}
// max(a, b, c) in one instruction, at this point of the instruction stream
// (fmaxf behind the pins below would quiet every input first).
__device__ __forceinline__ float max3(float a, float b, float c) {
  float r;
  asm volatile("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}
// Pins a value computed by VALU code to this point of the instruction stream
// (between two MFMA statements).
__device__ __forceinline__ void pin(float& x) { asm volatile("" : "+v"(x)); }
__device__ __forceinline__ void pin(bf16x8& x) { asm volatile("" : "+v"(x)); }

}  // namespace

template <bool H>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
void flash_ks_kernel(AttnArgs p, Work w) {
  constexpr int NQF = 8, NDB = 4;
  __shared__ __align__(16) unsigned char lds[KS_LDS];
  __shared__ int flag;
  // Alone on its SIMD: declaring an AGPR use makes the compiler keep the O
  // accumulators in AGPRs.
  asm volatile("" ::: "a255");
  prefetch_kernargs<sizeof(AttnArgs) + sizeof(Work)>();

  const int tid = threadIdx.x, lane = tid & 63;
  const int wq = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int h32 = lane >> 5, l32 = lane & 31;
  const int S = p.S, dlim = p.d;
  const float c = p.c;

  // Per-lane LDS addresses.  Fragment f of a K or Q tile is row l32, logical
  // chunk 2 f + h32, at physical chunk (2 f + h32) ^ row_swz(l32): byte
  // offset l32 * 256 + ((32 f) ^ (16 (h32 ^ row_swz(l32)))), which is
  // kbase ^ (32 f) with the row, the half and a 256-byte aligned base folded
  // into kbase.  Likewise the V^T fragment of d-block db (first or second
  // 8-row read: rows r0 + 8 half, d = 32 db + 16 g2 + 4 (i16 % 4); +16 rows,
  // a constant 4096 bytes, for keys 16 .. 31) sits at vbase[half] ^ (64 db).
  // One register per base, one XOR per fragment read.
  // LDS addresses go through an empty asm, so that the copies' destinations
  // are opaque to the compiler (else it makes LDS reads wait for every copy).
  const unsigned lds0 = opaque_lds_addr(lds);
  const unsigned wb = lds0 + wq * KS_WAVEB;  // this wavefront's buffers
  const unsigned kbase = wb + l32 * KS_ROWB + ((h32 ^ row_swz(l32)) << 4);
  const unsigned qbase = lds0 + KS_QOFF + l32 * KS_ROWB + ((h32 ^ row_swz(l32)) << 4);
  unsigned vbase[2];
  {
    const int i16 = lane & 15, g2 = (lane >> 4) & 1;
    const int r0 = 4 * h32 + (i16 >> 2);
    const int cb = 2 * g2 + ((i16 & 3) >> 1);
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      const int row = r0 + 8 * half;
      vbase[half] = wb + KS_VOFF + row * KS_ROWB + ((cb ^ row_swz(row)) << 4) + (i16 & 1) * 8;
    }
  }
  // Copy offsets: instruction n = m + 4 k of a tile covers rows 4 n .. 4 n + 3;
  // lane l fills row 4 n + l / 16, physical chunk l % 16, with logical chunk
  // (l % 16) ^ row_swz(row).  row_swz depends on row % 16 = 4 m + l / 16 only,
  // so the lane's offset is dkv[m] plus 32 k rows (a scalar offset).  K and V
  // share the row stride.  Chunks past d read as zero (an offset past any
  // buffer; byte offsets stay below 2^30 with row strides of at most 2^21
  // elements, which the entry points enforce).
  int dkv[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const int row = 4 * m + (lane >> 4);
    const int lc = (lane & 15) ^ row_swz(row);
    dkv[m] = lc * 8 < dlim ? (int)(2u * ((unsigned)row * (unsigned)p.k_ss + 8u * lc)) : 0x40000000;
  }
  const int kv_row32 = 32 * (int)p.k_ss;  // bytes of 16 rows

  int u0, u1;
  const int vidx = wg_range_fast(w, p.H, u0, u1);
  Seg cur = decode_seg_t<int>(u1 - 1, u0, w);

  for (;;) {
    const int hh = cur.hh, b = cur.b, t0 = cur.t0, t1 = cur.t1, nt_b = cur.nt;
    const long bstart = cur.bstart;
    const int nt = t1 - t0;
    const int q0 = KS_QB * b;
    const int kvh = (int)div32(w.dv_group, (unsigned)hh);
    // This wavefront's tiles j = 0 .. ntw - 1 are the segment's tiles
    // wq + 4 j; the first jm of them lie wholly below the block's first query.
    const int ntw = max(0, (nt - wq + 3) >> 2);
    const int jm = max(0, min(ntw, (min(2 * b, t1) - t0 - wq + 3) >> 2));
    const int klim_seg = t1 * KS_BN;

    // The buffer resource of this wavefront's tile j of K (or V); tiles past
    // the segment are empty (their copies read no memory and write zeros).
    auto tile_rsrc = [&](const void* base, long sh, int j) __attribute__((always_inline)) {
      const int tj = t0 + wq + 4 * j;
      const int k0 = tj * KS_BN;
      const int nkeys = tj < t1 ? min(KS_BN, S - k0) : 0;
      const int bytes = nkeys > 0 ? (int)(2u * ((unsigned)(nkeys - 1) * (unsigned)p.k_ss + (unsigned)dlim)) : 0;
      return __builtin_amdgcn_make_buffer_rsrc(
          (void*)(static_cast<const bf16*>(base) + (long)kvh * sh + (long)k0 * p.k_ss), (short)0, bytes, kBufferFlags);
    };
    // Copy instruction n (rows 4 n .. 4 n + 3) of a tile to the LDS tile at dst.
    auto copy1 = [&](__amdgpu_buffer_rsrc_t rs, unsigned dst, int n) __attribute__((always_inline)) {
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, lds_ptr(dst + n * 1024), 16, dkv[n & 3], (n >> 2) * kv_row32, 0, 0);
    };
    auto copy = [&](const void* base, long sh, int j, unsigned dst) __attribute__((always_inline)) {
      const __amdgpu_buffer_rsrc_t rs = tile_rsrc(base, sh, j);
#pragma unroll
      for (int n = 0; n < 8; ++n) copy1(rs, dst, n);
    };
    auto copy_k = [&](int j, int buf) __attribute__((always_inline)) { copy(p.k, p.k_sh, j, wb + buf * KS_TILEB); };
    auto copy_v = [&](int j, int buf) __attribute__((always_inline)) {
      copy(p.v, p.v_sh, j, wb + KS_VOFF + buf * KS_TILEB);
    };

    // ---- prologue: Q (4 copies per wavefront), K(0), K(1), V(0)
    {
      const int nrows = min(KS_QB, S - q0);
      const int bytes = (int)(2u * ((unsigned)(nrows - 1) * (unsigned)p.q_ss + (unsigned)dlim));
      const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc(
          (void*)(static_cast<const bf16*>(p.q) + (long)hh * p.q_sh + (long)q0 * p.q_ss), (short)0, bytes,
          kBufferFlags);
#pragma unroll
      for (int u = 0; u < 4; ++u) {  // rows 16 wq + 4 u + l / 16 of the block
        const int row = 4 * u + (lane >> 4);
        const int lc = (lane & 15) ^ row_swz(row);
        const int dq = lc * 8 < dlim ? (int)(2u * ((unsigned)row * (unsigned)p.q_ss + 8u * lc)) : 0x40000000;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rq, lds_ptr(lds0 + KS_QOFF + (4 * wq + u) * 1024), 16, dq,
                                                 wq * 32 * (int)p.q_ss, 0, 0);
      }
    }
    auto mask_max = [&](int j, int hq, floatx16& sc) __attribute__((always_inline)) {
      const int k0 = (t0 + wq + 4 * j) * KS_BN;
      const int lim = min(q0 + 32 * hq + l32, klim_seg - 1);  // last key this query may see
      float mx = -INFINITY;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        sc[e] = k0 + 8 * (e >> 2) + 4 * h32 + (e & 3) > lim ? -INFINITY : sc[e];
        mx = fmaxf(mx, sc[e]);
      }
      return mx;
    };
    auto plain_max = [&](const floatx16& sc) __attribute__((always_inline)) {
      float mx = fmaxf(sc[0], sc[1]);
#pragma unroll
      for (int e = 2; e < 16; ++e) mx = fmaxf(mx, sc[e]);
      return mx;
    };
    auto to_p = [&](const floatx16& sc, int uu, bf16x8& pf) __attribute__((always_inline)) {
#pragma unroll
      for (int j = 0; j < 8; ++j) pf[j] = round16<H>(sc[8 * uu + j]);
    };

    bf16x8 qf[2][NQF], kf[NQF], k2[NQF], va[NDB][2], v2[NDB][2];
    floatx16 s0[2], s1[2];
    // V^T fragments of the V tile in buffer PAR.
    auto read_v = [&](auto par, bf16x8 (&v)[NDB][2]) __attribute__((always_inline)) {
      constexpr int PAR = decltype(par)::value;
#pragma unroll
      for (int db = 0; db < NDB; ++db) {
        const shortx4 x0 = ds_tr64_db<PAR * KS_TILEB>(vbase[0], db);
        const shortx4 y0 = ds_tr64_db<PAR * KS_TILEB>(vbase[1], db);
        const shortx4 x1 = ds_tr64_db<PAR * KS_TILEB + 4096>(vbase[0], db);
        const shortx4 y1 = ds_tr64_db<PAR * KS_TILEB + 4096>(vbase[1], db);
        v[db][0] = __builtin_bit_cast(bf16x8, __builtin_shufflevector(x0, y0, 0, 1, 2, 3, 4, 5, 6, 7));
        v[db][1] = __builtin_bit_cast(bf16x8, __builtin_shufflevector(x1, y1, 0, 1, 2, 3, 4, 5, 6, 7));
      }
    };
    auto tie_v = [&](bf16x8 (&v)[NDB][2]) __attribute__((always_inline)) {
#pragma unroll
      for (int db = 0; db < NDB; ++db) {
        lds_wait_tie(v[db][0]);
        lds_wait_tie(v[db][1]);
      }
    };
    float m_run[2], l_run[2];
    floatx16 oacc[2][NDB];
    // K(0), K(1) and V(0) go out with Q, so that their latencies overlap:
    // one wait for Q and K(0), the others land during S(0).
    copy_k(0, 0);
    copy_k(1, 1);
    copy_v(0, 0);
    wait_vm<16>();                 // Q and K(0) have landed (K(1), V(0) in flight)
    __builtin_amdgcn_s_barrier();  // ... for every wavefront (Q)
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    {
      bf16x8 k0f[NQF];
#pragma unroll
      for (int f = 0; f < NQF; ++f) {
        qf[0][f] = ds_b128_acc_f<0>(qbase, f);
        qf[1][f] = ds_b128_acc_f<32 * KS_ROWB>(qbase, f);
      }
#pragma unroll
      for (int f = 0; f < NQF; ++f) k0f[f] = ds_b128_f<0>(kbase, f);
#pragma unroll
      for (int f = 0; f < NQF; ++f) {
        lds_wait_tie_acc(qf[0][f]);
        lds_wait_tie_acc(qf[1][f]);
        lds_wait_tie(k0f[f]);
      }
      // S(0), with the copies of K(2) into K buffer 0 (its fragments are in
      // registers) one per odd MFMA; O starts at zero (MFMAs of zeros, so that
      // O is made in the registers it stays in).
      const __amdgpu_buffer_rsrc_t rk2 = tile_rsrc(p.k, p.k_sh, 2);
#pragma unroll
      for (int k = 0; k < 2 * NQF; ++k) {
        if (k < 2)
          qk_first<H>(s0[k & 1], k0f[k >> 1], qf[k & 1][k >> 1]);
        else
          qk_acc<H>(s0[k & 1], k0f[k >> 1], qf[k & 1][k >> 1]);
        if (k & 1) copy1(rk2, wb, k >> 1);
      }
      o_zero<H>(oacc);
      wait_vm<16>();  // K(1) has landed (V(0), K(2) in flight)
#pragma unroll
      for (int f = 0; f < NQF; ++f) kf[f] = ds_b128_f<KS_TILEB>(kbase, f);
#pragma unroll
      for (int f = 0; f < NQF; ++f) lds_wait_tie(kf[f]);
      wait_vm<8>();  // V(0) has landed
      read_v(std::integral_constant<int, 0>{}, va);
      tie_v(va);
      // V buffer 0 and K buffer 1 are free: V(1), K(3).  In flight from here:
      // K(2), V(1), K(3).
      copy_v(1, 1);
      copy_k(3, 1);
      qk_settle(s0);
    }
    {  // the running max starts at the first tile's (O and l are zero)
      const bool msk = jm == 0;
#pragma unroll
      for (int hq = 0; hq < 2; ++hq) {
        m_run[hq] = max_xor32(msk ? mask_max(0, hq, s0[hq]) : plain_max(s0[hq])) * c;
        l_run[hq] = 0.f;
      }
    }
    // Raises the running maxima when a tile's max exceeds one by the slack
    // (rescaling O and l after the P V of the previous tile).
    auto rescale = [&](float (&mx)[2]) __attribute__((always_inline)) {
      bool up = false;
#pragma unroll
      for (int hq = 0; hq < 2; ++hq) {
        mx[hq] = max_xor32(mx[hq]) * c;
        up = up || mx[hq] > m_run[hq] + kRescaleSlack;
      }
      if (__builtin_amdgcn_ballot_w64(up)) {
        o_settle(oacc);
#pragma unroll
        for (int hq = 0; hq < 2; ++hq) {
          const float m_new = fmaxf(m_run[hq], mx[hq]);
          const float corr = m_run[hq] == -INFINITY ? 0.f : fast_exp2(m_run[hq] - m_new);
          m_run[hq] = m_new;
          l_run[hq] *= corr;
#pragma unroll
          for (int db = 0; db < NDB; ++db)
#pragma unroll
            for (int e = 0; e < 16; ++e) oacc[hq][db][e] *= corr;
        }
      }
    };

    // Step i: P V of tile i, S of tile i+1.  PAR = i % 2.  On entry kc holds
    // the K(i+1) fragments and vc the V(i) fragments; K buffer PAR holds
    // K(i+2), V buffer 1 - PAR V(i+1), K buffer 1 - PAR K(i+3), the copies of
    // those three still in flight in that order, and V buffer PAR is free.
    // The step copies V(i+2) into V buffer PAR during region 1, reads the
    // K(i+2) fragments into kn during region 2 and the V(i+1) fragments into
    // vn during region 3, where it copies K(i+4) into K buffer PAR.  The
    // copies go one per MFMA or two: a burst of them would hold the
    // wavefront's issue while the address unit drains it.  Every MFMA is an
    // asm statement and the VALU work and copies between two of them are
    // pinned there, so the interleave below is the instruction order.
    auto step = [&](auto par, auto masked, int i, floatx16 (&sc)[2], floatx16 (&sn)[2], const bf16x8 (&kc)[NQF],
                    bf16x8 (&kn)[NQF], const bf16x8 (&vc)[NDB][2], bf16x8 (&vn)[NDB][2])
                    __attribute__((always_inline)) {
      constexpr int PAR = decltype(par)::value;
      constexpr bool MSK = decltype(masked)::value;
      constexpr std::integral_constant<int, 1 - PAR> kNext{};
      float mneg[2], rs[2][2];
#pragma unroll
      for (int hq = 0; hq < 2; ++hq) {
        mneg[hq] = m_run[hq] == -INFINITY ? 0.f : -m_run[hq];  // an empty row keeps exp2(-inf) = 0
        rs[hq][0] = rs[hq][1] = 0.f;
      }
      bf16x8 pf[2][2];
      // The exp work of S(i) runs as a two-stage pipeline over the MFMA
      // slots: a slot issues the scaled exps of its scores and the row-sum
      // adds of the previous slot's, so that no VALU instruction waits on the
      // one just before it.  Scores: half 0 in slots 0-15 (one each), half 1
      // in the even slots 0-14 and slots 16-23 of region 2.
      float xe[2][16];
      auto ex_issue = [&](floatx16& s, int hq, int e) __attribute__((always_inline)) {
        float x = fmaf(s[e], c, mneg[hq]);
        pin(x);
        x = fast_exp2(x);
        pin(x);
        xe[hq][e] = x;
      };
      auto ex_sum = [&](floatx16& s, int hq, int e) __attribute__((always_inline)) {
        rs[hq][e & 1] += xe[hq][e];
        pin(rs[hq][e & 1]);
        s[e] = xe[hq][e];
      };
      auto cvt = [&](const floatx16& s, int uu, bf16x8& p) __attribute__((always_inline)) {
        to_p(s, uu, p);
        pin(p);
      };
      // ---- region 1: S(i+1) x exp of S(i) x V(i+2) copies -- MFMA k (d-step
      // k / 2, half k % 2), then the exp work of slot k and for odd k copy
      // instruction k / 2.
      const __amdgpu_buffer_rsrc_t rv = tile_rsrc(p.v, p.v_sh, i + 2);
      const unsigned vdst = wb + KS_VOFF + PAR * KS_TILEB;
#pragma unroll
      for (int k = 0; k < 2 * NQF; ++k) {
        if (k < 2)
          qk_first<H>(sn[k & 1], kc[k >> 1], qf[k & 1][k >> 1]);
        else
          qk_acc<H>(sn[k & 1], kc[k >> 1], qf[k & 1][k >> 1]);
        ex_issue(sc[0], 0, k);
        if ((k & 1) == 0) ex_issue(sc[1], 1, k >> 1);
        if (k > 0) {
          ex_sum(sc[0], 0, k - 1);
          if (((k - 1) & 1) == 0) ex_sum(sc[1], 1, (k - 1) >> 1);
        }
        if (k & 1) copy1(rv, vdst, k >> 1);
        if (k == 8) cvt(sc[0], 0, pf[0][0]);
      }
      wait_vm<24>();  // K(i+2) has landed
#pragma unroll
      for (int f = 0; f < NQF; ++f) kn[f] = ds_b128_f<PAR * KS_TILEB>(kbase, f);
      // ---- region 2: O(half 0) += P V x exp of half 1's last 8 scores
#pragma unroll
      for (int k = 0; k < 2 * NDB; ++k) {
        pv_acc<H>(oacc[0][k >> 1], vc[k >> 1][k & 1], pf[0][k & 1]);
        ex_issue(sc[1], 1, 8 + k);
        if (k == 0) {
          ex_sum(sc[0], 0, 15);
          cvt(sc[0], 1, pf[0][1]);  // for the second MFMA of this region
        } else {
          ex_sum(sc[1], 1, 7 + k);
        }
        if (k == 1) cvt(sc[1], 0, pf[1][0]);
      }
      ex_sum(sc[1], 1, 15);
      cvt(sc[1], 1, pf[1][1]);
#pragma unroll
      for (int f = 0; f < NQF; ++f) lds_wait_tie(kn[f]);  // K buffer PAR is free
      wait_vm<16>();  // V(i+1) has landed
      read_v(kNext, vn);
      // ---- region 3: O(half 1) += P V x (mask and) max of S(i+1) x K(i+4)
      // copies, one per MFMA
      const __amdgpu_buffer_rsrc_t rk = tile_rsrc(p.k, p.k_sh, i + 4);
      const unsigned kdst = wb + PAR * KS_TILEB;
      const int k0 = (t0 + wq + 4 * (i + 1)) * KS_BN;
      float mx[2] = {-INFINITY, -INFINITY};
#pragma unroll
      for (int k = 0; k < 2 * NDB; ++k) {
        pv_acc<H>(oacc[1][k >> 1], vc[k >> 1][k & 1], pf[1][k & 1]);
        copy1(rk, kdst, k);
#pragma unroll
        for (int hq = 0; hq < 2; ++hq) {
          if constexpr (MSK) {
            const int lim = min(q0 + 32 * hq + l32, klim_seg - 1);  // last key this query may see
#pragma unroll
            for (int e = 2 * k; e < 2 * k + 2; ++e) {
              float x = k0 + 8 * (e >> 2) + 4 * h32 + (e & 3) > lim ? -INFINITY : sn[hq][e];
              pin(x);
              sn[hq][e] = x;
            }
          }
          mx[hq] = max3(mx[hq], sn[hq][2 * k], sn[hq][2 * k + 1]);
        }
      }
#pragma unroll
      for (int hq = 0; hq < 2; ++hq) l_run[hq] += rs[hq][0] + rs[hq][1];
      tie_v(vn);
      rescale(mx);
    };

    constexpr std::integral_constant<int, 0> kEven{};
    constexpr std::integral_constant<int, 1> kOdd{};
    constexpr std::integral_constant<bool, false> kPlain{};
    constexpr std::integral_constant<bool, true> kMasked{};
    int i = 0;
    // Steps whose S(i+1) and S(i+2) need no mask, two at a time; then the rest.
#pragma unroll 1
    for (; i + 2 < jm; i += 2) {
      step(kEven, kPlain, i, s0, s1, kf, k2, va, v2);
      step(kOdd, kPlain, i + 1, s1, s0, k2, kf, v2, va);
    }
#pragma unroll 1
    for (; i < ntw; i += 2) {
      step(kEven, kMasked, i, s0, s1, kf, k2, va, v2);
      if (i + 1 >= ntw) break;
      step(kOdd, kMasked, i + 1, s1, s0, k2, kf, v2, va);
    }
    // A split block's arrival count, read now so that its latency overlaps the
    // exchange below (only thread 0's value is used).
    int arrived = 0;
    if (w.sched == kBalanced && tid == 0) arrived = __hip_atomic_load(&w.count[hh * w.nqb + b], __ATOMIC_RELAXED,
                                                                      __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_s_waitcnt(0);  // every copy (the tiles past the segment too) has landed
    o_settle(oacc);
    __syncthreads();

    // ---- combine the four wavefronts' states through LDS
    float l_tot[2];
#pragma unroll
    for (int hq = 0; hq < 2; ++hq) l_tot[hq] = sum_xor32(l_run[hq]);
    float2* xml = reinterpret_cast<float2*>(lds + KS_XML);
    if (h32 == 0) {
#pragma unroll
      for (int hq = 0; hq < 2; ++hq) xml[(wq * 2 + hq) * 32 + l32] = make_float2(m_run[hq], l_tot[hq]);
    }
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
      if (db == wq) continue;
      float4* slot = reinterpret_cast<float4*>(lds + KS_XO + (3 * wq + (db < wq ? db : db - 1)) * KS_XSLOT);
#pragma unroll
      for (int hq = 0; hq < 2; ++hq)
#pragma unroll
        for (int k4 = 0; k4 < 4; ++k4)
          slot[(4 * hq + k4) * 64 + lane] = make_float4(oacc[hq][db][4 * k4], oacc[hq][db][4 * k4 + 1],
                                                        oacc[hq][db][4 * k4 + 2], oacc[hq][db][4 * k4 + 3]);
    }
    __syncthreads();
    float M[2], L[2], a[KS_NW][2];
#pragma unroll
    for (int hq = 0; hq < 2; ++hq) {
      float mv[KS_NW], lv[KS_NW];
#pragma unroll
      for (int v = 0; v < KS_NW; ++v) {
        const float2 ml = xml[(v * 2 + hq) * 32 + l32];
        mv[v] = ml.x;
        lv[v] = ml.y;
      }
      M[hq] = fmaxf(fmaxf(mv[0], mv[1]), fmaxf(mv[2], mv[3]));
      L[hq] = 0.f;
#pragma unroll
      for (int v = 0; v < KS_NW; ++v) {
        a[v][hq] = mv[v] == -INFINITY ? 0.f : fast_exp2(mv[v] - M[hq]);
        L[hq] = fmaf(lv[v], a[v][hq], L[hq]);
      }
    }
    // Wavefront wq finishes d-block wq: the four states folded in wavefront order.
    floatx16 fin[2];
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
      if (db != wq) continue;
#pragma unroll
      for (int hq = 0; hq < 2; ++hq) {
#pragma unroll
        for (int e = 0; e < 16; ++e) fin[hq][e] = 0.f;
#pragma unroll
        for (int v = 0; v < KS_NW; ++v) {
          if (v == db) {
#pragma unroll
            for (int e = 0; e < 16; ++e) fin[hq][e] = fmaf(oacc[hq][db][e], a[v][hq], fin[hq][e]);
          } else {
            const float4* slot =
                reinterpret_cast<const float4*>(lds + KS_XO + (3 * v + (db < v ? db : db - 1)) * KS_XSLOT);
#pragma unroll
            for (int k4 = 0; k4 < 4; ++k4) {
              const float4 x = slot[(4 * hq + k4) * 64 + lane];
              fin[hq][4 * k4] = fmaf(x.x, a[v][hq], fin[hq][4 * k4]);
              fin[hq][4 * k4 + 1] = fmaf(x.y, a[v][hq], fin[hq][4 * k4 + 1]);
              fin[hq][4 * k4 + 2] = fmaf(x.z, a[v][hq], fin[hq][4 * k4 + 2]);
              fin[hq][4 * k4 + 3] = fmaf(x.w, a[v][hq], fin[hq][4 * k4 + 3]);
            }
          }
        }
      }
    }

    auto store_out = [&]() __attribute__((always_inline)) {
#pragma unroll
      for (int hq = 0; hq < 2; ++hq) {
        const float linv = 1.0f / L[hq];
        const int myq = q0 + 32 * hq + l32;
        if (myq < S) {
          bf16* orow = static_cast<bf16*>(p.o) + (long)hh * p.o_sh + (long)myq * p.o_ss;
#pragma unroll
          for (int k4 = 0; k4 < 4; ++k4) {
            const int dd = 32 * wq + 8 * k4 + 4 * h32;
            if (dd < dlim) {
              uint2 t;
              t.x = (unsigned)__builtin_bit_cast(unsigned short, round16<H>(fin[hq][4 * k4] * linv)) |
                    ((unsigned)__builtin_bit_cast(unsigned short, round16<H>(fin[hq][4 * k4 + 1] * linv)) << 16);
              t.y = (unsigned)__builtin_bit_cast(unsigned short, round16<H>(fin[hq][4 * k4 + 2] * linv)) |
                    ((unsigned)__builtin_bit_cast(unsigned short, round16<H>(fin[hq][4 * k4 + 3] * linv)) << 16);
              *reinterpret_cast<uint2*>(orow + dd) = t;
            }
          }
        }
      }
    };

    int nparts = 1, vf = vidx;
    if (w.sched == kBalanced) {
      vf = range_of_t<int>((int)bstart, w);
      nparts = range_of_t<int>((int)bstart + nt_b - 1, w) - vf + 1;
    }
    if (nparts == 1) {
      store_out();
    } else {
      typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
      int* const cnt = &w.count[hh * w.nqb + b];
      const __amdgpu_buffer_rsrc_t prs = __builtin_amdgcn_make_buffer_rsrc(w.part, (short)0, w.part_bytes, kBufferFlags);
      // Byte offsets in the workspace: part (v, slot), d-block db chunk k, or (m, l) of half hq.
      auto obyte = [&](int v, int s2, int db, int k) __attribute__((always_inline)) {
        return 4 * ((v * 2 + s2) * KS_PARTF + db * KS_PDB + (k * 64 + lane) * 4);
      };
      auto mlbyte = [&](int v, int s2, int hq) __attribute__((always_inline)) {
        return 4 * ((v * 2 + s2) * KS_PARTF + 4 * KS_PDB + (hq * 64 + lane) * 4);
      };
      const int slot = range_start_t<int>(vidx, w) >= bstart ? 0 : 1;
      // Every other part has already arrived (the count was read before the
      // exchange): merge without storing this one.
      if (tid == 0) flag = arrived == nparts - 1;
      __syncthreads();
      if (!flag) {
#pragma unroll
        for (int hq = 0; hq < 2; ++hq)
#pragma unroll
          for (int k4 = 0; k4 < 4; ++k4)
            __builtin_amdgcn_raw_buffer_store_b128(
                __builtin_bit_cast(u32x4, make_float4(fin[hq][4 * k4], fin[hq][4 * k4 + 1], fin[hq][4 * k4 + 2],
                                                      fin[hq][4 * k4 + 3])),
                prs, obyte(vidx, slot, wq, 4 * hq + k4), 0, kDeviceCoherent);
        if (wq == 0) {
#pragma unroll
          for (int hq = 0; hq < 2; ++hq)
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, make_float4(M[hq], L[hq], 0.f, 0.f)),
                                                   prs, mlbyte(vidx, slot, hq), 0, kDeviceCoherent);
        }
        __builtin_amdgcn_s_waitcnt(0);  // the state is stored (device-coherent) before the arrival
        __syncthreads();
        if (tid == 0) flag = atomicAdd(cnt, 1) == nparts - 1;
        __syncthreads();
      }
      if (flag) {
        // Fold every part into a running state in range order (this one from
        // registers): the largest max so far, the sum and O rescaled to it.
        // The other parts' chunks for this lane -- (m, l) of both halves and
        // d-block wq of O, ten 1 KB chunks per wavefront and part -- are
        // copied by the buffer unit into this wavefront's K/V buffers (free
        // after the exchange), KS_MB parts per memory round trip, and read
        // back from there: no registers held for them.
        const int vl = vf + nparts - 1;
        float Mt[2] = {-INFINITY, -INFINITY}, Lt[2] = {0.f, 0.f};
        floatx16 acc[2];
#pragma unroll
        for (int hq = 0; hq < 2; ++hq)
#pragma unroll
          for (int e = 0; e < 16; ++e) acc[hq][e] = 0.f;
        // Folds a part with maxima m2, sums l2 and O chunks getx(hq, k4).
        auto fold = [&](const float (&m2)[2], const float (&l2)[2], auto getx) __attribute__((always_inline)) {
#pragma unroll
          for (int hq = 0; hq < 2; ++hq) {
            const float Mn = fmaxf(Mt[hq], m2[hq]);
            const float a1 = Mt[hq] == -INFINITY ? 0.f : fast_exp2(Mt[hq] - Mn);
            const float a2 = m2[hq] == -INFINITY ? 0.f : fast_exp2(m2[hq] - Mn);
            Mt[hq] = Mn;
            Lt[hq] = fmaf(l2[hq], a2, Lt[hq] * a1);
#pragma unroll
            for (int k4 = 0; k4 < 4; ++k4) {
              const float4 x = getx(hq, k4);
              acc[hq][4 * k4] = fmaf(x.x, a2, acc[hq][4 * k4] * a1);
              acc[hq][4 * k4 + 1] = fmaf(x.y, a2, acc[hq][4 * k4 + 1] * a1);
              acc[hq][4 * k4 + 2] = fmaf(x.z, a2, acc[hq][4 * k4 + 2] * a1);
              acc[hq][4 * k4 + 3] = fmaf(x.w, a2, acc[hq][4 * k4 + 3] * a1);
            }
          }
        };
        // Staging of part i of a batch: chunk j (j < 8: O chunk 4 hq + k4;
        // 8, 9: (m, l) of half j - 8) at stg + (10 i + j) KB, lane l's 16
        // bytes at + 16 l.
        const unsigned stg = wb;
        const float4* stgp = reinterpret_cast<const float4*>(lds + wq * KS_WAVEB) + lane;
#pragma unroll 1
        for (int v0 = vf; v0 <= vl; v0 += KS_MB) {
#pragma unroll
          for (int i = 0; i < KS_MB; ++i) {
            const int v2 = v0 + i;
            if (v2 <= vl && v2 != vidx) {
              const int s2 = range_start_t<int>(v2, w) >= bstart ? 0 : 1;
#pragma unroll
              for (int j = 0; j < 10; ++j) {
                // (The offset and the LDS address go through locals: written
                // inline in the builtin's arguments they made the host pass
                // drop this kernel's launch stub without a diagnostic.)
                const int off = j < 8 ? obyte(v2, s2, wq, j) : mlbyte(v2, s2, j - 8);
                const unsigned dst = stg + (10 * i + j) * 1024;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(prs, lds_ptr(dst), 16, off, 0, 0, kDeviceCoherent);
              }
            }
          }
          __builtin_amdgcn_s_waitcnt(0);  // the batch has landed in LDS
          __atomic_signal_fence(__ATOMIC_SEQ_CST);
#pragma unroll
          for (int i = 0; i < KS_MB; ++i) {
            const int v2 = v0 + i;
            if (v2 > vl) continue;
            if (v2 == vidx) {
              fold(M, L, [&](int hq, int k4) __attribute__((always_inline)) {
                return make_float4(fin[hq][4 * k4], fin[hq][4 * k4 + 1], fin[hq][4 * k4 + 2], fin[hq][4 * k4 + 3]);
              });
            } else {
              const float4 ml0 = stgp[(10 * i + 8) * 64], ml1 = stgp[(10 * i + 9) * 64];
              const float m2[2] = {ml0.x, ml1.x}, l2[2] = {ml0.y, ml1.y};
              fold(m2, l2, [&](int hq, int k4) __attribute__((always_inline)) {
                return stgp[(10 * i + 4 * hq + k4) * 64];
              });
            }
          }
          __atomic_signal_fence(__ATOMIC_SEQ_CST);
          __builtin_amdgcn_s_waitcnt(0xC07F);  // the batch is read before the next one lands (lgkmcnt(0))
        }
#pragma unroll
        for (int hq = 0; hq < 2; ++hq) {
          L[hq] = Lt[hq];
          fin[hq] = acc[hq];
        }
        store_out();
        if (tid == 0) __hip_atomic_store(cnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }

    const long next_u = bstart + t0 - 1;  // the last unit of the previous segment
    if (next_u < u0) break;
    cur = decode_seg_t<int>((int)next_u, u0, w);
    __syncthreads();  // the exchange area is read before the next segment's copies land there
  }
}

// ------------------------------------------------------------------ host --

size_t flash_ks_part_bytes() { return (size_t)KS_PARTF * 4; }

void launch_flash_ks(const AttnArgs& a, const Work& w, hipStream_t st) {
  if (a.f16)
    flash_ks_kernel<true><<<dim3((unsigned)w.grid), dim3(64 * KS_NW), 0, st>>>(a, w);
  else
    flash_ks_kernel<false><<<dim3((unsigned)w.grid), dim3(64 * KS_NW), 0, st>>>(a, w);
}

}  // namespace nkl
