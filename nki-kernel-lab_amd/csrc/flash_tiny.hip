// bf16 / fp16 causal flash attention for gfx950, 64 < d <= 128 and S <= 256:
// the one-pass kernel for short sequences.
//
// One workgroup per (head, 128-query block), the heavier block first; four
// wavefronts compute, wavefront w owning queries 128 b + 32 w .. + 31, and
// four more only help issue the copies.
// Every key row the block can see (at most 256, whole 32-key tiles) is copied
// global -> LDS at once by the buffer unit (buffer_load ... lds: lane l's 16
// bytes land at the instruction's LDS base + 16 l), K rows then V rows, 256
// bytes each with their 16-byte chunks swizzled (logical chunk c of row r at
// c ^ fsched::row_swz(r)), behind one barrier.  Each wavefront then runs the
// online softmax over its own key tiles, 0 .. its diagonal, reading K and V^T
// fragments from LDS with no further synchronisation, and writes its 32 rows
// of O.  Nothing is handed over between wavefronts and no partial state
// leaves the workgroup: a launch is one load phase, one loop and one store.
//
// Per wavefront and tile, with 32x32x16 MFMAs (H: the fp16 form):
//     S^T[32 keys x 32 queries] = K . Q^T       8 MFMAs, Q^T in registers
//     O^T[128 d x 32 queries]  += V^T . P^T     8 MFMAs, V^T from transposed
//                                               LDS reads (ds_read_b64_tr_b16)
// Lane l holds query l % 32; its 16 scores are keys 8 (i / 4) + 4 (l / 32) +
// i % 4 of the tile.  The running max is raised lazily (fsched::kRescaleSlack)
// and P is rounded to the 16-bit operand format before P V, as in the other
// kernels of this library, so results agree with theirs to rounding.
#include <math.h>

#include "attention.h"
#include "flash_sched.h"

namespace nkl {

namespace {

using namespace fsched;

constexpr int TY_BN = 32;                     // keys per tile
constexpr int TY_QB = 128;                    // queries per block
constexpr int TY_NW = 4;                      // wavefronts that compute
constexpr int TY_NC = 8;                      // wavefronts that copy (the last four only copy)
constexpr int TY_ROWB = 256;                  // bytes of a 128-element 16-bit row
constexpr int TY_VOFF = kTinyMaxS * TY_ROWB;  // V rows follow the K rows
constexpr int TY_LDS = 2 * TY_VOFF;           // 128 KB

// One V^T operand fragment from two transposed 8-byte LDS reads (rows a, b).
__device__ __forceinline__ bf16x8 read_vt16(const unsigned char* a, const unsigned char* b) {
  typedef __attribute__((address_space(3))) shortx4 lds_s4;
  const shortx4 x = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)(a));
  const shortx4 y = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)(b));
  return __builtin_bit_cast(bf16x8, __builtin_shufflevector(x, y, 0, 1, 2, 3, 4, 5, 6, 7));
}

}  // namespace

template <bool H>
__global__ __launch_bounds__(64 * TY_NC) void flash_tiny_kernel(AttnArgs p) {
  prefetch_kernargs<sizeof(AttnArgs)>();
  constexpr int D = 128, NQF = D / 16, NDB = D / 32;
  __shared__ __align__(16) unsigned char lds[TY_LDS];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wq = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int h32 = lane >> 5, l32 = lane & 31;
  const int S = p.S, dlim = p.d;
  const float c = p.c;
  const int nqb = (S + TY_QB - 1) / TY_QB;
  const int hh = (int)(blockIdx.x % (unsigned)p.H);
  const int b = nqb - 1 - (int)(blockIdx.x / (unsigned)p.H);  // the heavier block first
  const int nk = min(S, TY_QB * (b + 1));                     // keys the block can see
  const int nrow = (nk + TY_BN - 1) / TY_BN * TY_BN;          // rows staged: whole tiles, rows past nk read as 0

  // ---- every K and V row of the block into LDS.  Copy n (rows 4 n .. 4 n + 3,
  // 1 KB) is wavefront n % 8's (a wavefront issues a copy every ~80 ns, so
  // eight share them); lane l fills row 4 n + l / 16, physical chunk
  // l % 16, which holds logical chunk (l % 16) ^ row_swz(row).  Chunks past d
  // get an offset past the buffer's range and read as zeros.
  {
    const int kvh = hh / p.group;
    const int kbytes = 2 * ((nk - 1) * (int)p.k_ss + dlim);
    const int vbytes = 2 * ((nk - 1) * (int)p.v_ss + dlim);
    const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(static_cast<const bf16*>(p.k) + (long)kvh * p.k_sh), (short)0, kbytes, kBufferFlags);
    const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(static_cast<const bf16*>(p.v) + (long)kvh * p.v_sh), (short)0, vbytes, kBufferFlags);
    const unsigned kbase = opaque_lds_addr(lds);
    const unsigned vbase = kbase + TY_VOFF;
    const int ncopy = nrow / 4;
#pragma unroll 1
    for (int n = wq; n < ncopy; n += TY_NC) {
      const int row = 4 * n + (lane >> 4);
      const int lc = (lane & 15) ^ row_swz(row);
      const bool ok = lc * 8 < dlim;
      const int ko = ok ? 2 * (row * (int)p.k_ss + lc * 8) : 0x40000000;
      const int vo = ok ? 2 * (row * (int)p.v_ss + lc * 8) : 0x40000000;
      const unsigned kdst = kbase + (unsigned)n * 1024u;
      const unsigned vdst = vbase + (unsigned)n * 1024u;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, lds_ptr(kdst), 16, ko, 0, 0, 0);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, lds_ptr(vdst), 16, vo, 0, 0, 0);
    }
  }

  // ---- this wavefront's Q^T fragments, straight into registers.
  const int qw = TY_QB * b + 32 * wq;  // first query of this wavefront
  const int myq = qw + l32;
  bf16x8 qf[NQF];
  {
    const bf16* Q = static_cast<const bf16*>(p.q) + (long)hh * p.q_sh;
#pragma unroll
    for (int f = 0; f < NQF; ++f) {
      const int dd = 16 * f + 8 * h32;
      const bool ok = wq < TY_NW && myq < S && dd < dlim;  // copy-only wavefronts load none
      qf[f] = __builtin_bit_cast(bf16x8, ld16_or_zero(Q, (long)myq * p.q_ss + dd, ok));
    }
  }
  __builtin_amdgcn_s_waitcnt(0);  // this wavefront's copies (and Q) have landed
  __syncthreads();                // ... and every other wavefront's
  if (wq >= TY_NW || qw >= S) return;  // a copy-only wavefront, or one wholly past the sequence

  // Per-lane byte offsets of the MFMA operands within tile 0 (row_swz depends
  // on the row modulo 16, so every tile shares them).
  //   K fragment f: row l32, logical chunk 2 f + h32.
  int koff[NQF];
  {
    const int sw = row_swz(l32);
#pragma unroll
    for (int f = 0; f < NQF; ++f) koff[f] = l32 * TY_ROWB + (((2 * f + h32) ^ sw) << 4);
  }
  //   V^T fragment (d-block db, first or second 8-row read): rows r0 + 8 half
  //   (+ 16 uu: 4096 bytes), d = 32 db + 16 g2 + 4 (i16 % 4).
  int voff[NDB][2];
  {
    const int i16 = lane & 15, g2 = (lane >> 4) & 1;
    const int r0 = 4 * h32 + (i16 >> 2);
    const int cb = 2 * g2 + ((i16 & 3) >> 1);
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        const int row = r0 + 8 * half;
        voff[db][half] = TY_VOFF + row * TY_ROWB + (((4 * db + cb) ^ row_swz(row)) << 4) + (i16 & 1) * 8;
      }
  }

  float m_run = -INFINITY, l_run = 0.f;
  floatx16 oacc[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int e = 0; e < 16; ++e) oacc[db][e] = 0.f;

  const int ntw = min(nrow, qw + 32) / TY_BN;  // tiles up to this wavefront's diagonal
#pragma unroll 1
  for (int t = 0; t < ntw; ++t) {
    const unsigned char* tb = lds + t * (TY_BN * TY_ROWB);
    const int k0 = t * TY_BN;
    bf16x8 kf[NQF];
#pragma unroll
    for (int f = 0; f < NQF; ++f) kf[f] = *reinterpret_cast<const bf16x8*>(tb + koff[f]);
    floatx16 sc;
#pragma unroll
    for (int e = 0; e < 16; ++e) sc[e] = 0.f;
#pragma unroll
    for (int f = 0; f < NQF; ++f) sc = mma32_16b<H>(kf[f], qf[f], sc);
    // V^T fragments of the tile, read while the QK^T MFMAs run.
    bf16x8 va[NDB][2];
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int uu = 0; uu < 2; ++uu)
        va[db][uu] = read_vt16(tb + voff[db][0] + 4096 * uu, tb + voff[db][1] + 4096 * uu);

    // Online softmax: keys after the query masked on the diagonal tile.
    if (k0 + TY_BN - 1 > qw) {
#pragma unroll
      for (int e = 0; e < 16; ++e)
        if (k0 + 8 * (e >> 2) + 4 * h32 + (e & 3) > myq) sc[e] = -INFINITY;
    }
    float mloc = sc[0];
#pragma unroll
    for (int e = 1; e < 16; ++e) mloc = fmaxf(mloc, sc[e]);
    mloc = max_xor32(mloc) * c;
    if (__builtin_amdgcn_ballot_w64(mloc > m_run + kRescaleSlack)) {
      const float m_new = fmaxf(m_run, mloc);
      const float corr = fast_exp2(m_run - m_new);
      m_run = m_new;
      l_run *= corr;
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int e = 0; e < 16; ++e) oacc[db][e] *= corr;
    }
    float rs = 0.f;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      sc[e] = fast_exp2(fmaf(sc[e], c, -m_run));
      rs += sc[e];
    }
    l_run += rs;
    bf16x8 pf[2];
#pragma unroll
    for (int uu = 0; uu < 2; ++uu)
#pragma unroll
      for (int j = 0; j < 8; ++j) pf[uu][j] = round16<H>(sc[8 * uu + j]);
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int uu = 0; uu < 2; ++uu) oacc[db] = mma32_16b<H>(va[db][uu], pf[uu], oacc[db]);
  }

  // ---- O = O^T / l for this wavefront's 32 queries.  Lane l holds query
  // l % 32 and, per d-block, d = 32 db + 8 g + 4 (l / 32) + 0..3 for g = 0..3;
  // d and every stride are multiples of 8 elements and o is 16-byte aligned
  // (the entry points check), so each 4-element group is whole and 8-byte
  // aligned.
  if (myq >= S) return;
  const float linv = 1.0f / sum_xor32(l_run);  // lanes l and l ^ 32 hold the same query
  bf16* orow = static_cast<bf16*>(p.o) + (long)hh * p.o_sh + (long)myq * p.o_ss;
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int d0 = 32 * db + 8 * g + 4 * h32;
      bf16x4 v4;
#pragma unroll
      for (int e = 0; e < 4; ++e) v4[e] = round16<H>(oacc[db][4 * g + e] * linv);
      if (d0 < dlim) *reinterpret_cast<bf16x4*>(orow + d0) = v4;
    }
}

bool flash_tiny_fits(const AttnArgs& a) {
  return a.S >= 1 && a.S <= kTinyMaxS && a.d > 64 && a.d <= 128 && a.c > 0.f;
}

void launch_flash_tiny(const AttnArgs& a, hipStream_t st) {
  const int nqb = (a.S + TY_QB - 1) / TY_QB;
  const dim3 grid((unsigned)(a.H * nqb)), block(64 * TY_NC);
  if (a.f16)
    flash_tiny_kernel<true><<<grid, block, 0, st>>>(a);
  else
    flash_tiny_kernel<false><<<grid, block, 0, st>>>(a);
}

}  // namespace nkl
