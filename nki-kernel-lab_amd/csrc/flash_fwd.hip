// bf16 causal flash attention for gfx950, head dim in (64, 128]: the kernel
// behind the headline workload (8 heads x 2048 x 128).
//
// Decomposition.  Queries in blocks of QB = 128, keys in tiles of BN = 64; a
// unit is one (head, block, tile) at or below the diagonal, and the units are
// split over one 512-thread workgroup per CU by the balanced (stream-K)
// schedule of flash_sched.h.
//
// Workgroup.  Eight wavefronts, two per SIMD (256 registers each).  Wavefront
// w owns queries 32 (w % 4) .. + 31 of the block and key half kh = w / 4 of
// every tile (keys 32 kh .. 32 kh + 31), so the two wavefronts of a SIMD
// (w and w + 4) hold the same queries and split each tile's keys.  At the end
// of a segment they merge their two online-softmax states through LDS, each
// finishing half of the head dim.
//
// Per tile a wavefront computes, with 32x32x16 bf16 MFMAs,
//     S^T[32 keys x 32 queries] = K . Q^T        (8 MFMAs)
//     O^T[128 x 32 queries]    += V^T . P^T      (8 MFMAs)
// Lane l holds query l % 32 throughout.  Its 16 scores are keys
// 8 (i / 4) + 4 (l / 32) + i % 4 (i < 16) of the wavefront's half, so the
// probabilities of 16-key chunk u are elements 8 u .. 8 u + 7 -- already the
// B operand of the P V MFMA.  The V^T operand is read with ds_read_b64_tr_b16
// in the same key order.
//
// Pipeline.  K/V tiles are copied global -> LDS by the buffer unit
// (buffer_load ... lds) into NS = 4 stages, two tiles ahead of the tile being
// read, with one barrier per tile.  The K tiles of the four stages fill the
// first 64 KB of LDS and the V tiles the next 64 KB, so every fragment
// address is a per-lane register plus an instruction immediate.  Each
// wavefront overlaps its own MFMA and VALU work: the QK^T MFMAs of tile j+1
// run beside the exp, row sum and bf16 rounding of tile j (and the V^T reads
// of tile j), the P V MFMAs of tile j beside the (mask and) row max of tile
// j+1.
//
// Split blocks.  A block whose units span several workgroups is finished by
// the last to arrive, which folds every part's (max, sum, O) state in the
// fixed order of the parts' ranges, so the output does not depend on which
// part arrived last.
#include <math.h>

#include <type_traits>

#include "attention.h"
#include "flash_sched.h"

namespace nkl {

namespace {

using namespace fsched;

namespace fwd {
constexpr int QB = 128;                  // queries per block
constexpr int BN = 64;                   // keys per tile
constexpr int NS = 4;                    // LDS stages
constexpr int ROWB = 256;                // bytes of a K/V row (d = 128)
constexpr int TILEB = BN * ROWB;         // bytes of a K (or V) tile
constexpr int VOFF = NS * TILEB;         // V tiles after the four K tiles
constexpr int MLOFF = 2 * NS * TILEB;    // hand-over (max, sum) pairs: 512 bytes per wavefront
constexpr int LDS_BYTES = MLOFF + 8 * 64 * 8;
constexpr int PCH = 9;                   // float4 chunks per lane of a partial state: 8 of O, 1 of (m, l)
constexpr int PART_BYTES = 8 * PCH * 64 * 16;  // one workgroup's partial state of a block
constexpr int STG_PITCH = 72;            // bf16 elements per staged output row (64 + 8)
// Hand-over slot of wavefront w (8 KB): the K and V halves of stages 2 and 3.
__device__ __forceinline__ int xslot(int w) { return (w < 4 ? 2 * TILEB : VOFF + 2 * TILEB) + (w & 3) * 8192; }

// One 1 KB copy global -> LDS by the buffer unit: lane l's 16 bytes from
// rsrc + voffset land at LDS address lds_addr + 16 l.  Issued through inline
// assembly, so that the compiler does not see an LDS write by DMA: it would
// otherwise make every later LDS read wait for the copies it might alias
// (vmcnt), which keeps only one tile in flight.  The kernel orders copies and
// reads itself (per-tile vmcnt waits and barriers).  M0 carries the LDS
// address; nothing else in these kernels uses M0.
__device__ __forceinline__ void copy_1k(__amdgpu_buffer_rsrc_t rsrc, int voffset, unsigned lds_addr) {
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds"
               :
               : "v"(voffset), "s"(rsrc), "s"(lds_addr)
               : "memory", "m0");
#pragma clang diagnostic pop
}
typedef __attribute__((address_space(3))) shortx4 lds_shortx4;
template <int N>
using I = std::integral_constant<int, N>;
}  // namespace fwd

}  // namespace

template <bool PP, bool F = false>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
void flash_fwd_kernel(AttnArgs p, Work w) {
  using namespace fwd;
  using MF = Mfma32<bf16>;
  __shared__ __align__(16) unsigned char lds[LDS_BYTES];
  __shared__ int arrival;

  prefetch_kernargs<sizeof(AttnArgs) + sizeof(Work)>();
  const int tid = threadIdx.x, lane = tid & 63;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wq = wid & 3, kh = wid >> 2;
  const int h32 = lane >> 5, l32 = lane & 31;
  const int S = p.S, dlim = p.d;
  const float c = p.c;

  // ---- per-lane LDS byte offsets within stage 0 (stage s adds s * TILEB)
  // K fragment f: row 32 kh + l32, logical chunk 2 f + h32.
  int koff[8];
#pragma unroll
  for (int f = 0; f < 8; ++f) koff[f] = (32 * kh + l32) * ROWB + (((2 * f + h32) ^ row_swz(l32)) << 4);
  // V^T fragment of d-block db, 16-key chunk uu (+ 4096 bytes): two
  // transposed 8-byte reads, rows 32 kh + r0 (+ 8), d = 32 db + 16 g2 + 4 (i16 % 4).
  int voff[4][2];
  {
    const int i16 = lane & 15, g2 = (lane >> 4) & 1;
    const int r0 = 4 * h32 + (i16 >> 2);
    const int cb = 2 * g2 + ((i16 & 3) >> 1);
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        const int row = r0 + 8 * half;
        voff[db][half] = VOFF + (32 * kh + row) * ROWB + (((4 * db + cb) ^ row_swz(row)) << 4) + (i16 & 1) * 8;
      }
  }
  // ---- copies: wavefront w fills rows 8 w .. 8 w + 7 of each K and V tile
  // with two 1 KB copies each (copy n = 2 w + u covers rows 4 n .. 4 n + 3;
  // lane l fills row 4 n + l / 16, physical chunk l % 16).  Chunks past d
  // read as zero (offset past the buffer's range).
  int dk[2], dv[2];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int row = 4 * (2 * wid + u) + (lane >> 4);
    const int lc = (lane & 15) ^ row_swz(row);
    const bool ok = lc * 8 < dlim;
    dk[u] = ok ? 2 * (row * (int)p.k_ss + lc * 8) : 0x40000000;
    dv[u] = ok ? 2 * (row * (int)p.v_ss + lc * 8) : 0x40000000;
  }

  long u0, u1;
  const int vidx = wg_range_x<F>(w, p.H, u0, u1);

  bf16x8 qf[8];
  auto load_q = [&](const Seg& sg) __attribute__((always_inline)) {
    const bf16* Q = static_cast<const bf16*>(p.q) + (long)sg.hh * p.q_sh;
    const int qrow = QB * sg.b + 32 * wq + l32;
#pragma unroll
    for (int f = 0; f < 8; ++f) {
      const int dd = 16 * f + 8 * h32;
      qf[f] = __builtin_bit_cast(bf16x8, ld16_or_zero(Q, (long)qrow * p.q_ss + dd, qrow < S && dd < dlim));
    }
  };
  // A segment's K/V source: the first key of its first tile, and the keys
  // left from there to the end of the sequence (tiles past them read zeros).
  struct Src {
    const bf16* k;
    const bf16* v;
    int keys;
  };
  auto seg_src = [&](const Seg& sg) __attribute__((always_inline)) {
    const long kvh = (long)(sg.hh / p.group);
    const long k0 = (long)sg.t0 * BN;
    return Src{static_cast<const bf16*>(p.k) + kvh * p.k_sh + k0 * p.k_ss,
               static_cast<const bf16*>(p.v) + kvh * p.v_sh + k0 * p.v_ss, S - (int)k0};
  };
  const unsigned lds0 = (unsigned)(size_t)(const __attribute__((address_space(3))) void*)lds + 2048 * wid;
  // Copies tile j of a segment into LDS stage j % NS.
  auto dma = [&](const Src& src, int j) __attribute__((always_inline)) {
    const int nkeys = min(BN, src.keys - j * BN);
    const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(src.k + (long)j * BN * p.k_ss), (short)0, 2 * ((nkeys - 1) * (int)p.k_ss + dlim), kBufferFlags);
    const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(src.v + (long)j * BN * p.v_ss), (short)0, 2 * ((nkeys - 1) * (int)p.v_ss + dlim), kBufferFlags);
    const unsigned sbase = lds0 + (j % NS) * TILEB;
    copy_1k(rk, dk[0], sbase);
    copy_1k(rk, dk[1], sbase + 1024);
    copy_1k(rv, dv[0], sbase + VOFF);
    copy_1k(rv, dv[1], sbase + VOFF + 1024);
  };
  // Every wavefront's LDS reads are done, then all wavefronts meet.  A bare
  // barrier: __syncthreads()' fence would wait for every outstanding copy.
  auto bar = [&]() __attribute__((always_inline)) {
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
  };

  Seg cur = decode_seg_x<F>(u1 - 1, u0, w);
  Src src = seg_src(cur);
  if constexpr (PP) {
    // The first segment's Q block is copied once for the workgroup into the
    // K halves of stages 2 and 3 (16 rows per wavefront, swizzled like the K
    // rows), which no copy writes before the first tile's barrier; the two
    // wavefronts of each SIMD read their Q fragments from there.  (Loaded
    // into registers in the MFMA operand layout, each wavefront instruction
    // would touch 32 rows, and both wavefronts of a SIMD would load them.
    // Later segments load their Q while the previous segment ends.)
    const int qrows = max(0, min(QB, S - QB * cur.b));
    const __amdgpu_buffer_rsrc_t qsrc = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(static_cast<const bf16*>(p.q) + (long)cur.hh * p.q_sh + (long)QB * cur.b * p.q_ss), (short)0,
        qrows > 0 ? 2 * ((qrows - 1) * (int)p.q_ss + dlim) : 0, kBufferFlags);
    const unsigned qbase = (unsigned)(size_t)(const __attribute__((address_space(3))) void*)lds + 2 * TILEB + 4096 * wid;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int row = 4 * (4 * wid + u) + (lane >> 4);
      const int lc = (lane & 15) ^ row_swz(row);
      copy_1k(qsrc, lc * 8 < dlim ? 2 * (row * (int)p.q_ss + lc * 8) : 0x40000000, qbase + 1024 * u);
    }
    dma(src, 0);
    if (cur.t1 - cur.t0 > 1) {
      dma(src, 1);
      wait_vm<8>();  // this wavefront's Q copies have landed
    } else {
      wait_vm<4>();
    }
    bar();  // and every wavefront's; the first tile's barrier follows these reads
#pragma unroll
    for (int f = 0; f < 8; ++f)
      qf[f] = *reinterpret_cast<const bf16x8*>(lds + 2 * TILEB + (32 * wq + l32) * ROWB +
                                               (((2 * f + h32) ^ row_swz(l32)) << 4));
  } else {
    load_q(cur);
    dma(src, 0);
    if (cur.t1 - cur.t0 > 1) dma(src, 1);
  }

  for (;;) {
    const int hh = cur.hh, b = cur.b, t0 = cur.t0, nt = cur.t1 - cur.t0;
    const long bstart = cur.bstart;
    const int qw = QB * b + 32 * wq;  // this wavefront's first query
    const int qi = qw >> 5;
    // Tile j is active for this wavefront when its key half starts at or
    // before the wavefront's first query (2 (t0 + j) + kh <= qi), and masked
    // when the two coincide (the 32 x 32 diagonal square): only the last
    // active tile can be.
    const int lastj = (qi - kh >= 0 ? (qi - kh) >> 1 : -1) - t0;  // last active tile (may lie past the segment)
    const int nw = __builtin_amdgcn_readfirstlane(max(0, min(nt, lastj + 1)));
    const bool diag_in = ((qi - kh) & 1) == 0 && lastj >= 0 && lastj < nt;  // tile nw - 1 is the diagonal one

    if constexpr (!PP) {
      if (nt > 1)
        wait_vm<4>();  // Q and tile 0 have landed
      else
        wait_vm<0>();
      bar();
      if (nt > 2) dma(src, 2);
    }

    float m_run = -INFINITY, l_run = 0.f;
    floatx16 oacc[4];
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int e = 0; e < 16; ++e) oacc[db][e] = 0.f;

    // Fragment reads from stage st (an instruction immediate where st is a
    // compile-time constant).
    auto kfrag = [&](int st, int f) __attribute__((always_inline)) {
      return *reinterpret_cast<const bf16x8*>(lds + st * TILEB + koff[f]);
    };
    auto vfrag = [&](int st, int db, int uu) __attribute__((always_inline)) {
      const shortx4 x = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_shortx4*)(lds + st * TILEB + voff[db][0] + 4096 * uu));
      const shortx4 y = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_shortx4*)(lds + st * TILEB + voff[db][1] + 4096 * uu));
      return __builtin_bit_cast(bf16x8, __builtin_shufflevector(x, y, 0, 1, 2, 3, 4, 5, 6, 7));
    };
    // Keys of the diagonal square after this lane's query are masked (key
    // offset 8 (e / 4) + 4 h32 + e % 4 against query offset l32).
    auto mask_max = [&](floatx16& sc) __attribute__((always_inline)) {
      float mx = -INFINITY;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        sc[e] = 8 * (e >> 2) + 4 * h32 + (e & 3) > l32 ? -INFINITY : sc[e];
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
    // Raises the running max when the tile's max exceeds it by the slack,
    // rescaling O and l (after the P V of the previous tile).
    auto rescale = [&](float mx) __attribute__((always_inline)) {
      mx = max_xor32(mx) * c;
      if (__builtin_amdgcn_ballot_w64(mx > m_run + kRescaleSlack)) {
        const float m_new = fmaxf(m_run, mx);
        const float corr = m_run == -INFINITY ? 0.f : fast_exp2(m_run - m_new);
        m_run = m_new;
        l_run *= corr;
#pragma unroll
        for (int db = 0; db < 4; ++db)
#pragma unroll
          for (int e = 0; e < 16; ++e) oacc[db][e] *= corr;
      }
    };

    if constexpr (!PP) {
    floatx16 s_cur;
    bf16x8 va[4][2];  // V^T fragments of the tile being multiplied (read one step ahead)
    if (nw > 0) {
      bf16x8 kf[8];
#pragma unroll
      for (int f = 0; f < 8; ++f) kf[f] = kfrag(0, f);
#pragma unroll
      for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int uu = 0; uu < 2; ++uu) va[db][uu] = vfrag(0, db, uu);
#pragma unroll
      for (int e = 0; e < 16; ++e) s_cur[e] = 0.f;
#pragma unroll
      for (int f = 0; f < 8; ++f) s_cur = MF::mma(kf[f], qf[f], s_cur);
      rescale(nw == 1 && diag_in ? mask_max(s_cur) : plain_max(s_cur));
    }

    // One pipeline step for tile j (stage st = j % NS, a compile-time
    // constant): S(j+1) when `next` (tile j+1 is active for this wavefront),
    // masked when `msk` (tile j+1 is its diagonal tile).  Both are
    // compile-time constants in the steady state, wave-uniform run-time
    // values in the tail.
    auto step = [&](auto st_c, bool next, bool msk) __attribute__((always_inline)) {
      constexpr int st = decltype(st_c)::value, sn = (st + 1) % NS;
      bf16x8 kf[8];
      if (next) {
#pragma unroll
        for (int f = 0; f < 8; ++f) kf[f] = kfrag(sn, f);
      }
      __builtin_amdgcn_sched_barrier(0);
      const float mneg = m_run == -INFINITY ? 0.f : -m_run;
      floatx16 s_nxt;
      // ---- region 1: S(j+1) = K(j+1) Q^T  x  exp, row sum, bf16 P(j)
      if (next) {
#pragma unroll
        for (int e = 0; e < 16; ++e) s_nxt[e] = 0.f;
#pragma unroll
        for (int f = 0; f < 8; ++f) s_nxt = MF::mma(kf[f], qf[f], s_nxt);
      }
      float rs = 0.f;
      bf16x8 pf[2];
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const float pe = fast_exp2(fmaf(s_cur[e], c, mneg));
        rs += pe;
        pf[e >> 3][e & 7] = (bf16)pe;
      }
      if (next) {
#pragma unroll
        for (int f = 0; f < 8; ++f) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
          __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);  // VALU
        }
      }
      __builtin_amdgcn_sched_barrier(0);
      l_run += rs;
      // ---- region 2: O += P(j) V(j)  x  (mask and) row max of S(j+1), and
      // the V^T fragments of tile j+1 read into the registers each MFMA frees
#pragma unroll
      for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int uu = 0; uu < 2; ++uu) {
          oacc[db] = MF::mma(va[db][uu], pf[uu], oacc[db]);
          if (next) va[db][uu] = vfrag(sn, db, uu);
        }
      float mx = 0.f;
      if (next) {
        mx = msk ? mask_max(s_nxt) : plain_max(s_nxt);
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);
          __builtin_amdgcn_sched_group_barrier(0x100, 2, 1);
          __builtin_amdgcn_sched_group_barrier(0x002, 2, 1);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
      if (next) {
        rescale(mx);
        s_cur = s_nxt;
      }
    };
    // Top of iteration j: tile j+1 has landed (tile j+2 may be in flight) for
    // every wavefront, all are done with tile j-1's stage, which takes tile j+3.
    auto top = [&](int j) __attribute__((always_inline)) {
      if (j + 1 < nt) {
        if (j + 2 < nt)
          wait_vm<4>();
        else
          wait_vm<0>();
      }
      bar();
      if (j + 3 < nt) dma(src, j + 3);
    };

    // The tiles four at a time, so that the stages are compile-time
    // immediates.  Steady state: steps whose next tile is active and
    // unmasked (compile-time flags); then the rest, where whether a step
    // computes and masks the next tile's scores is a wave-uniform branch.
    const int nplain = __builtin_amdgcn_readfirstlane(max(0, nw - 1 - (diag_in ? 1 : 0)));
    int j = 0;
#pragma unroll 1
    for (; j + 4 <= nplain; j += 4) {
      top(j);
      step(I<0>{}, true, false);
      top(j + 1);
      step(I<1>{}, true, false);
      top(j + 2);
      step(I<2>{}, true, false);
      top(j + 3);
      step(I<3>{}, true, false);
    }
    auto iter = [&](auto st_c, int j) __attribute__((always_inline)) {
      top(j);
      if (j < nw) step(st_c, j + 1 < nw, j + 2 == nw && diag_in);
    };
#pragma unroll 1
    for (; j < nt; j += 4) {
      iter(I<0>{}, j);
      if (j + 1 >= nt) break;
      iter(I<1>{}, j + 1);
      if (j + 2 >= nt) break;
      iter(I<2>{}, j + 2);
      if (j + 3 >= nt) break;
      iter(I<3>{}, j + 3);
    }

    } else {
      // ---- ping-pong: the two wavefronts of a SIMD (key halves kh = 0, 1 of
      // every tile, same queries) run the same work per tile -- P V and
      // S = K Q^T on the matrix cores (16 MFMAs), the online softmax on the
      // vector ALUs -- half an iteration apart.  After the barrier of
      // iteration j, kh = 0 issues its MFMAs (P V of tile j-1, S of tile j)
      // while kh = 1 runs the softmax of tile j-1 and reads its MFMA operands
      // (V of tile j-1, K of tile j) from LDS; then kh = 1 issues its MFMAs
      // while kh = 0 runs the softmax of tile j and reads V of tile j and K of
      // tile j+1.  One wavefront on the matrix cores beside one on the vector
      // ALUs keeps both busy (a wavefront interleaving the two kinds itself
      // hides about half its vector work), and each half-iteration carries
      // half of the LDS fragment reads.  K tiles are therefore copied one tile
      // further ahead than V tiles: iteration j needs K of tiles j, j+1 and V
      // of tiles j-1, j, and refills the K stage of tile j-1 with tile j+3 and
      // the V stage of tile j-2 with tile j+2 (tile t in stage t % 4 of each).
      floatx16 sc;
      bf16x8 pf[2], va[4][2], kf[8];
      // Masks keys after each lane's query in the scores sc of tile jt (first
      // key 64 (t0 + jt) + 32 kh), raises the running max lazily and leaves
      // the bf16 probabilities in pf.
      auto softmax = [&](int jt) __attribute__((always_inline)) {
        const int dlt = 64 * (t0 + jt) + 32 * kh - qw;  // first key - first query: 0 on the diagonal
        float mx;
        if (dlt > -32) {
          mx = -INFINITY;
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            sc[e] = dlt + 8 * (e >> 2) + 4 * h32 + (e & 3) > l32 ? -INFINITY : sc[e];
            mx = fmaxf(mx, sc[e]);
          }
        } else {
          mx = plain_max(sc);
        }
        rescale(mx);
        const float mneg = m_run == -INFINITY ? 0.f : -m_run;
        float rs = 0.f;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const float pe = fast_exp2(fmaf(sc[e], c, mneg));
          rs += pe;
          pf[e >> 3][e & 7] = (bf16)pe;
        }
        l_run += rs;
      };
      auto pv = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int db = 0; db < 4; ++db)
#pragma unroll
          for (int uu = 0; uu < 2; ++uu) oacc[db] = MF::mma(va[db][uu], pf[uu], oacc[db]);
      };
      auto qk = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int e = 0; e < 16; ++e) sc[e] = 0.f;
#pragma unroll
        for (int f = 0; f < 8; ++f) sc = MF::mma(kf[f], qf[f], sc);
      };
      auto read_k = [&](auto st_c) __attribute__((always_inline)) {
        constexpr int st = decltype(st_c)::value;
#pragma unroll
        for (int f = 0; f < 8; ++f) kf[f] = kfrag(st, f);
      };
      auto read_v = [&](auto st_c) __attribute__((always_inline)) {
        constexpr int st = decltype(st_c)::value;
#pragma unroll
        for (int db = 0; db < 4; ++db)
#pragma unroll
          for (int uu = 0; uu < 2; ++uu) va[db][uu] = vfrag(st, db, uu);
      };
      // Copies of K (or V) of tile t into its stage st = t % 4: two 1 KB
      // copies per wavefront, through a buffer resource over the tile's rows
      // (rows past the sequence read as zeros).  (One resource per segment
      // with the tile offset in the per-lane offset was measured slower:
      // 8 x 2048 25.8 -> 30.3 us, 8 x 8192 150 -> 156 us.)
      auto dma_k = [&](auto st_c, int t) __attribute__((always_inline)) {
        constexpr int st = decltype(st_c)::value;
        const int nkeys = min(BN, src.keys - t * BN);
        const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(
            (void*)(src.k + (long)t * BN * p.k_ss), (short)0, 2 * ((nkeys - 1) * (int)p.k_ss + dlim), kBufferFlags);
        const unsigned sb = lds0 + st * TILEB;
        copy_1k(rk, dk[0], sb);
        copy_1k(rk, dk[1], sb + 1024);
      };
      auto dma_v = [&](auto st_c, int t) __attribute__((always_inline)) {
        constexpr int st = decltype(st_c)::value;
        const int nkeys = min(BN, src.keys - t * BN);
        const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
            (void*)(src.v + (long)t * BN * p.v_ss), (short)0, 2 * ((nkeys - 1) * (int)p.v_ss + dlim), kBufferFlags);
        const unsigned sb = lds0 + VOFF + st * TILEB;
        copy_1k(rv, dv[0], sb);
        copy_1k(rv, dv[1], sb + 1024);
      };
      // Top of iteration j: K of tile j+1 and V of tile j have landed for
      // every wavefront (the copies issued after them are those of the
      // previous iteration: K of tile j+2 and V of tile j+1), every wavefront
      // is done with the K stage of tile j-1 and the V stage of tile j-2.
      auto top = [&](int j) __attribute__((always_inline)) {
        if (j + 2 < nt)
          wait_vm<4>();
        else if (j + 1 < nt)
          wait_vm<2>();
        else
          wait_vm<0>();
        bar();
      };
      // The copies of iteration j (K of tile j+3 and V of tile j+2 into the
      // stages top(j) freed).  Each wavefront issues its share at the start
      // of its vector half: a burst of copies holds a wavefront's issue while
      // the vector memory unit takes them (32 KB per CU), which would delay
      // the MFMAs of the wavefront whose matrix half comes first.
      auto copies = [&](auto st_c, int j) __attribute__((always_inline)) {
        constexpr int st = decltype(st_c)::value;
        if (j + 3 < nt) dma_k(I<(st + 3) % 4>{}, j + 3);
        if (j + 2 < nt) dma_v(I<(st + 2) % 4>{}, j + 2);
      };
      // One iteration j >= 1 (st = j % 4, a compile-time constant).
      auto body0 = [&](auto st_c, int j) __attribute__((always_inline)) {
        constexpr int st = decltype(st_c)::value;
        top(j);
        pv();
        qk();
        __builtin_amdgcn_sched_barrier(0);
        copies(I<st>{}, j);
        read_v(I<st>{});
        if (j + 1 < nt) read_k(I<(st + 1) % 4>{});
        softmax(j);
        __builtin_amdgcn_sched_barrier(0);
      };
      auto body1 = [&](auto st_c, int j) __attribute__((always_inline)) {
        constexpr int st = decltype(st_c)::value;
        top(j);
        copies(I<st>{}, j);
        read_v(I<(st + 3) % 4>{});
        read_k(I<st>{});
        softmax(j - 1);
        __builtin_amdgcn_sched_barrier(0);
        pv();
        qk();
        __builtin_amdgcn_sched_barrier(0);
      };
      auto run = [&](auto body, auto kh_c) __attribute__((always_inline)) {
        // Tile 0: S only (kh = 0 also its softmax, V of tile 0 and K of tile
        // 1).  The segment's first two tiles were copied before the previous
        // segment's hand-over (stages 0 and 1); stages 2 and 3 held that
        // hand-over, so their copies wait for the barrier.  Every copy issued
        // after K of tile 1 is V of tile 1 (or a store of the previous segment,
        // which this wait also covers).
        if (nt > 1)
          wait_vm<2>();
        else
          wait_vm<0>();
        bar();
        auto copies0 = [&]() __attribute__((always_inline)) {
          if (nt > 2) dma_k(I<2>{}, 2);
          copies(I<0>{}, 0);
        };
        if constexpr (decltype(kh_c)::value == 1) copies0();
        read_k(I<0>{});
        __builtin_amdgcn_sched_barrier(0);
        qk();
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (decltype(kh_c)::value == 0) {
          copies0();
          read_v(I<0>{});
          if (nt > 1) read_k(I<1>{});
          softmax(0);
        }
        int j = 1;
#pragma unroll 1
        for (; j + 4 <= nt; j += 4) {
          body(I<1>{}, j);
          body(I<2>{}, j + 1);
          body(I<3>{}, j + 2);
          body(I<0>{}, j + 3);
        }
        if (j < nt) {
          body(I<1>{}, j);
          if (j + 1 < nt) {
            body(I<2>{}, j + 1);
            if (j + 2 < nt) body(I<3>{}, j + 2);
          }
        }
      };
      if (kh == 0) {
        run(body0, I<0>{});
        pv();  // P V of the last tile (its V^T fragments are in va)
      } else {
        run(body1, I<1>{});
        // softmax and P V of the last tile, from stage (nt - 1) % 4
        const int sl = (nt - 1) & 3;
#pragma unroll
        for (int db = 0; db < 4; ++db)
#pragma unroll
          for (int uu = 0; uu < 2; ++uu) va[db][uu] = vfrag(sl, db, uu);
        softmax(nt - 1);
        pv();
      }
    }

    // ---- segment end.  The next segment's Q and first two tiles are
    // requested now (its tiles go to stages 0 and 1; the hand-over uses
    // stages 2 and 3), so that their latency overlaps the hand-over and the
    // stores of this segment.
    const long next_u = bstart + t0 - 1;  // the last unit of the previous segment
    const bool more = next_u >= u0;
    Seg nxt = cur;
    if (more) nxt = decode_seg_x<F>(next_u, u0, w);
    bar();  // every wavefront is done with the stages
    const Src nsrc = seg_src(nxt);
    if (more) {
      load_q(nxt);
      dma(nsrc, 0);
      if (nxt.t1 - nxt.t0 > 1) dma(nsrc, 1);
    }

    // ---- hand-over between the two key halves.  Wavefront (wq, kh) keeps
    // d-blocks 2 kh and 2 kh + 1 and writes the other two, with its (max,
    // sum), for its partner (wq, 1 - kh).  Slot layout: float4 chunk k
    // (d-block 2 (1 - kh) + k / 4, elements 4 (k % 4) ..) of lane l at
    // (k * 64 + l) * 16.
    float l_tot = sum_xor32(l_run);  // lanes l and l ^ 32 hold the same query
    {
      float4* xs = reinterpret_cast<float4*>(lds + xslot(wid)) + lane;
      auto put = [&](const floatx16& o, int t) __attribute__((always_inline)) {
#pragma unroll
        for (int k = 0; k < 4; ++k) xs[(4 * t + k) * 64] = make_float4(o[4 * k], o[4 * k + 1], o[4 * k + 2], o[4 * k + 3]);
      };
      if (kh == 0) {
        put(oacc[2], 0);
        put(oacc[3], 1);
      } else {
        put(oacc[0], 0);
        put(oacc[1], 1);
      }
      reinterpret_cast<float2*>(lds + MLOFF)[wid * 64 + lane] = make_float2(m_run, l_tot);
    }
    bar();
    floatx16 own[2];
    {
      const int pw = wid ^ 4;
      const float4* xo = reinterpret_cast<const float4*>(lds + xslot(pw)) + lane;
      const float2 ml = reinterpret_cast<const float2*>(lds + MLOFF)[pw * 64 + lane];
      // The state of key half 0 is A, that of half 1 is B; both wavefronts
      // compute O = A aA + B aB in the same order.
      const float mA = kh == 0 ? m_run : ml.x, mB = kh == 0 ? ml.x : m_run;
      const float lA = kh == 0 ? l_tot : ml.y, lB = kh == 0 ? ml.y : l_tot;
      const float M = fmaxf(mA, mB);
      const float aA = mA == -INFINITY ? 0.f : fast_exp2(mA - M);
      const float aB = mB == -INFINITY ? 0.f : fast_exp2(mB - M);
      m_run = M;
      l_tot = fmaf(lB, aB, lA * aA);
      // mine: this wavefront's d-block t; the partner's copy comes from LDS.
      auto fold = [&](const floatx16& mine, int t, floatx16& out) __attribute__((always_inline)) {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const float4 x = xo[(4 * t + k) * 64];
          const float xv[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float oa = kh == 0 ? mine[4 * k + e] : xv[e], ob = kh == 0 ? xv[e] : mine[4 * k + e];
            out[4 * k + e] = fmaf(ob, aB, oa * aA);
          }
        }
      };
      if (kh == 0) {
        fold(oacc[0], 0, own[0]);
        fold(oacc[1], 1, own[1]);
      } else {
        fold(oacc[2], 0, own[0]);
        fold(oacc[3], 1, own[1]);
      }
    }

    // Normalises and writes this wavefront's 32 queries x 64 d-columns
    // (d-blocks 2 kh, 2 kh + 1).  The register layout of O^T (a lane holds one
    // query and groups of 4 columns) would make every 8-byte store touch a
    // different row, so the block is staged as bf16 rows in the partner's
    // hand-over slot (read above; nobody else touches it) and written 16 bytes
    // per lane, 8 lanes per 128-byte row segment.
    auto store_out = [&](const floatx16 (&o)[2], float l) __attribute__((always_inline)) {
      bf16* stg = reinterpret_cast<bf16*>(lds + xslot(wid ^ 4));
      const float linv = 1.0f / l;
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int bq = 0; bq < 4; ++bq) {
          bf16x4 v4;
#pragma unroll
          for (int e = 0; e < 4; ++e) v4[e] = (bf16)(o[t][4 * bq + e] * linv);
          *reinterpret_cast<bf16x4*>(stg + l32 * STG_PITCH + 32 * t + 8 * bq + 4 * h32) = v4;
        }
      bf16* obase = static_cast<bf16*>(p.o) + (long)hh * p.o_sh + 64 * kh;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int cidx = lane + 64 * i, row = cidx >> 3, cc = cidx & 7;
        const uint4 x = *reinterpret_cast<const uint4*>(stg + row * STG_PITCH + 8 * cc);
        if (qw + row < S && 64 * kh + 8 * cc < dlim)
          *reinterpret_cast<uint4*>(obase + (long)(qw + row) * p.o_ss + 8 * cc) = x;
      }
    };

    // ---- finish the query block, or hand a partial state to the last arriver
    int nparts = 1, vf = vidx;
    if (w.sched == kBalanced) {
      vf = range_of_x<F>(bstart, w);
      nparts = range_of_x<F>(bstart + cur.nt - 1, w) - vf + 1;
    }
    if (nparts == 1) {
      store_out(own, l_tot);
    } else {
      // Partial state of range v's slot s (0: the first segment of the range,
      // 1: its last): per wavefront PCH float4 chunks per lane, chunk k of
      // lane l at ((v * 2 + s) * 8 + wavefront) * PCH * 1024 + (k * 64 + l) * 16.
      typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
      const __amdgpu_buffer_rsrc_t prsrc =
          __builtin_amdgcn_make_buffer_rsrc(w.part, (short)0, w.part_bytes, kBufferFlags);
      auto pbase = [&](int v) __attribute__((always_inline)) {
        const int s = range_start_x<F>(v, w) >= bstart ? 0 : 1;
        return ((v * 2 + s) * 8 + wid) * (PCH * 1024) + lane * 16;
      };
      // The holder of the block's last range merges: it waits for the other
      // parts' arrivals instead of storing its own state (await_parts).
      const int vl = vf + nparts - 1;
      if (vidx == vl) await_parts(&w.count[hh * w.nqb + b], nparts, w.polls, arrival);
      if (vidx != vl || arrival != nparts - 1) {
        const int base = pbase(vidx);
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int k = 0; k < 4; ++k)
            __builtin_amdgcn_raw_buffer_store_b128(
                __builtin_bit_cast(u32x4, make_float4(own[t][4 * k], own[t][4 * k + 1], own[t][4 * k + 2],
                                                      own[t][4 * k + 3])),
                prsrc, base + (4 * t + k) * 1024, 0, kDeviceCoherent);
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, make_float4(m_run, l_tot, 0.f, 0.f)), prsrc,
                                               base + 8 * 1024, 0, kDeviceCoherent);
        // Release: every wavefront's device-coherent stores have completed
        // before the barrier and so before the arrival atomic.
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (tid == 0) arrival = atomicAdd(&w.count[hh * w.nqb + b], 1);
        __syncthreads();
      }
      if (arrival == nparts - 1) {
        // Last to arrive: the others' states were complete before their
        // arrivals, which precede this one; device-coherent loads read them.
        // The parts are folded in range order, this workgroup's own (in
        // registers) at its place, so the result is the same whichever part
        // arrived last.  Every part's (m, l) is read first for the common max.
        float M = m_run;
#pragma unroll 1
        for (int v2 = vf; v2 < vf + nparts; ++v2)
          if (v2 != vidx)
            M = fmaxf(M, __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(
                                                        prsrc, pbase(v2) + 8 * 1024, 0, kDeviceCoherent)).x);
        floatx16 acc[2];
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int e = 0; e < 16; ++e) acc[t][e] = 0.f;
        float lacc = 0.f;
#pragma unroll 1
        for (int v2 = vf; v2 < vf + nparts; ++v2) {
          if (v2 == vidx) {
            const float a = m_run == -INFINITY ? 0.f : fast_exp2(m_run - M);
            lacc = fmaf(l_tot, a, lacc);
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
              for (int e = 0; e < 16; ++e) acc[t][e] = fmaf(own[t][e], a, acc[t][e]);
          } else {
            const int base = pbase(v2);
            float4 x[PCH];
#pragma unroll
            for (int k = 0; k < PCH; ++k)
              x[k] = __builtin_bit_cast(float4,
                                        __builtin_amdgcn_raw_buffer_load_b128(prsrc, base + k * 1024, 0, kDeviceCoherent));
            const float a = x[8].x == -INFINITY ? 0.f : fast_exp2(x[8].x - M);
            lacc = fmaf(x[8].y, a, lacc);
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
              for (int k = 0; k < 4; ++k) {
                const float4 y = x[4 * t + k];
                acc[t][4 * k] = fmaf(y.x, a, acc[t][4 * k]);
                acc[t][4 * k + 1] = fmaf(y.y, a, acc[t][4 * k + 1]);
                acc[t][4 * k + 2] = fmaf(y.z, a, acc[t][4 * k + 2]);
                acc[t][4 * k + 3] = fmaf(y.w, a, acc[t][4 * k + 3]);
              }
          }
        }
        store_out(acc, lacc);
        if (tid == 0) atomicExch(&w.count[hh * w.nqb + b], 0);
      }
    }
    if (!more) break;
    cur = nxt;
    src = nsrc;
  }
}

void launch_flash_fwd(const AttnArgs& a, const Work& w, bool pingpong, hipStream_t st) {
  // Instantiated over the schedule arithmetic too: 32-bit only when the plan
  // fits (Work::fast).
  const dim3 grid((unsigned)w.grid), block(512);
  if (pingpong) {
    if (w.fast)
      flash_fwd_kernel<true, true><<<grid, block, 0, st>>>(a, w);
    else
      flash_fwd_kernel<true, false><<<grid, block, 0, st>>>(a, w);
  } else {
    if (w.fast)
      flash_fwd_kernel<false, true><<<grid, block, 0, st>>>(a, w);
    else
      flash_fwd_kernel<false, false><<<grid, block, 0, st>>>(a, w);
  }
}

size_t flash_fwd_part_bytes() { return fwd::PART_BYTES; }

}  // namespace nkl
