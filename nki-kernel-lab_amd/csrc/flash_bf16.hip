// bf16 causal flash attention for gfx950 -- the hot path.
//
// Work decomposition.  Queries are grouped in blocks of QB (64 or 128); keys
// in tiles of BN = 32.  A "unit" is one (head, query block, key tile) triple
// with the tile at or below the diagonal (tiles above it are never visited).
// The units of a head are numbered block by block, either in block order or
// in pair order -- blocks 0, n-1, 1, n-2, ... so that consecutive pairs
// (b, n-1-b) all hold the same number of units.  Three schedules:
//   block     one workgroup per query block, heaviest first;
//   pairs     one workgroup per pair of blocks (equal work everywhere);
//   balanced  the units cut into equal contiguous ranges, one per workgroup
//             and at most one workgroup per CU (stream-K).  A workgroup walks
//             its range as segments (one per block it touches); a block split
//             across workgroups is finished by whichever arrives last, which
//             folds in the others' partial (max, sum, output) states from the
//             workspace.  In pair order with 64-query blocks, 8 x 2048 cuts
//             into exactly two workgroups per pair.
//
// Workgroup.  NT teams of WPT wavefronts (QB = 32 WPT).  Wavefront q of a
// team owns queries 32 q .. 32 q + 31 of the block; team t takes the tiles
// t, t + NT, ... of the segment, so each SIMD runs wavefronts of different
// teams whose MFMA and exp work interleave.  At the end of a segment the
// teams' states are combined through LDS, each team finishing its own share
// of the head dim.
//
// Per 32-key tile a wavefront computes, with 32x32x16 bf16 MFMAs,
//     S^T[32 keys x 32 queries] = K . Q^T        (8 MFMAs for d = 128)
//     O^T[d x 32 queries]      += V^T . P^T      (8 MFMAs for d = 128)
// Lane l holds query l % 32 throughout.  Its 16 scores are keys
// 8 (i / 4) + 4 (l / 32) + i % 4 (i < 16), so the probabilities of MFMA u
// (keys 16 u .. 16 u + 15) are elements 8 u .. 8 u + 7 -- already the B
// operand.  K and V sit in LDS row-major ([key][d]); the V^T operand is read
// with ds_read_b64_tr_b16, whose 16-lane groups return lane i the elements
// (i % 4) of the 8-byte rows addressed by lanes 4 k + i / 4, k < 4: pointing
// lane j at V[r0 + j / 4][d0 + 4 (j % 4)] gives lane i V[r0 + k][d0 + i].
//
// K/V tiles are staged global -> VGPR -> LDS one tile ahead of use, double
// buffered in LDS, through bounds-checked buffer loads (out-of-range chunks
// read as zero with no branch, so every pipeline step issues the same loads).
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include <vector>

#include "attention.h"
#include "flash_sched.h"

namespace nkl {

namespace {

using namespace fsched;

constexpr int BN = 32;  // keys per tile
// Smallest unit range a workgroup is given in the balanced schedule (16 left
// half the CUs idle at 2 x 2048: 24.7 -> 20.6 us at 8; 2 x 1024: 25.5 -> 17.6).
constexpr long kMinUnits = 8;
// The merging workgroup's default poll budget, and the part count (the
// longest block over the mean range) from which it does not wait at all.
constexpr int kPolls = 256;
// Split blocks of up to kMaskParts parts (the teams kernel's 128-query form)
// record arrivals as a bit per part in the block's counter: part vf + i sets
// bit i, the holder of the last range kHolderBit, with the number of parts it
// folded before it gave up waiting from bit kFoldShift.  Blocks of more parts
// count arrivals and their holder does not wait, which is also where the
// planner's no-wait rule (kNoWaitParts) applies.
constexpr int kMaskParts = 6;
constexpr int kHolderBit = 1 << 24;
constexpr int kFoldShift = 25;
constexpr long kNoWaitParts = 6;
// Longest sequence for which the one-pass kernel (flash_tiny.hip) is always
// chosen; up to kTinyMaxS it is chosen for launches in the 64-query regime.
constexpr int kTinyAutoS = 224;


template <int D, int WPT, int NT>
struct Layout {
  static constexpr int QB = 32 * WPT;      // queries per block
  static constexpr int TT = 64 * WPT;      // threads per team
  static constexpr int LDK = D + 8;        // K row stride: rows 4 banks apart (16-lane b128 reads)
  static constexpr int LDV = D + 32;       // V row stride: rows 16 banks apart (32-lane b64 transposed reads)
  static constexpr int K_ELEMS = BN * LDK;
  static constexpr int STAGE = K_ELEMS + BN * LDV;
  static constexpr int TEAM = 2 * STAGE;
  static constexpr int TOTAL = NT * TEAM;
  static constexpr int NDB = D / 32;                       // 32-row d-blocks of O^T
  static constexpr int OWN = NDB >= NT ? NDB / NT : 1;     // d-blocks a team finishes
  static constexpr int NCO = 4 * NDB;                      // float4 chunks of O per lane
  static constexpr int SLOT = 64 * 4 * (NCO + 1);          // floats of one wavefront's state
  static constexpr int PART = WPT * SLOT;                  // floats of one partial block state
  static constexpr int XBYTES = NT * WPT * SLOT * 4;       // team hand-over area (reuses the stages)
  // bf16 elements of LDS (a single team hands nothing over)
  static constexpr int SMEM = NT == 1 || TOTAL * 2 > XBYTES ? TOTAL : XBYTES / 2;
  // The first segment's Q block, staged in LDS with the K row stride: past
  // the stages where it fits, else in team 0's second stage (read into
  // registers before the first tile's barrier, ahead of any write there);
  // -1: loaded straight into registers.
  static constexpr int QELEMS = QB * LDK;
  static constexpr int QOFF = NT == 1 ? -1 : TOTAL + QELEMS <= SMEM ? TOTAL : QELEMS <= STAGE ? STAGE : -1;
};


__device__ __forceinline__ bf16x8 read_vt_frag(const bf16* row_a, const bf16* row_b) {
  typedef short shortx4 __attribute__((ext_vector_type(4)));
  typedef short shortx8 __attribute__((ext_vector_type(8)));
  typedef __attribute__((address_space(3))) shortx4 lds_s4;
  const shortx4 a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)(row_a));
  const shortx4 b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)(row_b));
  const shortx8 c = __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7);
  return __builtin_bit_cast(bf16x8, c);
}


}  // namespace

template <int D, int WPT, int NT, bool H = false, bool F = false>
// Two wavefronts per SIMD (at most 256 registers each): a 4-wavefront
// workgroup then shares its CU with a second one.  H: fp16 operands, P and O
// (the 16-bit values move as raw bits; only the MFMA and the roundings of P
// and O depend on the format).
__global__ __launch_bounds__(64 * WPT * NT) __attribute__((amdgpu_waves_per_eu(2)))
void flash_bf16_kernel(AttnArgs p, Work w) {
  using L = Layout<D, WPT, NT>;
  constexpr int QB = L::QB, TT = L::TT;
  constexpr int CPR = D / 8;                    // 16-byte chunks per K/V row
  constexpr int NCHUNK = BN * CPR;              // chunks per K (or V) tile
  constexpr int CH = (NCHUNK + TT - 1) / TT;    // chunks per team thread, per tensor
  constexpr int NQF = D / 16;                   // Q^T fragments (K = 16 per MFMA)
  constexpr int NDB = L::NDB, OWN = L::OWN;
  __shared__ __align__(16) bf16 smem[L::SMEM];
  __shared__ int arrival;

  prefetch_kernargs<sizeof(AttnArgs) + sizeof(Work)>();
  const int tid = threadIdx.x, lane = tid & 63;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int team = wid / WPT, wq = wid % WPT;
  const int ttid = tid % TT;
  const int h32 = lane >> 5, l32 = lane & 31;
  const int S = p.S, dlim = p.d;
  const float c = p.c;
  bf16* const team_base = smem + team * L::TEAM;

  // Per-thread chunk coordinates within a tile (surplus threads of a small
  // head dim repeat the last chunk).
  int goff_k[CH], goff_v[CH], loff_k[CH], loff_v[CH];
  bool dok[CH];
#pragma unroll
  for (int i = 0; i < CH; ++i) {
    const int ci = min(ttid + TT * i, NCHUNK - 1);
    const int row = ci / CPR, col = (ci % CPR) * 8;
    goff_k[i] = 2 * (row * (int)p.k_ss + col);
    goff_v[i] = 2 * (row * (int)p.v_ss + col);
    loff_k[i] = row * L::LDK + col;
    loff_v[i] = L::K_ELEMS + row * L::LDV + col;
    dok[i] = col < dlim;
  }
  // Per-lane LDS element offsets of the MFMA operands within a stage.
  const int kfrag_off = l32 * L::LDK + 8 * h32;
  const int i16 = lane & 15, g2 = (lane >> 4) & 1;
  const int vfrag_off = L::K_ELEMS + (4 * h32 + (i16 >> 2)) * L::LDV + 16 * g2 + 4 * (i16 & 3);

  long u0, u1;
  const int vidx = wg_range_x<F>(w, p.H, u0, u1);  // this workgroup's range index and units [u0, u1)

  // The segment of the range that ends with unit u (fsched::decode_seg: a
  // range is walked from its last segment to its first).
  auto decode = [&](long u) __attribute__((always_inline)) { return decode_seg_x<F>(u, u0, w); };
  auto load_q = [&](const Seg& sg, bf16x8 (&q)[NQF]) __attribute__((always_inline)) {
    const bf16* Q = static_cast<const bf16*>(p.q) + (long)sg.hh * p.q_sh;
    const int qrow = QB * sg.b + 32 * wq + l32;
#pragma unroll
    for (int f = 0; f < NQF; ++f) {
      const int dd = 16 * f + 8 * h32;
      q[f] = __builtin_bit_cast(bf16x8, ld16_or_zero(Q, (long)qrow * p.q_ss + dd, qrow < S && dd < dlim));
    }
  };
  // Loads of one tensor (K or V) for step `it` of this team within segment sg
  // (K/V head hh / group: grouped-query attention shares a K/V head).
  auto gload = [&](const Seg& sg, int it, const void* base, long sh, long ss, const int (&goff)[CH],
                   uint4 (&rr)[CH]) __attribute__((always_inline)) {
    const int tj = sg.t0 + team + NT * it;
    const int k0 = tj * BN;
    const int nkeys = tj < sg.t1 ? min(BN, S - k0) : 0;
    const int bytes = nkeys > 0 ? 2 * ((nkeys - 1) * (int)ss + dlim) : 0;
    const __amdgpu_buffer_rsrc_t src = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(static_cast<const bf16*>(base) + (long)(sg.hh / p.group) * sh + (long)k0 * ss), (short)0, bytes,
        kBufferFlags);
#pragma unroll
    for (int i = 0; i < CH; ++i)
      rr[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(src, goff[i], 0, 0));
  };
  auto lstore = [&](int stage, const uint4 (&rk)[CH], const uint4 (&rv)[CH]) __attribute__((always_inline)) {
    bf16* sb = team_base + stage * L::STAGE;
    if (dlim == D) {
#pragma unroll
      for (int i = 0; i < CH; ++i) {
        *reinterpret_cast<uint4*>(sb + loff_k[i]) = rk[i];
        *reinterpret_cast<uint4*>(sb + loff_v[i]) = rv[i];
      }
    } else {  // head-dim columns past d (a padded head dim) are stored as zeros
#pragma unroll
      for (int i = 0; i < CH; ++i) {
        *reinterpret_cast<uint4*>(sb + loff_k[i]) = dok[i] ? rk[i] : make_uint4(0, 0, 0, 0);
        *reinterpret_cast<uint4*>(sb + loff_v[i]) = dok[i] ? rv[i] : make_uint4(0, 0, 0, 0);
      }
    }
  };

  // Every wavefront's LDS accesses are done, then all wavefronts meet.  A
  // bare barrier: __syncthreads()' fence would also wait for every
  // outstanding global load (vmcnt(0)) -- the next tile's K/V in the loop,
  // the next segment's Q and first tile at a segment end -- which the
  // registers they land in are waited for where they are used.
  auto lds_barrier = [&]() __attribute__((always_inline)) {
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
  };

  // A segment's Q block is loaded once for the workgroup, 16 contiguous
  // bytes per lane (four 256-byte rows per wavefront instruction), and staged
  // in LDS, where each wavefront reads its MFMA fragments: loaded into
  // registers in the operand layout, every wavefront instruction would touch
  // 32 rows and every team would load the block again.  Past the stages
  // (QLA) the staging area is free at every segment start; in team 0's
  // second stage only the first segment's Q goes through it (later ones are
  // loaded straight into registers).
  constexpr bool QL = L::QOFF >= 0, QLA = L::QOFF == L::TOTAL;
  constexpr int QCHUNKS = QB * CPR, QCH = (QCHUNKS + TT * NT - 1) / (TT * NT);  // chunks per thread
  uint4 qc[QCH];
  auto load_qc = [&](const Seg& sg) __attribute__((always_inline)) {
    const int qrows = max(0, min(QB, S - QB * sg.b));
    const __amdgpu_buffer_rsrc_t qsrc = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(static_cast<const bf16*>(p.q) + (long)sg.hh * p.q_sh + (long)QB * sg.b * p.q_ss), (short)0,
        qrows > 0 ? 2 * ((qrows - 1) * (int)p.q_ss + dlim) : 0, kBufferFlags);
#pragma unroll
    for (int i = 0; i < QCH; ++i) {
      const int ci = min(tid + TT * NT * i, QCHUNKS - 1), row = ci / CPR, col = (ci % CPR) * 8;
      qc[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(qsrc, 2 * (row * (int)p.q_ss + col), 0, 0));
    }
  };
  auto store_qc = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < QCH; ++i) {
      const int ci = tid + TT * NT * i, row = ci / CPR, col = (ci % CPR) * 8;
      if (QCHUNKS % (TT * NT) == 0 || ci < QCHUNKS)
        *reinterpret_cast<uint4*>(smem + L::QOFF + row * L::LDK + col) = col < dlim ? qc[i] : make_uint4(0, 0, 0, 0);
    }
  };
  auto read_qf = [&](bf16x8 (&q)[NQF]) __attribute__((always_inline)) {
#pragma unroll
    for (int f = 0; f < NQF; ++f) q[f] = load_frag(smem + L::QOFF + (32 * wq + l32) * L::LDK + 16 * f + 8 * h32);
  };

  Seg cur = decode(u1 - 1);
  bf16x8 qf[NQF];
  uint4 rk[CH], rv[CH];  // the next tile's K and V on their way to LDS
  if constexpr (QL) load_qc(cur);
  else load_q(cur, qf);
  gload(cur, 0, p.k, p.k_sh, p.k_ss, goff_k, rk);
  gload(cur, 0, p.v, p.v_sh, p.v_ss, goff_v, rv);
  if constexpr (QL && !QLA) {  // staged in team 0's second stage: read before the first tile's barrier
    store_qc();
    __syncthreads();
    read_qf(qf);
  }

  for (;;) {
    const int hh = cur.hh, b = cur.b, t0 = cur.t0, t1 = cur.t1, nt_b = cur.nt;
    const long bstart = cur.bstart;
    const int qw = QB * b + 32 * wq;  // this wavefront's first query
    const int myq = qw + l32;
    const int nit = (t1 - t0 + NT - 1) / NT;

    if constexpr (QLA) store_qc();
    lstore(0, rk, rv);
    lds_barrier();
    if constexpr (QLA) read_qf(qf);
    gload(cur, 1, p.k, p.k_sh, p.k_ss, goff_k, rk);
    gload(cur, 1, p.v, p.v_sh, p.v_ss, goff_v, rv);

    float m_run = -INFINITY, l_run = 0.f;
    floatx16 oacc[NDB];
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int e = 0; e < 16; ++e) oacc[db][e] = 0.f;

    // Online softmax of one tile's scores (keys k0 ..): masks the diagonal
    // tile, raises the running max lazily, turns S into bf16 P.
    auto softmax = [&](int k0, floatx16& sc, bf16x8 (&pf)[2]) __attribute__((always_inline)) {
      if (k0 + BN - 1 > qw) {  // diagonal tile: mask keys after the query
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
#pragma unroll
      for (int uu = 0; uu < 2; ++uu)
#pragma unroll
        for (int j = 0; j < 8; ++j) pf[uu][j] = round16<H>(sc[8 * uu + j]);
    };
    // O += P V for the tile in stage sb.  The V^T fragments of two d-blocks
    // are read together before their MFMAs, so that the MFMAs wait on LDS
    // once per pair of d-blocks rather than once each.
    auto pv = [&](const bf16* sb, const bf16x8 (&pf)[2]) __attribute__((always_inline)) {
      constexpr int G = NDB >= 2 ? 2 : 1;
#pragma unroll
      for (int d0 = 0; d0 < NDB; d0 += G) {
        bf16x8 a[G][2];
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
          for (int uu = 0; uu < 2; ++uu) {
            const bf16* vaddr = sb + vfrag_off + 16 * uu * L::LDV + 32 * (d0 + g);
            a[g][uu] = read_vt_frag(vaddr, vaddr + 8 * L::LDV);
          }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
          for (int uu = 0; uu < 2; ++uu) oacc[d0 + g] = mma32_16b<H>(a[g][uu], pf[uu], oacc[d0 + g]);
      }
    };

    {
      // One step per tile: tile it computes from LDS stage it & 1.  Between
      // its QK^T MFMAs and its softmax, tile it + 1 (loaded into registers one
      // step earlier) is written to the other stage, which step it - 1 was the
      // last to read, and tile it + 2 is loaded into the registers; the LDS
      // writes then overlap the MFMA and VALU work of the step instead of
      // holding up its closing barrier (8 x 8192: 157 -> 151 us).
#pragma unroll 1
      for (int it = 0; it < nit; ++it) {
        const int tj = t0 + team + NT * it;
        const int k0 = tj * BN;
        const bool active = tj < t1 && k0 <= qw + 31;  // inside the segment and not above the diagonal
        const bf16* sb = team_base + (it & 1) * L::STAGE;
        floatx16 sacc;
        if (active) {
#pragma unroll
          for (int e = 0; e < 16; ++e) sacc[e] = 0.f;
          // Every K fragment read is in flight before the first MFMA waits
          // for one (left to itself the compiler reads one fragment, waits for
          // it and runs its MFMA, eight times over).
          bf16x8 kf[NQF];
#pragma unroll
          for (int f = 0; f < NQF; ++f) kf[f] = load_frag(sb + kfrag_off + 16 * f);
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int f = 0; f < NQF; ++f) sacc = mma32_16b<H>(kf[f], qf[f], sacc);
          __builtin_amdgcn_sched_barrier(0);
        }
        lstore((it + 1) & 1, rk, rv);
        gload(cur, it + 2, p.k, p.k_sh, p.k_ss, goff_k, rk);
        gload(cur, it + 2, p.v, p.v_sh, p.v_ss, goff_v, rv);
        if (active) {
          bf16x8 pf[2];
          softmax(k0, sacc, pf);
          __builtin_amdgcn_sched_barrier(0);
          pv(sb, pf);
        }
        lds_barrier();
      }
    }

    // ---- the next segment of the range: its Q and first K/V tile are loaded
    // as soon as the loop is done with Q and the staging registers, so that
    // their latency overlaps the hand-over between the teams and the stores
    // of this segment (issued after the stores they would wait for them too:
    // loads and stores share the vector memory counter).
    const long next_u = bstart + t0 - 1;  // the last unit of the previous segment
    const bool more = next_u >= u0;
    Seg nxt = cur;
    if (more) nxt = decode(next_u);
    if (more) {
      if constexpr (QLA)
        load_qc(nxt);
      else
        load_q(nxt, qf);  // this segment's Q fragments are no longer needed
      gload(nxt, 0, p.k, p.k_sh, p.k_ss, goff_k, rk);
      gload(nxt, 0, p.v, p.v_sh, p.v_ss, goff_v, rv);
    }

    // ---- hand-over between the teams.  Team t finishes d-blocks
    // [t OWN, (t + 1) OWN) of O (teams past the last d-block finish none) and
    // writes the other d-blocks of its state, with its (m, l), to LDS.  A
    // wavefront's state is float4 chunk k of lane l at k * 64 + l: chunks
    // 4 db .. 4 db + 3 hold d-block db, chunk NCO holds (m, l).
    const int own0 = team * OWN;
    const bool keeps = own0 < NDB;
    float l_tot = sum_xor32(l_run);  // lanes l and l ^ 32 hold the same query
    if constexpr (NT > 1) {
      float4* xs = reinterpret_cast<float4*>(smem) + (team * WPT + wq) * (L::SLOT / 4) + lane;
#pragma unroll
      for (int db = 0; db < NDB; ++db)
        if (db / OWN != team)
#pragma unroll
          for (int k = 0; k < 4; ++k)
            xs[(4 * db + k) * 64] =
                make_float4(oacc[db][4 * k], oacc[db][4 * k + 1], oacc[db][4 * k + 2], oacc[db][4 * k + 3]);
      xs[L::NCO * 64] = make_float4(m_run, l_tot, 0.f, 0.f);
    }
    floatx16 own[OWN];  // the d-blocks this team finishes, with compile-time indices
#pragma unroll
    for (int j = 0; j < OWN; ++j) own[j] = oacc[j];
#pragma unroll
    for (int t = 1; t < NT; ++t)
      if (team == t && t * OWN < NDB)
#pragma unroll
        for (int j = 0; j < OWN; ++j) own[j] = oacc[t * OWN + j < NDB ? t * OWN + j : NDB - 1];
    if constexpr (NT > 1) lds_barrier();

    // Folds a state with max m2 and sum l2 into (m_run, l_tot) and returns the
    // weights of the running state (a1) and of the other (a2).  An empty state
    // has m = -inf and weight 0, and two empty states stay empty.
    auto weights = [&](float m2, float l2, float& a1, float& a2) __attribute__((always_inline)) {
      const float M = fmaxf(m_run, m2);
      a1 = m_run == -INFINITY ? 0.f : fast_exp2(m_run - M);
      a2 = m2 == -INFINITY ? 0.f : fast_exp2(m2 - M);
      l_tot = l_tot * a1 + l2 * a2;
      m_run = M;
    };
    // Folds a wavefront state whose float4 chunk k (this lane's) is get(k);
    // all of its loads are issued before any is used.
    // A 4-wavefront workgroup holds twice the staging registers per thread;
    // it loads and folds one d-block at a time to stay within 256 registers.
    constexpr int GJ = WPT * NT == 4 ? 1 : OWN;
    auto fold_state = [&](auto get) __attribute__((always_inline)) {
      const float4 st = get(L::NCO);
      float a1 = 0.f, a2 = 0.f;
#pragma unroll
      for (int j0 = 0; j0 < OWN; j0 += GJ) {
        float4 v[GJ][4];
        if (keeps) {
#pragma unroll
          for (int j = 0; j < GJ; ++j)
#pragma unroll
            for (int k = 0; k < 4; ++k) v[j][k] = get(4 * (own0 + j0 + j) + k);
        }
        if (j0 == 0) weights(st.x, st.y, a1, a2);
        if (keeps) {
#pragma unroll
          for (int j = 0; j < GJ; ++j)
#pragma unroll
            for (int k = 0; k < 4; ++k) {
              floatx16& o = own[j0 + j];
              o[4 * k] = fmaf(v[j][k].x, a2, o[4 * k] * a1);
              o[4 * k + 1] = fmaf(v[j][k].y, a2, o[4 * k + 1] * a1);
              o[4 * k + 2] = fmaf(v[j][k].z, a2, o[4 * k + 2] * a1);
              o[4 * k + 3] = fmaf(v[j][k].w, a2, o[4 * k + 3] * a1);
            }
        }
      }
    };
#pragma unroll
    for (int t2 = 0; t2 < NT; ++t2)
      if (t2 != team) {
        const float4* xo = reinterpret_cast<const float4*>(smem) + (t2 * WPT + wq) * (L::SLOT / 4) + lane;
        fold_state([&](int k) __attribute__((always_inline)) { return xo[k * 64]; });
      }
    if constexpr (NT > 1) {
      // l summed over the teams in team order from their (m, l) in LDS, the
      // same sum in every team (the folds above add in a team-dependent
      // order): the merge of a split block, which starts either from a team's
      // registers or from the (m, l) team 0 stored, then gives the same bits.
      float lc = 0.f;
#pragma unroll
      for (int t2 = 0; t2 < NT; ++t2) {
        const float4 st = (reinterpret_cast<const float4*>(smem) + (t2 * WPT + wq) * (L::SLOT / 4) + lane)[L::NCO * 64];
        lc += st.x == -INFINITY ? 0.f : st.y * fast_exp2(st.x - m_run);
      }
      l_tot = lc;
    }

    // Writes this team's d-blocks of O / l for the wavefront's 32 queries.
    // The lane layout of O^T (lane: one query, 4-column groups of d) would
    // make every 8-byte store touch a different row, so the wavefront stages
    // its 32 x W block as bf16 rows in LDS and stores 16 bytes per lane, 8
    // consecutive lanes per 128-byte row segment.  The staging area is the
    // part of the wavefront's own hand-over slot that holds the d-blocks it
    // keeps, which the hand-over neither writes nor reads (no barrier needed);
    // a single team uses the idle stages.
    auto store_out = [&]() __attribute__((always_inline)) {
      if (!keeps) return;
      constexpr int W = 32 * OWN;     // d columns this team writes
      constexpr int PITCH = W + 8;    // staging row pitch, elements
      constexpr int CPRW = W / 8;     // 16-byte chunks per staged row
      static_assert(NT > 1 || WPT * 32 * PITCH <= L::SMEM, "single-team staging fits the stages");
      static_assert(NT == 1 || 32 * PITCH * 2 <= 4 * OWN * 1024, "staging fits the kept d-blocks of a slot");
      bf16* stg = NT == 1 ? smem + wq * (32 * PITCH)
                          : reinterpret_cast<bf16*>(reinterpret_cast<float4*>(smem) + (team * WPT + wq) * (L::SLOT / 4) +
                                                    4 * own0 * 64);
      const float linv = 1.0f / l_tot;
#pragma unroll
      for (int j = 0; j < OWN; ++j)
#pragma unroll
        for (int bq = 0; bq < 4; ++bq) {
          bf16x4 v4;
#pragma unroll
          for (int e = 0; e < 4; ++e) v4[e] = round16<H>(own[j][4 * bq + e] * linv);
          *reinterpret_cast<bf16x4*>(stg + l32 * PITCH + 32 * j + 8 * bq + 4 * h32) = v4;
        }
      bf16* obase = static_cast<bf16*>(p.o) + (long)hh * p.o_sh + 32 * own0;
#pragma unroll
      for (int i = 0; i < 32 * CPRW / 64; ++i) {
        const int cidx = lane + 64 * i, row = cidx / CPRW, cc = cidx % CPRW;
        const uint4 x = *reinterpret_cast<const uint4*>(stg + row * PITCH + 8 * cc);
        if (qw + row < S && 32 * own0 + 8 * cc < dlim)
          *reinterpret_cast<uint4*>(obase + (long)(qw + row) * p.o_ss + 8 * cc) = x;
      }
    };

    // ---- finish the query block, or hand a partial state to the last arriver
    int nparts = 1, vf = vidx;
    if (w.sched == kBalanced) {
      vf = range_of_x<F>(bstart, w);
      nparts = range_of_x<F>(bstart + nt_b - 1, w) - vf + 1;
    }
    if (nparts == 1) {
      store_out();
    } else {
      // A partial state is PART floats: one wavefront state (layout above) per
      // wavefront; each workgroup has two slots, for the first and the last
      // segment of its range.
      // Byte offset of this lane's chunk k of wavefront wq's state in slot s of
      // workgroup v (two slots: the first and the last segment of its range).
      typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
      const __amdgpu_buffer_rsrc_t prsrc = __builtin_amdgcn_make_buffer_rsrc(w.part, (short)0, w.part_bytes, kBufferFlags);
      auto poff = [&](int v, int s, int k) __attribute__((always_inline)) {
        return 4 * (((v * 2 + s) * L::PART) + wq * L::SLOT + k * 256 + 4 * lane);
      };
      const int slot = range_start_x<F>(vidx, w) >= bstart ? 0 : 1;
      auto pstore = [&](int k, float4 x) __attribute__((always_inline)) {
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, x), prsrc, poff(vidx, slot, k), 0,
                                               kDeviceCoherent);
      };
      if constexpr (WPT == 4 && NT == 2) {  // 128-query blocks, two teams
        // The parts are folded in one order whoever merges: the last range's
        // state first, then the others from the first range up.  The holder of
        // the last range walks that segment last, when the block's first part
        // (walked first by its range) has long been stored, so it folds the
        // parts from its registers as each arrives (a bit per part in the
        // block's counter) instead of after the slowest.  Past its poll budget
        // it stores what it has folded so far, with how many parts that is,
        // and arrives; the part that completes the counter then merges the
        // rest.  A fold into an empty state copies a part exactly, so every
        // path gives the same bits.  Blocks of more than kMaskParts parts count
        // arrivals instead, and their holder does not wait.
        const int vl = vf + nparts - 1;
        int* const cnt = &w.count[hh * w.nqb + b];
        const bool masked = nparts <= kMaskParts;
        const int full = masked ? ((1 << (nparts - 1)) - 1) | kHolderBit : 0;  // masked: every part in
        auto load_part = [&](int v2) __attribute__((always_inline)) {
          const int slot2 = range_start_x<F>(v2, w) >= bstart ? 0 : 1;
          fold_state([&](int k) __attribute__((always_inline)) {
            return __builtin_bit_cast(float4,
                                      __builtin_amdgcn_raw_buffer_load_b128(prsrc, poff(v2, slot2, k), 0, kDeviceCoherent));
          });
        };
        auto store_state = [&]() __attribute__((always_inline)) {
          if (keeps) {
#pragma unroll
            for (int j = 0; j < OWN; ++j)
#pragma unroll
              for (int k = 0; k < 4; ++k)
                pstore(4 * (own0 + j) + k,
                       make_float4(own[j][4 * k], own[j][4 * k + 1], own[j][4 * k + 2], own[j][4 * k + 3]));
          }
          if (team == 0) pstore(L::NCO, make_float4(m_run, l_tot, 0.f, 0.f));
          // Release: every wavefront's device-coherent stores have completed
          // (vmcnt) before the barrier and so before the arrival atomic.
          __builtin_amdgcn_s_waitcnt(0);
          __syncthreads();
        };
        int from = nparts;  // merging: fold parts vf + from .. vl - 1 after the start state (nparts: not merging)
        bool start_own = false;  // the start state is this workgroup's registers (else vl's stored state)
        if (vidx == vl && masked) {
          // m: the arrivals last read (one poll serves every part already in).
          int j = 0, budget = w.polls, m = 0;
          for (; j < nparts - 1; ++j) {
            if (!((m >> j) & 1)) {
              if (tid == 0) {
                int mm = __hip_atomic_load(cnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                while (!((mm >> j) & 1) && budget > 0) {
                  --budget;
                  __builtin_amdgcn_s_sleep(8);
                  mm = __hip_atomic_load(cnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
                arrival = mm;
              }
              __syncthreads();
              m = arrival;
              __syncthreads();
              if (!((m >> j) & 1)) break;
            }
            load_part(vf + j);
          }
          if (j == nparts - 1) {
            from = nparts - 1;  // all folded
            start_own = true;
          } else {  // out of budget: hand over what is folded
            store_state();
            if (tid == 0) {
              const int add = kHolderBit | (j << kFoldShift);
              arrival = ((atomicOr(cnt, add) | add) & full) == full;
            }
            __syncthreads();
            if (arrival) {  // the awaited part came in meanwhile: this workgroup is last
              from = j;
              start_own = true;
            }
          }
        } else {
          store_state();
          if (tid == 0) {
            if (masked) {
              const int bit = vidx == vl ? kHolderBit : 1 << (vidx - vf);
              const int now = atomicOr(cnt, bit) | bit;
              arrival = (now & full) == full ? (now >> kFoldShift) & 63 : -1;  // last: parts the holder folded
            } else {
              arrival = atomicAdd(cnt, 1) == nparts - 1 ? 0 : -1;
            }
          }
          __syncthreads();
          if (arrival >= 0) from = arrival;
          start_own = vidx == vl;
        }
        if (from < nparts) {  // this workgroup merges
          if (!start_own) {
            m_run = -INFINITY;
            l_tot = 0.f;
#pragma unroll
            for (int j = 0; j < OWN; ++j)
#pragma unroll
              for (int e = 0; e < 16; ++e) own[j][e] = 0.f;
            load_part(vl);
          }
#pragma unroll 1
          for (int j = from; j < nparts - 1; ++j) load_part(vf + j);
          store_out();
          if (tid == 0) atomicExch(cnt, 0);
        }
      } else {
        // The holder of the block's last range waits for the other parts to
        // arrive instead of storing its own state (see await_parts).
        const int vl = vf + nparts - 1;
        if (vidx == vl) await_parts(&w.count[hh * w.nqb + b], nparts, w.polls, arrival);
        if (vidx != vl || arrival != nparts - 1) {
          if (keeps) {
#pragma unroll
            for (int j = 0; j < OWN; ++j)
#pragma unroll
              for (int k = 0; k < 4; ++k)
                pstore(4 * (own0 + j) + k,
                       make_float4(own[j][4 * k], own[j][4 * k + 1], own[j][4 * k + 2], own[j][4 * k + 3]));
          }
          if (team == 0) pstore(L::NCO, make_float4(m_run, l_tot, 0.f, 0.f));
          // Release: every wavefront's device-coherent stores have completed
          // (vmcnt) before the barrier and so before the arrival atomic.
          __builtin_amdgcn_s_waitcnt(0);
          __syncthreads();
          if (tid == 0) arrival = atomicAdd(&w.count[hh * w.nqb + b], 1);
          __syncthreads();
        }
        if (arrival == nparts - 1) {  // last to arrive: merge the others and write O
          // The others' states were complete before their arrivals, which
          // precede this one; device-coherent loads read them from memory.
          // The parts are folded last range first, whichever workgroup arrived
          // last, so the result is bitwise reproducible: the holder of the last
          // range (the usual last arriver) starts from its own registers; any
          // other restarts from an empty state and reads its own part back (a
          // fold into an empty state copies a part exactly).
          if (vidx != vl) {
            m_run = -INFINITY;
            l_tot = 0.f;
#pragma unroll
            for (int j = 0; j < OWN; ++j)
#pragma unroll
              for (int e = 0; e < 16; ++e) own[j][e] = 0.f;
          }
#pragma unroll 1
          for (int v2 = vl; v2 >= vf; --v2) {
            if (v2 == vidx && vidx == vl) continue;
            const int slot2 = range_start_x<F>(v2, w) >= bstart ? 0 : 1;
            fold_state([&](int k) __attribute__((always_inline)) {
              return __builtin_bit_cast(float4,
                                        __builtin_amdgcn_raw_buffer_load_b128(prsrc, poff(v2, slot2, k), 0, kDeviceCoherent));
            });
          }
          store_out();
          if (tid == 0) atomicExch(&w.count[hh * w.nqb + b], 0);
        }
      }
    }
    lds_barrier();  // the LDS is restaged by the next segment
    if (!more) break;
    cur = nxt;
  }
}

// ------------------------------------------------- one wavefront per SIMD --
//
// The same unit schedules for d in (64, 128], with every wavefront alone on
// its SIMD (512 registers: O in AGPRs, Q in VGPRs).  A wavefront owns QW = 32
// or 64 queries (one or two 32-query halves): with 64, every K and V fragment
// read from LDS feeds two MFMAs, which halves the LDS read traffic per FLOP.
// A workgroup of NW wavefronts takes blocks of QB = QW * NW queries; with
// NW = 2 two workgroups share a CU.  The
// wavefront overlaps its own MFMA and VALU work: the QK^T MFMAs of tile i+1
// are issued before the softmax and P V of tile i.  K/V tiles are copied
// global -> LDS by the buffer unit (buffer_load ... lds: lane l's 16 bytes
// land at the instruction's LDS base + 16 l), W1_NS - 2 tiles ahead of use,
// into W1_NS stages of unpadded 256-byte rows whose 16-byte chunks are
// swizzled: logical chunk c of row r sits at chunk c ^ row_swz(r), with
// row_swz(r) = 4 (r % 4) + 2 ((r / 4) % 2) + (r / 8) % 2.  The 16 rows of a
// K-fragment read (b128, one chunk each, also as rows 0-7 x chunks 2f, 2f+1)
// and the 4 aligned rows x 4 aligned chunks of a transposed V read (b64)
// then all fall in distinct bank groups.  W1_NS = 4 stages of 16 KB keep
// every stage-relative LDS offset an instruction immediate (the loop is
// unrolled by the stage count).

namespace {

constexpr int W1_NS = 4;                    // LDS stages (offsets stay below 64 KB)
constexpr int W1_ROWB = 256;                // bytes of a K/V row (d = 128)
constexpr int W1_TILEB = BN * W1_ROWB;      // bytes of a K (or V) tile
constexpr int W1_STAGEB = 2 * W1_TILEB;     // K tile then V tile

}  // namespace

template <int QH, int NW, int OCC = 1, bool F = false>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(OCC, OCC)))
void flash_bf16_w1_kernel(AttnArgs p, Work w) {
  static_assert((QH == 1 || QH == 2) && (NW == 2 || NW == 4), "32 or 64 queries per wavefront, 2 or 4 wavefronts");
  prefetch_kernargs<sizeof(AttnArgs) + sizeof(Work)>();
  constexpr int D = 128, NQF = D / 16, NDB = D / 32, QW = 32 * QH, QB = QW * NW;
  // Partial state of one 32-query half: NCO float4 chunks of O and one of
  // (m, l) per lane.
  constexpr int NCO = 4 * NDB, HS = 64 * 4 * (NCO + 1), SLOT = QH * HS, PART = NW * SLOT;
  constexpr int NI = 8 / NW;    // 1 KB copies per K (and per V) tile per wavefront
  constexpr int LPT = 2 * NI;   // copies per tile per wavefront
  using MF = Mfma32<bf16>;
  __shared__ __align__(16) unsigned char lds[W1_NS * W1_STAGEB];
  __shared__ int arrival;
  // Alone on its SIMD (OCC = 1), declaring an AGPR use makes the compiler
  // select the MFMA form whose accumulators live in AGPRs, which keeps O there
  // for the whole loop.  Two per SIMD (OCC = 2) share 256 registers.
  if constexpr (OCC == 1) asm volatile("" ::: "a255");

  const int tid = threadIdx.x, lane = tid & 63;
  const int wq = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int h32 = lane >> 5, l32 = lane & 31;
  const int S = p.S, dlim = p.d;
  const float c = p.c;

  // Per-lane byte offsets within a stage.
  //   K fragment f: row l32, logical chunk 2 f + h32.
  int koff[NQF];
  {
    const int sw = row_swz(l32);
#pragma unroll
    for (int f = 0; f < NQF; ++f) koff[f] = l32 * W1_ROWB + (((2 * f + h32) ^ sw) << 4);
  }
  //   V^T fragment (d-block db, first or second 8-row read): rows
  //   r0 + 8 half (+ 16 uu, a constant 4096 bytes), d = 32 db + 16 g2 + 4 (i16 % 4).
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
        voff[db][half] = W1_TILEB + row * W1_ROWB + (((4 * db + cb) ^ row_swz(row)) << 4) + (i16 & 1) * 8;
      }
  }
  //   DMA: this wavefront copies rows 4 NI wq .. 4 NI (wq + 1) - 1 of each
  //   tile, as NI 1 KB instructions n = NI wq + u (rows 4 n .. 4 n + 3); lane l
  //   fills row 4 n + l / 16, physical chunk l % 16.  Chunks past d read as zero.
  // The first NI entries are used.  (With a size that depends on the template
  // parameters, hipcc emitted no host launch stub for the kernel.)
  int dk[4], dv[4];
#pragma unroll
  for (int u = 0; u < NI; ++u) {
    const int row = 4 * (NI * wq + u) + (lane >> 4);
    const int lc = (lane & 15) ^ row_swz(row);
    const bool ok = lc * 8 < dlim;
    dk[u] = ok ? 2 * (row * (int)p.k_ss + lc * 8) : 0x40000000;
    dv[u] = ok ? 2 * (row * (int)p.v_ss + lc * 8) : 0x40000000;
  }

  long u0, u1;
  const int vidx = wg_range_x<F>(w, p.H, u0, u1);  // this workgroup's range index and units [u0, u1)

  // The segment of the range that ends with unit u (fsched::decode_seg).
  auto decode = [&](long u) __attribute__((always_inline)) { return decode_seg_x<F>(u, u0, w); };
  bf16x8 qf[QH][NQF];
  auto load_q = [&](const Seg& sg) __attribute__((always_inline)) {
    const bf16* Q = static_cast<const bf16*>(p.q) + (long)sg.hh * p.q_sh;
#pragma unroll
    for (int hq = 0; hq < QH; ++hq) {
      const int qrow = QB * sg.b + QW * wq + 32 * hq + l32;
#pragma unroll
      for (int f = 0; f < NQF; ++f) {
        const int dd = 16 * f + 8 * h32;
        qf[hq][f] = __builtin_bit_cast(bf16x8, ld16_or_zero(Q, (long)qrow * p.q_ss + dd, qrow < S && dd < dlim));
      }
    }
  };
  // Copies tile j (0-based within the segment) of K and V into LDS stage st;
  // tiles past the segment copy zeros (no memory is read).
  auto dma = [&](const Seg& sg, int j, int st) __attribute__((always_inline)) {
    const int tj = sg.t0 + j;
    const int k0 = tj * BN;
    const int nkeys = tj < sg.t1 ? min(BN, S - k0) : 0;
    const int kbytes = nkeys > 0 ? 2 * ((nkeys - 1) * (int)p.k_ss + dlim) : 0;
    const int vbytes = nkeys > 0 ? 2 * ((nkeys - 1) * (int)p.v_ss + dlim) : 0;
    const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(static_cast<const bf16*>(p.k) + (long)(sg.hh / p.group) * p.k_sh + (long)k0 * p.k_ss), (short)0, kbytes,
        kBufferFlags);
    const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(static_cast<const bf16*>(p.v) + (long)(sg.hh / p.group) * p.v_sh + (long)k0 * p.v_ss), (short)0, vbytes,
        kBufferFlags);
    // The stage's LDS address goes through an empty asm: with a destination
    // it can see, the compiler makes every later LDS read wait for all
    // outstanding copies (vmcnt(0)), which leaves one tile in flight; the
    // per-stage vmcnt waits and the barrier order the copies and reads.
    const unsigned sbase = opaque_lds_addr(lds + st * W1_STAGEB);
#pragma unroll
    for (int u = 0; u < NI; ++u) {
      const int n = NI * wq + u;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, lds_ptr(sbase + n * 1024), 16, dk[u], 0, 0, 0);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, lds_ptr(sbase + W1_TILEB + n * 1024), 16, dv[u], 0, 0, 0);
    }
  };

  Seg cur = decode(u1 - 1);
  load_q(cur);

  for (;;) {
    const int hh = cur.hh, b = cur.b, t0 = cur.t0, t1 = cur.t1, nt_b = cur.nt;
    const long bstart = cur.bstart;
    const int qw = QB * b + QW * wq;  // first query of this wavefront
    const int nt = t1 - t0;

#pragma unroll
    for (int j = 0; j < W1_NS - 1; ++j) dma(cur, j, j);
    wait_vm<(W1_NS - 2) * LPT>();  // tile 0 has landed (and Q)
    __syncthreads();

    float m_run[QH], l_run[QH];
    floatx16 oacc[QH][NDB];
#pragma unroll
    for (int hq = 0; hq < QH; ++hq) {
      m_run[hq] = -INFINITY;
      l_run[hq] = 0.f;
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int e = 0; e < 16; ++e) oacc[hq][db][e] = 0.f;
    }

    // Software pipeline, per tile i (two scheduling regions, each a
    // fixed interleave of MFMA and VALU instructions):
    //   region 1: S(i+1) = K(i+1) Q^T     x  exp, row sums, bf16 P(i)
    //   region 2: O += P(i) V(i)          x  mask and row max of S(i+1)
    //   then the lazy rescale decision for tile i+1.
    // Every tile runs the same instructions: keys past a query or past the
    // segment are masked to -inf, so a tile wholly above a wavefront's
    // diagonal contributes exact zeros.
    const int klim_seg = (t0 + nt) * BN;  // keys at or past this are outside the segment
    auto mask_max = [&](int j, int hq, floatx16& sc) __attribute__((always_inline)) {
      const int k0 = (t0 + j) * BN;
      const int lim = min(qw + 32 * hq + l32, klim_seg - 1);  // last key this query may see in the segment
      float mx = -INFINITY;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        sc[e] = k0 + 8 * (e >> 2) + 4 * h32 + (e & 3) > lim ? -INFINITY : sc[e];
        mx = fmaxf(mx, sc[e]);
      }
      return mx;
    };
    auto plain_max = [&](const floatx16& sc) __attribute__((always_inline)) {
      float mx = sc[0];
#pragma unroll
      for (int e = 1; e < 16; ++e) mx = fmaxf(mx, sc[e]);
      return mx;
    };
    // Tile j needs masking when it reaches past this wavefront's first query
    // (tile index t0 + j >= qw / BN) or lies outside the segment; the tiles
    // j >= jm of the segment do.  jm is uniform over the wavefront.
    const int jm = __builtin_amdgcn_readfirstlane(max(0, min(nt, qw / BN - t0)));
    // Raises the running maxima when a tile's max exceeds one by the slack
    // (rescaling O and l after the P V of the previous tile).
    auto rescale = [&](float (&mx)[QH]) __attribute__((always_inline)) {
      bool up = false;
#pragma unroll
      for (int hq = 0; hq < QH; ++hq) {
        mx[hq] = max_xor32(mx[hq]) * c;
        up = up || mx[hq] > m_run[hq] + kRescaleSlack;
      }
      if (__builtin_amdgcn_ballot_w64(up)) {
#pragma unroll
        for (int hq = 0; hq < QH; ++hq) {
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
    // exp2 of scaled scores e0 .. e1 - 1 of half hq, added to the row sum.
    auto expo = [&](floatx16& sc, float mneg, float& rs, int e0, int e1) __attribute__((always_inline)) {
#pragma unroll
      for (int e = e0; e < e1; ++e) {
        sc[e] = fast_exp2(fmaf(sc[e], c, mneg));
        rs += sc[e];
      }
    };
    auto to_p = [&](const floatx16& sc, int uu, bf16x8& pf) __attribute__((always_inline)) {
#pragma unroll
      for (int j = 0; j < 8; ++j) pf[j] = (bf16)sc[8 * uu + j];
    };
    // The V^T reads are untracked (ds_read_tr16_b64_async): the builtin
    // transposed read would make the compiler wait for every outstanding copy
    // first, leaving no tile in flight.  vties() orders them before P V.
    auto kfrags = [&](int st, bf16x8 (&kf)[NQF]) __attribute__((always_inline)) {
      const unsigned char* sb = lds + st * W1_STAGEB;
#pragma unroll
      for (int f = 0; f < NQF; ++f) kf[f] = *reinterpret_cast<const bf16x8*>(sb + koff[f]);
    };
    auto vfrags = [&](int st, bf16x8 (&a)[NDB][2]) __attribute__((always_inline)) {
      const unsigned char* sb = lds + st * W1_STAGEB;
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int uu = 0; uu < 2; ++uu) {
          const shortx4 x = ds_read_tr16_b64_async(sb + voff[db][0] + 4096 * uu);
          const shortx4 y = ds_read_tr16_b64_async(sb + voff[db][1] + 4096 * uu);
          a[db][uu] = __builtin_bit_cast(bf16x8, __builtin_shufflevector(x, y, 0, 1, 2, 3, 4, 5, 6, 7));
        }
    };
    // Every LDS read so far has landed; P V uses the tied V^T fragments.
    auto vties = [&](bf16x8 (&a)[NDB][2]) __attribute__((always_inline)) {
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int uu = 0; uu < 2; ++uu) lds_wait_tie(a[db][uu]);
    };

    auto pv = [&](int hq, const bf16x8 (&va)[NDB][2], const bf16x8 (&pf)[2]) __attribute__((always_inline)) {
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int uu = 0; uu < 2; ++uu) oacc[hq][db] = MF::mma(va[db][uu], pf[uu], oacc[hq][db]);
    };

    floatx16 s0[QH], s1[QH];
    {  // S(0), its mask, max and rescale
      bf16x8 kf[NQF];
      kfrags(0, kf);
      const bool msk = jm == 0;
      float mx[QH];
#pragma unroll
      for (int hq = 0; hq < QH; ++hq) {
#pragma unroll
        for (int e = 0; e < 16; ++e) s0[hq][e] = 0.f;
#pragma unroll
        for (int f = 0; f < NQF; ++f) s0[hq] = MF::mma(kf[f], qf[hq][f], s0[hq]);
        mx[hq] = msk ? mask_max(0, hq, s0[hq]) : plain_max(s0[hq]);
      }
      rescale(mx);
    }
    // Software pipeline, per tile i.  With one half (32 queries):
    //   region 1: S(i+1) = K(i+1) Q^T     x  exp, row sums, bf16 P(i)
    //   region 2: O += P(i) V(i)          x  mask and row max of S(i+1)
    // With two halves the exp work of S(i) is spread over the QK MFMAs and the
    // P V MFMAs of half 0, which need only half 0's P:
    //   region 1: S(i+1), both halves     x  exp of half 0, first 8 keys of half 1
    //   region 2: O(half 0) += P V        x  exp of half 1's last 8 keys
    //   region 3: O(half 1) += P V        x  mask and row max of S(i+1)
    // A step either masks S(i+1) or does not (a compile-time choice), so that
    // no branch separates MFMAs that update O and every P V updates O in place.
    auto step = [&](auto masked, int i, int st, floatx16 (&sc)[QH], floatx16 (&sn)[QH])
                    __attribute__((always_inline)) {
      constexpr bool MSK = decltype(masked)::value;
      const int st1 = (st + 1) % W1_NS, stp = (st + W1_NS - 1) % W1_NS;
      wait_vm<(W1_NS - 3) * LPT>();  // tile i+1 has landed
      // ... for every wavefront; all are done with tile i-1.  A bare barrier:
      // __syncthreads()' fence would wait for every outstanding copy.
      __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wavefront's LDS reads are done
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
      __builtin_amdgcn_s_barrier();
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
      dma(cur, i + W1_NS - 1, stp);  // into tile i-1's stage
      bf16x8 kf[NQF], va[NDB][2];
      kfrags(st1, kf);  // every fragment read of the tile is in flight
      vfrags(st, va);   // before the first MFMA waits for one
      __builtin_amdgcn_sched_barrier(0);
      float mneg[QH], rs[QH];
#pragma unroll
      for (int hq = 0; hq < QH; ++hq) {
        mneg[hq] = m_run[hq] == -INFINITY ? 0.f : -m_run[hq];  // an empty row keeps exp2(-inf) = 0
        rs[hq] = 0.f;
#pragma unroll
        for (int e = 0; e < 16; ++e) sn[hq][e] = 0.f;
      }
      bf16x8 pf[QH][2];
      // ---- region 1
#pragma unroll
      for (int f = 0; f < NQF; ++f)
#pragma unroll
        for (int hq = 0; hq < QH; ++hq) sn[hq] = MF::mma(kf[f], qf[hq][f], sn[hq]);
      expo(sc[0], mneg[0], rs[0], 0, 16);
      to_p(sc[0], 0, pf[0][0]);
      to_p(sc[0], 1, pf[0][1]);
      if constexpr (QH == 2) {
        expo(sc[1], mneg[1], rs[1], 0, 8);
        to_p(sc[1], 0, pf[1][0]);
      }
#pragma unroll
      for (int f = 0; f < NQF * QH; ++f) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);             // one MFMA
        __builtin_amdgcn_sched_group_barrier(0x002, QH == 1 ? 6 : 5, 0);  // VALU
      }
      __builtin_amdgcn_sched_barrier(0);
      vties(va);
      if constexpr (QH == 2) {
        // ---- region 2
        pv(0, va, pf[0]);
        expo(sc[1], mneg[1], rs[1], 8, 16);
        to_p(sc[1], 1, pf[1][1]);
#pragma unroll
        for (int k = 0; k < 2 * NDB; ++k) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 3);
          __builtin_amdgcn_sched_group_barrier(0x002, 4, 3);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int hq = 0; hq < QH; ++hq) l_run[hq] += rs[hq];
      // ---- last region: P V of the last half x (mask and) max of S(i+1)
      float mx[QH];
      pv(QH - 1, va, pf[QH - 1]);
      if constexpr (MSK) {
#pragma unroll
        for (int hq = 0; hq < QH; ++hq) mx[hq] = mask_max(i + 1, hq, sn[hq]);
#pragma unroll
        for (int k = 0; k < 2 * NDB; ++k) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);
          __builtin_amdgcn_sched_group_barrier(0x002, 5 * QH, 1);
        }
      } else {
#pragma unroll
        for (int hq = 0; hq < QH; ++hq) mx[hq] = plain_max(sn[hq]);
#pragma unroll
        for (int k = 0; k < 2 * NDB; ++k) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 2);
          __builtin_amdgcn_sched_group_barrier(0x002, 2 * QH, 2);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
      rescale(mx);
    };
    // Steps i whose S(i+1) needs no mask (i + 1 < jm) run four at a time from
    // stage 0; the rest mask every tile.
    static_assert(W1_NS == 4, "the loops below are unrolled by the stage count");
    constexpr std::integral_constant<bool, false> kPlain{};
    constexpr std::integral_constant<bool, true> kMasked{};
    int i = 0;
#pragma unroll 1
    for (; i + 4 < jm; i += 4) {
      step(kPlain, i, 0, s0, s1);
      step(kPlain, i + 1, 1, s1, s0);
      step(kPlain, i + 2, 2, s0, s1);
      step(kPlain, i + 3, 3, s1, s0);
    }
#pragma unroll 1
    for (; i < nt; ++i) {  // one step per iteration (stage from i, S(i+1) moved into s0)
      step(kMasked, i, i & (W1_NS - 1), s0, s1);
#pragma unroll
      for (int hq = 0; hq < QH; ++hq) s0[hq] = s1[hq];
    }
    __builtin_amdgcn_s_waitcnt(0);  // the copies of tiles past the segment have landed
    __syncthreads();

    float l_tot[QH];
#pragma unroll
    for (int hq = 0; hq < QH; ++hq) l_tot[hq] = sum_xor32(l_run[hq]);
    auto weights = [&](int hq, float m2, float l2, float& a1, float& a2) __attribute__((always_inline)) {
      const float M = fmaxf(m_run[hq], m2);
      a1 = m_run[hq] == -INFINITY ? 0.f : fast_exp2(m_run[hq] - M);
      a2 = m2 == -INFINITY ? 0.f : fast_exp2(m2 - M);
      l_tot[hq] = l_tot[hq] * a1 + l2 * a2;
      m_run[hq] = M;
    };
    auto store_out = [&]() __attribute__((always_inline)) {
#pragma unroll
      for (int hq = 0; hq < QH; ++hq) {
        const float linv = 1.0f / l_tot[hq];
        const int myq = qw + 32 * hq + l32;
        if (myq < S) {
          bf16* orow = static_cast<bf16*>(p.o) + (long)hh * p.o_sh + (long)myq * p.o_ss;
#pragma unroll
          for (int db = 0; db < NDB; ++db)
#pragma unroll
            for (int bq = 0; bq < 4; ++bq) {
              const int dd = 32 * db + 8 * bq + 4 * h32;
              if (dd < dlim) {
                float ov[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) ov[e] = oacc[hq][db][4 * bq + e] * linv;
                store_vec<4>(orow + dd, ov);
              }
            }
        }
      }
    };

    const long next_u = bstart + t0 - 1;  // the last unit of the previous segment
    const bool more = next_u >= u0;
    Seg nxt = cur;
    if (more) nxt = decode(next_u);

    int nparts = 1, vf = vidx;
    if (w.sched == kBalanced) {
      vf = range_of_x<F>(bstart, w);
      nparts = range_of_x<F>(bstart + nt_b - 1, w) - vf + 1;
    }
    if (nparts == 1) {
      store_out();
      if (more) load_q(nxt);
    } else {
      typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
      const __amdgpu_buffer_rsrc_t prsrc = __builtin_amdgcn_make_buffer_rsrc(w.part, (short)0, w.part_bytes, kBufferFlags);
      auto poff = [&](int v, int s2, int hq, int k) __attribute__((always_inline)) {
        return 4 * (((v * 2 + s2) * PART) + wq * SLOT + hq * HS + k * 256 + 4 * lane);
      };
      const int slot = range_start_x<F>(vidx, w) >= bstart ? 0 : 1;
      const int vl = vf + nparts - 1;
      if (vidx == vl) await_parts(&w.count[hh * w.nqb + b], nparts, w.polls, arrival);
      const bool stored = vidx != vl || arrival != nparts - 1;
#pragma unroll
      for (int hq = 0; hq < QH && stored; ++hq) {
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
          for (int k = 0; k < 4; ++k)
            __builtin_amdgcn_raw_buffer_store_b128(
                __builtin_bit_cast(u32x4, make_float4(oacc[hq][db][4 * k], oacc[hq][db][4 * k + 1],
                                                      oacc[hq][db][4 * k + 2], oacc[hq][db][4 * k + 3])),
                prsrc, poff(vidx, slot, hq, 4 * db + k), 0, kDeviceCoherent);
        __builtin_amdgcn_raw_buffer_store_b128(
            __builtin_bit_cast(u32x4, make_float4(m_run[hq], l_tot[hq], 0.f, 0.f)), prsrc,
            poff(vidx, slot, hq, NCO), 0, kDeviceCoherent);
      }
      if (stored) {
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (tid == 0) arrival = atomicAdd(&w.count[hh * w.nqb + b], 1);
      }
      if (more) load_q(nxt);
      __syncthreads();
      if (arrival == nparts - 1) {
        // Folded last range first, whichever workgroup arrived last (the
        // order of the teams kernel above): bitwise reproducible.
        if (vidx != vl) {
#pragma unroll
          for (int hq = 0; hq < QH; ++hq) {
            m_run[hq] = -INFINITY;
            l_tot[hq] = 0.f;
#pragma unroll
            for (int db = 0; db < NDB; ++db)
#pragma unroll
              for (int e = 0; e < 16; ++e) oacc[hq][db][e] = 0.f;
          }
        }
#pragma unroll 1
        for (int v2 = vl; v2 >= vf; --v2) {
          if (v2 == vidx && vidx == vl) continue;
          const int slot2 = range_start_x<F>(v2, w) >= bstart ? 0 : 1;
#pragma unroll
          for (int hq = 0; hq < QH; ++hq) {
            // (m, l) first, then O one d-block (4 float4 per lane) at a time.
            const float4 ml = __builtin_bit_cast(
                float4, __builtin_amdgcn_raw_buffer_load_b128(prsrc, poff(v2, slot2, hq, NCO), 0, kDeviceCoherent));
            float a1, a2;
            weights(hq, ml.x, ml.y, a1, a2);
#pragma unroll
            for (int db = 0; db < NDB; ++db) {
              float4 v[4];
#pragma unroll
              for (int k = 0; k < 4; ++k)
                v[k] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(
                                                      prsrc, poff(v2, slot2, hq, 4 * db + k), 0, kDeviceCoherent));
#pragma unroll
              for (int k = 0; k < 4; ++k) {
                floatx16& o = oacc[hq][db];
                o[4 * k] = fmaf(v[k].x, a2, o[4 * k] * a1);
                o[4 * k + 1] = fmaf(v[k].y, a2, o[4 * k + 1] * a1);
                o[4 * k + 2] = fmaf(v[k].z, a2, o[4 * k + 2] * a1);
                o[4 * k + 3] = fmaf(v[k].w, a2, o[4 * k + 3] * a1);
              }
            }
          }
        }
        store_out();
        if (tid == 0) atomicExch(&w.count[hh * w.nqb + b], 0);
      }
    }
    __syncthreads();
    if (!more) break;
    cur = nxt;
  }
}

// ------------------------------------------------------------------ host --

namespace {

int cu_count() {
  int dev = 0, n = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) return 256;
  return n;
}

// Kernels: teams of wavefronts sharing SIMDs (8 wavefronts per workgroup, or
// 4 with two workgroups per CU); the software-pipelined kernel with one
// wavefront per SIMD and 32 queries (4 per workgroup) or 64 queries (2 or 4
// per workgroup); or that kernel with 32 queries at two wavefronts per SIMD
// (256 registers each, two independent workgroups per CU); or the
// 64-key-tile kernel of flash_fwd.hip (kFwd: 128-query blocks, two
// wavefronts per SIMD splitting each tile's keys, LDS-DMA stages).
enum Kern {
  kTeams = 0,
  kW32x4 = 1,
  kW64x2 = 2,
  kW64x4 = 3,
  kTeams4 = 4,
  kW32x4x2 = 5,
  kFwd = 6,
  kFwdPP = 7,
  kKS = 8,
  kTiny = 9
};

// Launch-configuration overrides (-1: the automatic choice), process-wide:
// read from the environment once, at first use -- NKL_FLASH_SCHEDULE=
// block|pairs|balanced, NKL_FLASH_QB=64|128,
// NKL_FLASH_KERNEL=teams|teams4|w1|w1o2|w64|w64x4|fwd|pp|ks|tiny, NKL_FLASH_CPB=<units>
// -- or set by nkl_flash_attn_configure() (tests, tuning), so that a
// workspace sized by one call fits the launch of the next.
struct Overrides {
  int sched = -1, qb = -1, kern = -1, cpb = -1;
  int polls = -1;  // the merging workgroup's poll budget (-1: the automatic choice in plan())
};
Overrides& overrides() {
  static Overrides o = [] {
    Overrides r;
    if (const char* f = getenv("NKL_FLASH_SCHEDULE")) {
      if (!strcmp(f, "block")) r.sched = kBlock;
      if (!strcmp(f, "pairs")) r.sched = kPairs;
      if (!strcmp(f, "balanced")) r.sched = kBalanced;
    }
    if (const char* f = getenv("NKL_FLASH_QB")) {
      if (!strcmp(f, "64")) r.qb = 64;
      if (!strcmp(f, "128")) r.qb = 128;
    }
    if (const char* f = getenv("NKL_FLASH_KERNEL")) {
      if (!strcmp(f, "teams")) r.kern = kTeams;
      if (!strcmp(f, "teams4")) r.kern = kTeams4;
      if (!strcmp(f, "w1")) r.kern = kW32x4;
      if (!strcmp(f, "w1o2")) r.kern = kW32x4x2;
      if (!strcmp(f, "w64")) r.kern = kW64x2;
      if (!strcmp(f, "w64x4")) r.kern = kW64x4;
      if (!strcmp(f, "fwd")) r.kern = kFwd;
      if (!strcmp(f, "pp")) r.kern = kFwdPP;
      if (!strcmp(f, "ks")) r.kern = kKS;
      if (!strcmp(f, "tiny")) r.kern = kTiny;
    }
    if (const char* f = getenv("NKL_FLASH_CPB")) r.cpb = min(max(atoi(f), 0), 4096);
    return r;
  }();
  return o;
}

}  // namespace

int flash_bf16_configure(int kern, int sched, int qb, int cpb) {
  if (kern < -1 || kern > kTiny || sched < -1 || sched > kPairs || (qb != -1 && qb != 64 && qb != 128) || cpb < -1 ||
      cpb > 4096)
    return set_error(NKL_EINVAL, "nkl_flash_attn_configure: kernel %d, schedule %d, qb %d, cpb %d out of range", kern,
                     sched, qb, cpb);
  Overrides& o = overrides();
  o.kern = kern;
  o.sched = sched;
  o.qb = qb;
  o.cpb = cpb;
  return NKL_OK;
}

int flash_bf16_configure_polls(int polls) {
  if (polls < -1 || polls > (1 << 20))
    return set_error(NKL_EINVAL, "nkl_flash_attn_configure_polls: %d outside [-1, 2^20]", polls);
  overrides().polls = polls;
  return NKL_OK;
}

namespace {

// A launch configuration: queries per block, a schedule and a kernel.  The
// teams kernel takes 64-query blocks (2 wavefronts x 4 teams, or x 2 teams in
// its 4-wavefront form) or 128-query blocks (4 wavefronts x 2 teams, or one
// team); the others take 32 or 64 queries per wavefront times their
// wavefront count.
struct Config {
  int qb;
  int sched;
  int kern;
};

// Resident workgroups per CU: two for the two-wavefront kernel, else one.
int wgs_per_cu(int kern) { return kern == kW64x2 || kern == kTeams4 || kern == kW32x4x2 ? 2 : 1; }

Work plan(int H, int S, Config cfg) {
  Work w{};
  const bool fwd = cfg.kern == kFwd || cfg.kern == kFwdPP;
  const int bn = fwd ? 64 : BN;  // keys per tile
  w.tpb = cfg.qb / bn;
  w.nqb = (S + cfg.qb - 1) / cfg.qb;
  w.last_nt = (S - 1) / bn + 1;
  w.units_head = (long)w.tpb * (w.nqb - 1) * w.nqb / 2 + w.last_nt;
  w.units = (long)H * w.units_head;
  w.sched = cfg.sched;
  w.paired = cfg.sched != kBlock;
  if (cfg.sched == kBalanced) {
    // As many workgroups as are resident at once, and no range shorter than
    // kMinUnits: a short range spends most of its time filling the pipeline,
    // and splits a block into many parts for its last workgroup to merge.
    const long by_size = (w.units + kMinUnits - 1) / kMinUnits;
    const int cus = cu_count() * wgs_per_cu(cfg.kern);
    w.grid = (int)(by_size < cus ? by_size : cus);
    // Block start cost, in units: about a segment's fixed work over the time
    // of one unit in the loop, tuned on MI355X with rotating inputs.  With
    // fewer blocks than workgroups every block is split and a higher cost
    // pays (teams kernel, 128-query blocks: 6 against 12 since every
    // segment's Q is staged in LDS, 8 x 2048 25.3 -> 24.4-24.8 us, 12 x 2048
    // 31.5 -> 29.9, 6 x 2048 24.6 -> 24.0); with at least as many, 4 is best
    // (16 x 2048, 8 x 4096, 4 x 8192).  64-query blocks:
    // 18 and 10 (1 x 4096: 32.3 -> 24.6 us at 14 against no cost, 23.4 ->
    // 23.0 at 18; 4 x 2048 21.4 -> 20.5); the pipelined
    // kernel's longer segments gain little.  At most a range's cost minus
    // one, so that every range holds a unit.
    const bool pipelined = cfg.kern == kW32x4 || cfg.kern == kW64x2 || cfg.kern == kW64x4 || cfg.kern == kW32x4x2;
    const long nblocks = (long)H * w.nqb;
    const bool few = nblocks < w.grid;
    int cpb = fwd ? (few ? 4 : 2) : pipelined ? 2 : cfg.kern == kKS ? (few ? 8 : 6) : cfg.qb == 64 ? (few ? 18 : 10) : (few ? 6 : 4);
    if (overrides().cpb >= 0) cpb = overrides().cpb;
    while (cpb > 0 && (w.units + nblocks * cpb) / w.grid < cpb + 1) --cpb;
    w.cpb = cpb < 0 ? 0 : cpb;
  } else if (cfg.sched == kPairs) {
    w.grid = H * ((w.nqb + 1) / 2);
  } else {
    w.grid = H * w.nqb;
  }
  w.cost = w.units + (long)H * w.nqb * w.cpb;
  // The merging workgroup's poll budget (fsched::await_parts).  Waiting pays
  // while a split block has few parts; when the longest block spans six or
  // more ranges, the holder of its last range storing its state and leaving
  // the merge to the last part to arrive is faster (one session, us: 1 x 4096
  // 21.3-21.6 -> 20.0, 2 x 2048 18.3-18.5 -> 17.1, 1 x 2048 19.7-19.8 ->
  // 17.4; with fewer parts it was slower: 4 x 2048 18.7-18.9 -> 19.3,
  // 16 x 2048 31.0-31.3 -> 32.6).  256 polls (~0.15 ms) bound the wait when
  // the other parts cannot run (another kernel holding the CUs); budgets of
  // 16 to 4096 timed the same.
  if (overrides().polls >= 0)
    w.polls = overrides().polls;
  else
    w.polls = cfg.sched == kBalanced && (long)w.last_nt * w.grid >= kNoWaitParts * w.units ? 0 : kPolls;
  // 32-bit schedule arithmetic with magic divisors when every value fits in
  // an int: the largest are (cost + 1) grid (fsched::range_of) and r + delta
  // < 2 head_cost <= 2 cost (the pair index), both at most (cost + 1)
  // max(grid, 2).
  const long full = (long)w.tpb * (w.nqb + 1);
  const long fcost = full + 2L * w.cpb;
  const long head_cost = w.units_head + (long)w.nqb * w.cpb;
  w.fast = (w.cost + 1) * (long)(w.grid > 2 ? w.grid : 2) < (1L << 31);
  if (w.fast) {
    w.dv_units_head = make_div32((unsigned)w.units_head);
    w.dv_full = make_div32((unsigned)full);
    w.dv_fcost = make_div32((unsigned)fcost);
    w.dv_head_cost = make_div32((unsigned)head_cost);
    w.dv_grid = make_div32((unsigned)w.grid);
    w.dv_cost = make_div32((unsigned)w.cost);
  }
  return w;
}

// Schedule and kernel choice, from measured launches on MI355X (units of
// 128-query blocks per CU): below 12, 64-query blocks halve the unit and keep
// every CU busy (1 x 4096: 8); up to 100 the 8-wavefront teams kernel over
// balanced ranges (whole blocks leave CUs idle or unevenly loaded; 6 x 2048:
// 24.5 us against 27.2 for the ping-pong kernel, 12 x 2048 30.8 against
// 31.6; with its 128-query merge folding parts as they arrive, one session,
// us: 24 x 2048 44.8 against 47.1, 28 x 2048 51.3 / 54.1, 40 x 2048 67.9 /
// 70.9, 2 x 8192 47.5 / 49.7, 10 x 4096 61.0 / 61.9, level at 32 x 2048 and
// 12 x 4096, 8 x 4096 47.1-47.4 / 46.8); up to 200 the ping-pong 64-key-tile
// kernel (flash_fwd.hip) for d > 64, whose steady state is faster (16 x 4096
// 83.5 against 85.8-86.1 us, 4 x 8192 78.9 against 81.7, 5 x 8192 102.2
// against 104.8; the teams kernel takes d <= 64 and fp16); from 200
// the software-pipelined kernel at two wavefronts per SIMD (d > 64), whose
// steady state is faster and whose longer segments amortise its start-up;
// from 1024 one workgroup per pair of blocks, which balances as well and
// needs no partial states.
// The overrides above replace the choice (tests, tuning); the
// one-wavefront-per-SIMD kernels and kFwd take 64 < d <= 128 and fix the block.
Config choose(int H, int S, int d, bool f16) {
  const long cus = cu_count();
  const long nqb = (S + 127) / 128;
  const long units128 = (long)H * (2 * (nqb - 1) * nqb + (S - 1) / BN + 1);
  Config cfg = units128 < 12 * cus     ? Config{64, kBalanced, kTeams}
               : units128 < 100 * cus  ? Config{128, kBalanced, kTeams}
               : units128 < 200 * cus  ? Config{128, kBalanced, kFwdPP}
               : units128 < 1024 * cus ? Config{128, kBalanced, kW32x4x2}
                                       : Config{128, kPairs, kW32x4x2};
  if (cfg.qb == 64) {
    // One workgroup per 64-query block when every block fits one round of
    // workgroups and the heaviest block (S / 32 key tiles) exceeds a balanced
    // range by at most 18 tiles: a block alone then ends before ranges that
    // pay the partial-state stores and merges of split blocks (about 6 us,
    // or 18 tiles of the loop, more fixed cost than a whole block).  Inputs
    // rotated through twice the last-level cache, one session, us (blocks /
    // balanced ranges): 4 x 768 15.4 / 15.7, 14 x 1024 19.2 / 20.5, 1 x 768
    // and 12 x 1024 level; 10 x 1024 18.8 / 17.9, 8 x 1536 24.2 / 21.0.
    // With more blocks than a round holds, 128-query blocks over balanced
    // ranges (same protocol, us: 40 x 512 18.3 -> 16.0, 64 x 512 22.2 ->
    // 18.2, 20 x 1024 level).
    const long nqb64 = ((long)S + 63) / 64;
    const long units64 = (long)H * (2 * (nqb64 - 1) * nqb64 / 2 + (S - 1) / BN + 1);
    const long range = units64 / cus > kMinUnits ? units64 / cus : kMinUnits;
    if ((long)H * nqb64 > cus)
      cfg = Config{128, kBalanced, kTeams};
    else if ((S - 1) / BN + 1 <= range + 18)
      cfg.sched = kBlock;
  }
  // Up to 224 positions (64 < d <= 128), the one-pass kernel: every key row a
  // 128-query block sees is staged in LDS at once, and nothing is handed over
  // or merged (same session against one workgroup per 64-query block, us:
  // 1 x 64 4.6 / 7.4, 1 x 128 6.0 / 7.9, 16 x 128 6.3 / 8.1, 2 x 200 7.4 /
  // 9.0; 256 x 224 23.5 against 36.1-37.9; with inputs rotated through twice
  // the last-level cache, against the teams kernel: 1 x 64 5.1 / 7.2, 1 x 128
  // 7.1 / 8.2, 16 x 128 7.7 / 8.6, 2 x 200 8.7 / 10.1).  Up to 256 while the
  // launch is small enough for 64-query blocks (LLC-resident inputs, one
  // session against the default before this rule, us: 1 x 232 8.1 / 9.0,
  // 1 x 256 8.2 / 9.0, 8 x 256 8.9 / 9.3, 128 x 256 13.5 / 19.8; rotated
  // inputs: 1 x 256 9.95 / 10.17, 8 x 256 and 128 x 256 level); from there
  // the 128-query teams kernel is faster (256 x 256 23.0 against 25.1).
  // Either way while its workgroups (one per head and 128-query block) fit
  // one round, or the launch is too small for balanced ranges to give every
  // CU kMinUnits units, or every head is one 64-query tile pair; past that,
  // 128-query teams over balanced ranges (inputs rotated through twice the
  // last-level cache, two sessions, us: 512 x 128 20.2 against 22.1-22.2,
  // 1024 x 128 38.3 against 41.8, 256 x 224 22.9 against 23.9-24.1; the
  // one-pass kernel stays at 256 x 128, one round: 11.6 against 17.3,
  // 257 x 128, 129 ranges: 18.1 against 24.2, and 1024 x 64: 23.7 against
  // 26.7).
  const bool tiny_fits = (long)H * nqb <= cus || units128 < kMinUnits * cus || S <= 64;
  if (d > 64 && d <= 128 && (S <= kTinyAutoS || (S <= kTinyMaxS && cfg.qb == 64)) && tiny_fits)
    cfg = Config{128, kBlock, kTiny};
  const Overrides& ov = overrides();
  if (ov.sched >= 0) cfg.sched = ov.sched;
  if (ov.qb >= 0) cfg.qb = ov.qb;
  if (ov.kern >= 0) cfg.kern = ov.kern;
  if (d <= 64 && cfg.kern != kTeams4) cfg.kern = kTeams;
  if (f16 && cfg.kern != kTeams4 && cfg.kern != kKS && cfg.kern != kTiny)
    cfg.kern = kTeams;  // fp16: the teams, key-split and short-sequence kernels
  if (cfg.kern == kW32x4 || cfg.kern == kW64x2 || cfg.kern == kW32x4x2 || cfg.kern == kFwd || cfg.kern == kFwdPP)
    cfg.qb = 128;
  if (cfg.kern == kW64x4) cfg.qb = 256;
  if (cfg.kern == kKS && (d <= 64 || d > 128)) cfg.kern = kTeams;  // the key-split kernel: 64 < d <= 128
  if (cfg.kern == kKS) cfg.qb = 64;
  if (cfg.kern == kTiny && (S > kTinyMaxS || d <= 64 || d > 128)) cfg.kern = kTeams;
  if (cfg.kern == kTiny) cfg = Config{128, kBlock, kTiny};  // one workgroup per 128-query block
  return cfg;
}

// Floats of one workgroup's partial state (one of its two slots).  Every
// kernel stores (O, m, l) of each 32-query group as 4 * (d / 8 + 1) float4
// per lane, so the size depends on the block only.
template <int D>
size_t part_floats(int qb) {
  return qb == 64 ? Layout<D, 2, 4>::PART : (size_t)(qb / 128) * Layout<D, 4, 2>::PART;
}

size_t part_floats_for(int d, const Config& cfg) {
  if (cfg.kern == kFwd || cfg.kern == kFwdPP) return flash_fwd_part_bytes() / 4;
  if (cfg.kern == kKS) return flash_ks_part_bytes() / 4;
  return d <= 32 ? part_floats<32>(cfg.qb) : d <= 64 ? part_floats<64>(cfg.qb) : part_floats<128>(cfg.qb);
}

// Kernels are instantiated twice over their schedule arithmetic: 32-bit only
// when the plan fits (Work::fast, every realistic shape), else 64-bit.
template <int D, int WPT, int NT>
void launch(const AttnArgs& a, const Work& w, hipStream_t st) {
  const dim3 grid((unsigned)w.grid), block(64 * WPT * NT);
  if (a.f16) {
    if (w.fast)
      flash_bf16_kernel<D, WPT, NT, true, true><<<grid, block, 0, st>>>(a, w);
    else
      flash_bf16_kernel<D, WPT, NT, true, false><<<grid, block, 0, st>>>(a, w);
  } else {
    if (w.fast)
      flash_bf16_kernel<D, WPT, NT, false, true><<<grid, block, 0, st>>>(a, w);
    else
      flash_bf16_kernel<D, WPT, NT, false, false><<<grid, block, 0, st>>>(a, w);
  }
}

template <int QH, int NW, int OCC = 1>
void launch_w(const AttnArgs& a, const Work& w, hipStream_t st) {
  if (w.fast)
    flash_bf16_w1_kernel<QH, NW, OCC, true><<<dim3((unsigned)w.grid), dim3(64 * NW), 0, st>>>(a, w);
  else
    flash_bf16_w1_kernel<QH, NW, OCC, false><<<dim3((unsigned)w.grid), dim3(64 * NW), 0, st>>>(a, w);
}

template <int D>
void launch_qb(const AttnArgs& a, const Work& w, int qb, int kern, hipStream_t st) {
  if (kern == kTeams4) {
    if (qb == 64)
      launch<D, 2, 2>(a, w, st);
    else
      launch<D, 4, 1>(a, w, st);
  } else if (qb == 64) {
    launch<D, 2, 4>(a, w, st);
  } else {
    launch<D, 4, 2>(a, w, st);
  }
}

}  // namespace

size_t flash_bf16_workspace_bytes(int H, int S, int d, bool f16) {
  if (H <= 0 || S <= 0) return 0;
  const Config cfg = choose(H, S, d, f16);
  if (cfg.sched != kBalanced) return 0;
  return (size_t)plan(H, S, cfg).grid * 2 * part_floats_for(d, cfg) * 4;
}

// The counters do not depend on d: one per 64-query block (the smallest
// block) whenever some head dim takes the balanced schedule for this shape.
size_t flash_bf16_counter_bytes(int H, int S) {
  if (H <= 0 || S <= 0) return 0;
  if (choose(H, S, 32, false).sched != kBalanced && choose(H, S, 128, false).sched != kBalanced) return 0;
  return (size_t)H * ((S + 63) / 64) * 4;
}

// Host-side check of the launch plan for an H x S x d call under the
// configuration in force: the work split the kernels walk, invariant by
// invariant.  Balanced ranges tile the units in order, none empty; walking a
// range from its last segment to its first (as the kernels do) covers its
// units exactly; range_of agrees with the range that holds a unit; a split
// block's parts are the ranges that hold its units, its last range the one
// that merges; no range puts two parts in one of its two partial-state
// slots.  Pairs and blocks: every block taken by exactly one workgroup.
// info (optional, 4 longs): grid, units, split blocks, largest part count.
int flash_bf16_plan_check(int H, int S, int d, bool f16, long* info) {
  if (H < 1 || S < 1 || d < 1 || d > 128)
    return set_error(NKL_EINVAL, "plan check: shape H=%d S=%d d=%d outside the kernels' range", H, S, d);
  const Config cfg = choose(H, S, d, f16);
  const Work w = plan(H, S, cfg);
  auto fail = [&](const char* what, long x, long y) {
    return set_error(NKL_EINVAL, "plan check H=%d S=%d d=%d (kernel %d, schedule %d, qb %d, cpb %d, grid %d): %s "
                     "(%ld, %ld)", H, S, d, cfg.kern, cfg.sched, cfg.qb, w.cpb, w.grid, what, x, y);
  };
  if (w.grid < 1) return fail("empty grid", w.grid, 0);
  std::vector<int> owner(w.units, -1);
  long split = 0, max_parts = 1;
  if (cfg.sched == kBalanced) {
    if (fsched::range_start(0, w) != 0) return fail("range 0 does not start at unit 0", fsched::range_start(0, w), 0);
    if (fsched::range_start(w.grid, w) != w.units)
      return fail("the last range does not end at the last unit", fsched::range_start(w.grid, w), w.units);
    std::vector<int> slot_used(2L * w.grid, 0);
    for (int v = 0; v < w.grid; ++v) {
      const long u0 = fsched::range_start(v, w), u1 = fsched::range_start(v + 1, w);
      if (u1 <= u0) return fail("empty range", v, u0);
      // The 32-bit instances (magic divisors) must agree with the 64-bit ones.
      if (w.fast && fsched::range_start_t<long>(v, w) != u0)
        return fail("32- and 64-bit range starts differ", u0, fsched::range_start_t<long>(v, w));
      long u = u1 - 1, covered = 0;
      for (int guard = 0; guard <= w.units; ++guard) {
        const fsched::Seg sg = fsched::decode_seg(u, u0, w);
        if (w.fast) {
          const fsched::Seg sl = fsched::decode_seg_t<long>(u, u0, w);
          if (sl.hh != sg.hh || sl.b != sg.b || sl.t0 != sg.t0 || sl.t1 != sg.t1 || sl.bstart != sg.bstart)
            return fail("32- and 64-bit segment decodes differ", u, sl.bstart);
        }
        if (sg.t0 < 0 || sg.t1 > sg.nt || sg.t0 >= sg.t1) return fail("segment tiles out of order", sg.t0, sg.t1);
        if (sg.bstart + sg.t1 - 1 != u) return fail("segment does not end at its unit", sg.bstart + sg.t1 - 1, u);
        if (sg.bstart + sg.t0 != (u0 > sg.bstart ? u0 : sg.bstart))
          return fail("segment does not start at its range or block", sg.bstart + sg.t0, u0);
        for (long x = sg.bstart + sg.t0; x < sg.bstart + sg.t1; ++x) {
          if (owner[x] != -1) return fail("unit covered twice", x, v);
          owner[x] = v;
          ++covered;
        }
        const int vf = fsched::range_of(sg.bstart, w), vl = fsched::range_of(sg.bstart + sg.nt - 1, w);
        if (vf > v || vl < v) return fail("range_of disagrees with the segment's range", vf, vl);
        if (vl > vf) {
          const int slot = fsched::range_start(v, w) >= sg.bstart ? 0 : 1;
          if (slot_used[2 * v + slot]++) return fail("two parts in one slot", v, slot);
          if (v == vf && sg.t0 != 0) return fail("the block's first part does not start it", v, sg.t0);
          if (v == vl && sg.t1 != sg.nt) return fail("the merging range does not end the block", v, sg.t1);
          if (v == vl) {
            ++split;
            max_parts = max_parts > vl - vf + 1 ? max_parts : vl - vf + 1;
          }
        }
        const long next_u = sg.bstart + sg.t0 - 1;
        if (next_u < u0) break;
        u = next_u;
      }
      if (covered != u1 - u0) return fail("a range's segments do not cover it", covered, u1 - u0);
    }
    for (long x = 0; x < w.units; ++x) {
      if (fsched::range_of(x, w) != owner[x]) return fail("range_of disagrees with the owner", x, owner[x]);
      if (w.fast && fsched::range_of_t<long>(x, w) != owner[x])
        return fail("32- and 64-bit range_of differ", x, fsched::range_of_t<long>(x, w));
    }
  } else {
    // One workgroup per pair of blocks (pairs) or per block (fsched::wg_range
    // for workgroup g), walked like a balanced range: whole blocks only.
    for (int g = 0; g < w.grid; ++g) {
      const int hh = g % H;
      long u0, u1;
      if (cfg.sched == kPairs) {
        const int k = g / H;
        u0 = (long)hh * w.units_head + fsched::pair_before(k, w);
        u1 = 2 * k + 2 <= w.nqb ? (long)hh * w.units_head + fsched::pair_before(k + 1, w) : (long)(hh + 1) * w.units_head;
      } else {
        const int b = w.nqb - 1 - g / H;
        u0 = (long)hh * w.units_head + fsched::plain_before(b, w);
        u1 = u0 + fsched::block_tiles(b, w);
      }
      if (u1 <= u0) return fail("empty workgroup", g, u0);
      long u = u1 - 1;
      for (int guard = 0; guard <= w.units; ++guard) {
        const fsched::Seg sg = fsched::decode_seg(u, u0, w);
        if (sg.t0 != 0 || sg.t1 != sg.nt) return fail("a block split without the balanced schedule", g, sg.t0);
        if (sg.bstart + sg.t1 - 1 != u) return fail("segment does not end at its unit", sg.bstart + sg.t1 - 1, u);
        for (long x = sg.bstart; x < sg.bstart + sg.nt; ++x) {
          if (x < 0 || x >= w.units) return fail("unit out of range", x, g);
          if (owner[x] != -1) return fail("unit covered twice", x, g);
          owner[x] = g;
        }
        const long next_u = sg.bstart - 1;
        if (next_u < u0) break;
        u = next_u;
      }
    }
  }
  for (long x = 0; x < w.units; ++x)
    if (owner[x] < 0) return fail("unit not covered", x, 0);
  if (info) {
    info[0] = w.grid;
    info[1] = w.units;
    info[2] = split;
    info[3] = max_parts;
    info[4] = cfg.sched == kBalanced ? w.polls : -1;
  }
  return NKL_OK;
}

int flash_bf16_launch(const AttnArgs& a, void* workspace, size_t workspace_bytes, int* counters,
                      size_t counter_bytes, hipStream_t st) {
  Config cfg = choose(a.H, a.S, a.d, a.f16 != 0);
  // The key-split kernel copies K and V rows with one stride; other layouts
  // take the teams kernel over the same 64-query blocks (whose partial states
  // have the same size).
  if (cfg.kern == kKS && (a.k_ss != a.v_ss || !(a.c > 0.f))) cfg.kern = kTeams;
  if (cfg.kern == kTiny && !flash_tiny_fits(a)) cfg.kern = kTeams;  // same blocks and schedule
  if (cfg.sched == kBalanced && !workspace) cfg.sched = kPairs;  // the plain entry point: no scratch
  Work w = plan(a.H, a.S, cfg);
  if (cfg.sched == kBalanced) {
    const size_t need = flash_bf16_workspace_bytes(a.H, a.S, a.d, a.f16 != 0);
    const size_t need_c = (size_t)a.H * w.nqb * 4;
    if (workspace_bytes < need || !counters || counter_bytes < need_c)
      return set_error(NKL_EWORKSPACE,
                       "nkl_flash_attn_causal_ws: workspace of %zu bytes and counters of %zu bytes needed, "
                       "%zu and %zu given", need, need_c, workspace_bytes, counter_bytes);
    w.part = static_cast<float*>(workspace);
    w.part_bytes = (int)need;
    w.count = counters;
  }
  if (cfg.kern == kTiny) {
    launch_flash_tiny(a, st);
    return check_launch("nkl_flash_attn_causal");
  }
  if (cfg.kern == kFwd || cfg.kern == kFwdPP) {
    launch_flash_fwd(a, w, cfg.kern == kFwdPP, st);
    return check_launch("nkl_flash_attn_causal");
  }
  if (cfg.kern == kKS && w.fast) {
    w.dv_group = make_div32((unsigned)a.group);
    launch_flash_ks(a, w, st);
    return check_launch("nkl_flash_attn_causal");
  }
  if (cfg.kern == kW32x4 || cfg.kern == kW64x2 || cfg.kern == kW64x4 || cfg.kern == kW32x4x2) {
    if (cfg.kern == kW32x4)
      launch_w<1, 4>(a, w, st);
    else if (cfg.kern == kW32x4x2)
      launch_w<1, 4, 2>(a, w, st);
    else if (cfg.kern == kW64x2)
      launch_w<2, 2>(a, w, st);
    else
      launch_w<2, 4>(a, w, st);
    return check_launch("nkl_flash_attn_causal");
  }
  if (a.d <= 32)
    launch_qb<32>(a, w, cfg.qb, cfg.kern, st);
  else if (a.d <= 64)
    launch_qb<64>(a, w, cfg.qb, cfg.kern, st);
  else
    launch_qb<128>(a, w, cfg.qb, cfg.kern, st);
  return check_launch("nkl_flash_attn_causal");
}

}  // namespace nkl
