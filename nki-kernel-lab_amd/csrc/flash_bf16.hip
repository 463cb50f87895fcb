// bf16 causal flash attention for gfx950 -- the hot path.
//
// Work decomposition.  Queries are grouped in blocks of QB = 128; keys in
// tiles of BN = 32.  A "unit" is one (head, query block, key tile) triple with
// the tile at or below the diagonal (tiles above it are never visited), so
// the causal triangle of S = 2048 holds 8 x 544 units.  With a workspace the
// units are cut into equal contiguous ranges, one per workgroup and one
// workgroup per CU (stream-K): a workgroup walks its range as segments (one
// segment per query block it touches), and a query block split across
// workgroups is finished by whichever of them arrives last, which merges the
// others' partial (max, sum, output) states from the workspace.  Without a
// workspace every workgroup takes one whole query block, heaviest first.
//
// Workgroup.  512 threads = 8 wavefronts = 2 teams of 4.  Wavefront q of a
// team owns queries 32 q .. 32 q + 31 of the block; team t takes the tiles
// t, t + 2, ... of the segment, so each SIMD runs two wavefronts of different
// teams whose MFMA and exp work interleave.  At the end of a segment the two
// teams' states are merged through LDS.
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
// K/V tiles are staged global -> VGPR -> LDS two tiles ahead of use through
// bounds-checked buffer loads (out-of-range chunks read as zero with no
// branch, so every pipeline step issues the same loads and waits only for
// the older register set).
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "attention.h"

namespace nkl {

namespace {

constexpr int QB = 128;        // queries per block (4 wavefronts x 32)
constexpr int BN = 32;         // keys per tile
constexpr int WPT = 4;         // wavefronts per team
constexpr int NT = 2;          // teams
constexpr int TT = 64 * WPT;   // threads per team
// Buffer-resource word 3 for raw (untyped) dword loads on gfx9-family GPUs.
constexpr int kBufferFlags = 0x00020000;
// The running max is only raised (and O, l rescaled) when a score exceeds it
// by more than 2^8 in the exp2 domain: until then p = exp2(s c - m) stays
// below 256, which fp32 sums and bf16 probabilities represent with the same
// relative precision, and the final O / l is unchanged.
constexpr float kRescaleSlack = 8.0f;
// Smallest unit range a workgroup is given in the balanced mode.
constexpr long kMinUnits = 16;

template <int D>
struct Layout {
  static constexpr int LDK = D + 8;    // K row stride: rows 4 banks apart (16-lane b128 reads)
  static constexpr int LDV = D + 32;   // V row stride: rows 16 banks apart (32-lane b64 transposed reads)
  static constexpr int K_ELEMS = BN * LDK;
  static constexpr int STAGE = K_ELEMS + BN * LDV;
  static constexpr int TEAM = 2 * STAGE;
  static constexpr int TOTAL = NT * TEAM;
  static constexpr int NDB = D / 32;                  // 32-row d blocks of O^T
  static constexpr int SLOT = 64 * (16 * NDB + 2);    // floats per wavefront in the team merge
  static constexpr int PART = WPT * SLOT;             // floats of one partial query-block state
  static_assert((NT - 1) * WPT * SLOT * 4 <= TOTAL * 2, "team merge does not fit in the staging LDS");
};

struct Work {
  int nqb;          // query blocks per head
  int last_nt;      // key tiles of the last (possibly partial) query block
  long units_head;  // units per head
  long units;       // total units
  int grid;         // workgroups
  int streamk;      // 1: balanced unit ranges; 0: one workgroup per query block
  float* part;      // partial states [grid][2][PART]
  int* count;       // arrival counters [H][nqb], zero between calls
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

// Units before query block b of a head: blocks b' < b are full (4 (b'+1) tiles).
__device__ __forceinline__ long units_before(int b) { return 2L * b * (b + 1); }

__device__ __forceinline__ long range_start(long v, const Work& w) { return v * w.units / w.grid; }

// The workgroup (in range order) whose range holds unit u.
__device__ __forceinline__ int range_of(long u, const Work& w) {
  return (int)(((u + 1) * w.grid - 1) / w.units);
}

}  // namespace

template <int D>
__global__ __launch_bounds__(512) void flash_bf16_kernel(AttnArgs p, Work w) {
  using L = Layout<D>;
  using MF = Mfma32<bf16>;
  constexpr int CPR = D / 8;                    // 16-byte chunks per K/V row
  constexpr int NCHUNK = BN * CPR;              // chunks per K (or V) tile
  constexpr int CH = (NCHUNK + TT - 1) / TT;    // chunks per team thread, per tensor
  constexpr int NQF = D / 16;                   // Q^T fragments (K = 16 per MFMA)
  constexpr int NDB = L::NDB;
  __shared__ bf16 smem[L::TOTAL];
  __shared__ int arrival;

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

  // This workgroup's unit range.
  long u0, u1;
  int vidx = blockIdx.x;
  if (w.streamk) {
    if (w.grid % 8 == 0) vidx = (blockIdx.x % 8) * (w.grid / 8) + blockIdx.x / 8;  // XCD-contiguous ranges
    u0 = range_start(vidx, w);
    u1 = range_start(vidx + 1, w);
  } else {
    const int hh = blockIdx.x % p.H;
    const int b = w.nqb - 1 - blockIdx.x / p.H;  // heaviest first
    u0 = hh * w.units_head + units_before(b);
    u1 = u0 + (b == w.nqb - 1 ? w.last_nt : 4 * (b + 1));
  }

  // A segment: head hh, query block b, tiles [t0, t1) of the block's nt tiles.
  struct Seg {
    int hh, b, t0, t1, nt;
    long bstart;
  };
  auto decode = [&](long u) __attribute__((always_inline)) {
    Seg sg;
    sg.hh = (int)(u / w.units_head);
    const long r = u - (long)sg.hh * w.units_head;
    int b = (int)((sqrtf(1.0f + 2.0f * (float)r) - 1.0f) * 0.5f);
    b = min(b, w.nqb - 1);
    while (b + 1 <= w.nqb - 1 && units_before(b + 1) <= r) ++b;
    while (b > 0 && units_before(b) > r) --b;
    sg.b = b;
    sg.bstart = (long)sg.hh * w.units_head + units_before(b);
    sg.nt = b == w.nqb - 1 ? w.last_nt : 4 * (b + 1);
    sg.t0 = (int)(u - sg.bstart);
    sg.t1 = (int)(min(u1, sg.bstart + sg.nt) - sg.bstart);
    return sg;
  };
  auto load_q = [&](const Seg& sg, bf16x8 (&q)[NQF]) __attribute__((always_inline)) {
    const bf16* Q = static_cast<const bf16*>(p.q) + (long)sg.hh * p.q_sh;
    const int qrow = QB * sg.b + 32 * wq + l32;
#pragma unroll
    for (int f = 0; f < NQF; ++f) {
      const int dd = 16 * f + 8 * h32;
      q[f] = __builtin_bit_cast(bf16x8, ld16_or_zero(Q, (long)qrow * p.q_ss + dd, qrow < S && dd < dlim));
    }
  };
  // Loads of one tensor (K or V) for step `it` of team `team` within segment sg.
  auto gload = [&](const Seg& sg, int it, const void* base, long ss, const int (&goff)[CH], uint4 (&rr)[CH])
      __attribute__((always_inline)) {
    const int tj = sg.t0 + team + NT * it;
    const int k0 = tj * BN;
    const int nkeys = tj < sg.t1 ? min(BN, S - k0) : 0;
    const int bytes = nkeys > 0 ? 2 * ((nkeys - 1) * (int)ss + dlim) : 0;
    const __amdgpu_buffer_rsrc_t src = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(static_cast<const bf16*>(base) + (long)sg.hh * (base == p.k ? p.k_sh : p.v_sh) + (long)k0 * ss),
        (short)0, bytes, kBufferFlags);
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

  Seg cur = decode(u0);
  bf16x8 qf[NQF];
  uint4 ka[CH], va[CH], kb2[CH], vb2[CH];
  load_q(cur, qf);
  gload(cur, 0, p.k, p.k_ss, goff_k, ka);
  gload(cur, 0, p.v, p.v_ss, goff_v, va);
  gload(cur, 1, p.k, p.k_ss, goff_k, kb2);
  gload(cur, 1, p.v, p.v_ss, goff_v, vb2);
  lstore(0, ka, va);
  __syncthreads();

  for (;;) {
    const int hh = cur.hh, b = cur.b, t0 = cur.t0, t1 = cur.t1, nt_b = cur.nt;
    const long bstart = cur.bstart;
    const int qw = QB * b + 32 * wq;  // this wavefront's first query
    const int myq = qw + l32;
    const int nit = (t1 - t0 + NT - 1) / NT;

    float m_run = -INFINITY, l_run = 0.f;
    floatx16 oacc[NDB];
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int e = 0; e < 16; ++e) oacc[db][e] = 0.f;

    // One pipeline step: tile `it` computes from LDS stage `it & 1`; the next
    // step's K/V (register set rk/rv, loaded one step ago) are written to the
    // other stage; step it + 2 is loaded into (lk, lv), its V half only after
    // the QK^T MFMAs are issued so that the two halves' loads are spread out.
    auto step = [&](int it, uint4 (&lk)[CH], uint4 (&lv)[CH], const uint4 (&rk)[CH], const uint4 (&rv)[CH])
        __attribute__((always_inline)) {
      const int tj = t0 + team + NT * it;
      const int k0 = tj * BN;
      const bool active = tj < t1 && k0 <= qw + 31;  // inside the segment and not above the diagonal
      const bf16* sb = team_base + (it & 1) * L::STAGE;
      gload(cur, it + 2, p.k, p.k_ss, goff_k, lk);
      floatx16 sacc;
#pragma unroll
      for (int e = 0; e < 16; ++e) sacc[e] = 0.f;
      if (active) {
#pragma unroll
        for (int f = 0; f < NQF; ++f) sacc = MF::mma(load_frag(sb + kfrag_off + 16 * f), qf[f], sacc);
      }
      gload(cur, it + 2, p.v, p.v_ss, goff_v, lv);
      if (active) {
        __builtin_amdgcn_sched_barrier(0);
        if (k0 + BN - 1 > qw) {  // diagonal tile: mask keys after the query
#pragma unroll
          for (int i = 0; i < 16; ++i)
            if (k0 + 8 * (i >> 2) + 4 * h32 + (i & 3) > myq) sacc[i] = -INFINITY;
        }
        float mloc = sacc[0];
#pragma unroll
        for (int i = 1; i < 16; ++i) mloc = fmaxf(mloc, sacc[i]);
        mloc = fmaxf(mloc, __shfl_xor(mloc, 32, kWave)) * c;
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
        for (int i = 0; i < 16; ++i) {
          sacc[i] = fast_exp2(fmaf(sacc[i], c, -m_run));
          rs += sacc[i];
        }
        l_run += rs;
        bf16x8 pf[2];
#pragma unroll
        for (int uu = 0; uu < 2; ++uu)
#pragma unroll
          for (int j = 0; j < 8; ++j) pf[uu][j] = (bf16)sacc[8 * uu + j];
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int db = 0; db < NDB; ++db) {
#pragma unroll
          for (int uu = 0; uu < 2; ++uu) {
            const bf16* vaddr = sb + vfrag_off + 16 * uu * L::LDV + 32 * db;
            const bf16x8 a = read_vt_frag(vaddr, vaddr + 8 * L::LDV);
            oacc[db] = MF::mma(a, pf[uu], oacc[db]);
          }
        }
      }
      lstore((it + 1) & 1, rk, rv);
      __syncthreads();
    };

    for (int it = 0; it < nit; it += 2) {
      step(it, ka, va, kb2, vb2);
      if (it + 1 >= nit) break;
      step(it + 1, kb2, vb2, ka, va);
    }

    // ---- start fetching the next segment's Q and first two K/V tiles so their
    // latency overlaps this segment's merge and hand-off
    const long next_u = bstart + t1;
    const bool more = next_u < u1;
    Seg nxt = cur;
    if (more) {
      nxt = decode(next_u);
      load_q(nxt, qf);  // this segment's Q fragments are no longer needed
      gload(nxt, 0, p.k, p.k_ss, goff_k, ka);
      gload(nxt, 0, p.v, p.v_ss, goff_v, va);
      gload(nxt, 1, p.k, p.k_ss, goff_k, kb2);
      gload(nxt, 1, p.v, p.v_ss, goff_v, vb2);
    }

    // ---- merge the two teams (log2-domain states) into team 0
    float l_tot = l_run + __shfl_xor(l_run, 32, kWave);
    float* red = reinterpret_cast<float*>(smem);
    if (team > 0) {
      float* sl = red + ((team - 1) * WPT + wq) * L::SLOT;
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int e = 0; e < 16; ++e) sl[(db * 16 + e) * 64 + lane] = oacc[db][e];
      sl[16 * NDB * 64 + lane] = m_run;
      sl[(16 * NDB + 1) * 64 + lane] = l_tot;
    }
    __syncthreads();

    // Folds the state (m2, l2, O2 read via `get`) into (m_run, l_tot, oacc).
    auto fold = [&](float m2, float l2, auto get) __attribute__((always_inline)) {
      // An empty state has m = -inf: its weight is 0 (and two empty states stay empty).
      const float M = fmaxf(m_run, m2);
      const float a1 = m_run == -INFINITY ? 0.f : fast_exp2(m_run - M);
      const float a2 = m2 == -INFINITY ? 0.f : fast_exp2(m2 - M);
      l_tot = l_tot * a1 + l2 * a2;
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int e = 0; e < 16; ++e) oacc[db][e] = fmaf(get(db * 16 + e), a2, oacc[db][e] * a1);
      m_run = M;
    };
    auto store_out = [&]() __attribute__((always_inline)) {
      const float linv = 1.0f / l_tot;
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
              for (int e = 0; e < 4; ++e) ov[e] = oacc[db][4 * bq + e] * linv;
              store_vec<4>(orow + dd, ov);
            }
          }
      }
    };

    if (team == 0) {
#pragma unroll 1
      for (int t = 1; t < NT; ++t) {
        const float* sl = red + ((t - 1) * WPT + wq) * L::SLOT;
        fold(sl[16 * NDB * 64 + lane], sl[(16 * NDB + 1) * 64 + lane],
             [&](int j) __attribute__((always_inline)) { return sl[j * 64 + lane]; });
      }
    }

    // ---- finish the query block, or hand a partial state to the last arriver
    int nparts = 1, vf = vidx;
    if (w.streamk) {
      vf = range_of(bstart, w);
      nparts = range_of(bstart + nt_b - 1, w) - vf + 1;
    }
    if (nparts == 1) {
      if (team == 0) store_out();
    } else {
      const int slot = range_start(vidx, w) >= bstart ? 0 : 1;
      float* mine = w.part + ((long)vidx * 2 + slot) * L::PART + wq * L::SLOT;
      if (team == 0) {
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
          for (int e = 0; e < 16; ++e) mine[(db * 16 + e) * 64 + lane] = oacc[db][e];
        mine[16 * NDB * 64 + lane] = m_run;
        mine[(16 * NDB + 1) * 64 + lane] = l_tot;
      }
      // Release: every wavefront's stores have completed (waitcnt) before the
      // barrier; one device-scope fence then publishes them with the arrival.
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
      if (tid == 0) {
        __threadfence();
        arrival = atomicAdd(&w.count[hh * w.nqb + b], 1);
      }
      __syncthreads();
      if (arrival == nparts - 1) {  // last to arrive: merge the others and write O
        if (tid == 0) __threadfence();  // acquire: the other parts' states are visible
        __syncthreads();
        if (team == 0) {
#pragma unroll 1
          for (int v2 = vf; v2 < vf + nparts; ++v2) {
            if (v2 == vidx) continue;
            const int slot2 = range_start(v2, w) >= bstart ? 0 : 1;
            const float* o2 = w.part + ((long)v2 * 2 + slot2) * L::PART + wq * L::SLOT;
            // The part's weight first, then its output in 16-value batches whose
            // loads are each issued together before being folded in.
            const float m2 = o2[16 * NDB * 64 + lane], l2 = o2[(16 * NDB + 1) * 64 + lane];
            const float M = fmaxf(m_run, m2);
            const float a1 = m_run == -INFINITY ? 0.f : fast_exp2(m_run - M);
            const float a2 = m2 == -INFINITY ? 0.f : fast_exp2(m2 - M);
            l_tot = l_tot * a1 + l2 * a2;
            m_run = M;
            constexpr int HALF = 16;
#pragma unroll
            for (int h0 = 0; h0 < 16 * NDB; h0 += HALF) {
              float buf[HALF];
#pragma unroll
              for (int j = 0; j < HALF; ++j) buf[j] = h0 + j < 16 * NDB ? o2[(h0 + j) * 64 + lane] : 0.f;
#pragma unroll
              for (int j = 0; j < HALF; ++j)
                if (h0 + j < 16 * NDB) oacc[(h0 + j) / 16][(h0 + j) % 16] = fmaf(buf[j], a2, oacc[(h0 + j) / 16][(h0 + j) % 16] * a1);
              __builtin_amdgcn_sched_barrier(0);
            }
          }
          store_out();
        }
        if (tid == 0) w.count[hh * w.nqb + b] = 0;
      }
    }
    __syncthreads();  // the LDS is restaged by the next segment
    if (!more) break;
    cur = nxt;
    lstore(0, ka, va);
    __syncthreads();
  }
}

// ------------------------------------------------------------------ host --

static int cu_count() {
  int dev = 0, n = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) return 256;
  return n;
}

// Schedule choice by a cost model in units of one unit's steady-state time
// (about 0.66 us on MI355X), fitted to measured launches of both schedules:
//   one workgroup per block: 10.6 + max(heaviest block, units / CUs)
//   balanced:                45.5 + 1.44 * units per workgroup
// The balanced schedule pays for its partial states, hand-offs and shorter
// pipelines, so it wins only where whole blocks leave CUs idle or unevenly
// loaded (few heads, or long blocks next to short ones).
constexpr float kPerBlockFixed = 10.6f, kBalancedFixed = 45.5f, kBalancedPerUnit = 1.44f;

static Work plan(int H, int S) {
  Work w{};
  w.nqb = (S + QB - 1) / QB;
  w.last_nt = (S - 1) / BN + 1;
  w.units_head = 2L * (w.nqb - 1) * w.nqb + w.last_nt;
  w.units = (long)H * w.units_head;
  const int cus = cu_count();
  // One workgroup per CU, but no range shorter than kMinUnits: a short range
  // spends most of its time filling the pipeline, and splits a query block
  // into many parts for its last workgroup to merge.
  const long by_size = (w.units + kMinUnits - 1) / kMinUnits;
  w.grid = (int)(by_size < cus ? by_size : cus);
  const float per_cu = (float)w.units / (float)cus;
  const float per_block = kPerBlockFixed + fmaxf((float)w.last_nt, per_cu);
  const float balanced = kBalancedFixed + kBalancedPerUnit * (float)w.units / (float)w.grid;
  w.streamk = balanced < per_block;
  // NKL_FLASH_SCHEDULE=balanced|block overrides the choice (tests, tuning).
  if (const char* force = getenv("NKL_FLASH_SCHEDULE")) {
    if (!strcmp(force, "balanced")) w.streamk = 1;
    if (!strcmp(force, "block")) w.streamk = 0;
  }
  return w;
}

template <int D>
static size_t part_floats() { return Layout<D>::PART; }

static size_t part_floats_for(int d) {
  return d <= 32 ? part_floats<32>() : d <= 64 ? part_floats<64>() : part_floats<128>();
}

size_t flash_bf16_workspace_bytes(int H, int S, int d) {
  if (H <= 0 || S <= 0) return 0;
  const Work w = plan(H, S);
  return w.streamk ? (size_t)w.grid * 2 * part_floats_for(d) * 4 : 0;
}

size_t flash_bf16_counter_bytes(int H, int S) {
  if (H <= 0 || S <= 0) return 0;
  const Work w = plan(H, S);
  return w.streamk ? (size_t)H * w.nqb * 4 : 0;
}

template <int D>
static void launch(const AttnArgs& a, Work w, hipStream_t st) {
  const unsigned grid = w.streamk ? (unsigned)w.grid : (unsigned)(w.nqb * a.H);
  flash_bf16_kernel<D><<<dim3(grid), dim3(512), 0, st>>>(a, w);
}

int flash_bf16_launch(const AttnArgs& a, void* workspace, size_t workspace_bytes, int* counters,
                      size_t counter_bytes, hipStream_t st) {
  Work w = plan(a.H, a.S);
  if (!workspace) {
    w.streamk = 0;
  } else if (w.streamk) {
    const size_t need = flash_bf16_workspace_bytes(a.H, a.S, a.d);
    const size_t need_c = flash_bf16_counter_bytes(a.H, a.S);
    if (workspace_bytes < need || !counters || counter_bytes < need_c)
      return set_error(NKL_EWORKSPACE,
                       "nkl_flash_attn_causal_ws: workspace of %zu bytes and counters of %zu bytes needed, "
                       "%zu and %zu given", need, need_c, workspace_bytes, counter_bytes);
    w.part = static_cast<float*>(workspace);
    w.count = counters;
  }
  if (a.d <= 32)
    launch<32>(a, w, st);
  else if (a.d <= 64)
    launch<64>(a, w, st);
  else
    launch<128>(a, w, st);
  return check_launch("nkl_flash_attn_causal");
}

}  // namespace nkl
