// Work decomposition shared by the bf16 causal flash-attention kernels
// (flash_bf16.hip, flash_fwd.hip): units, the three schedules and the
// balanced (stream-K) range arithmetic.
//
// Queries are grouped in blocks of QB; keys in tiles of BN.  A "unit" is one
// (head, query block, key tile) triple with the tile at or below the diagonal
// (tiles above it are never visited: the causal tile skip of
// nkilab/kernels/attention.py:300-316).  Block b of a head holds tpb (b + 1)
// units (tpb = QB / BN), the last block those of its ragged end.  The units of
// a head are numbered block by block, either in block order or in pair order
// -- blocks 0, n-1, 1, n-2, ... so that consecutive pairs (b, n-1-b) all hold
// the same number of units.  Three schedules:
//   block     one workgroup per query block, heaviest first;
//   pairs     one workgroup per pair of blocks (equal work everywhere);
//   balanced  the units cut into contiguous ranges of equal cost, one per
//             workgroup (stream-K).  A workgroup walks its range as segments
//             (one per block it touches); a block split across workgroups is
//             finished by whichever arrives last, which folds in the others'
//             partial (max, sum, output) states from a workspace.
#pragma once

#include "attention.h"

namespace nkl {
namespace fsched {

// Buffer-resource word 3 for raw (untyped) dword loads on gfx9-family GPUs.
constexpr int kBufferFlags = 0x00020000;
// Cache policy of the partial-state stores and loads: SC1, coherent at device
// scope (the policy of an agent-scope atomic load or store).  Partial states
// travel between workgroups that may run on different XCDs; with every store
// and load of them device-coherent, the hand-off needs no L2 writeback or
// invalidate -- only each store's completion (vmcnt) before the arrival
// atomic.
constexpr int kDeviceCoherent = 16;
// The running max is only raised (and O, l rescaled) when a score exceeds it
// by more than 2^8 in the exp2 domain: until then p = exp2(s c - m) stays
// below 256, which fp32 sums and bf16 probabilities represent with the same
// relative precision, and the final O / l is unchanged.
constexpr float kRescaleSlack = 8.0f;

enum Sched { kBlock = 0, kBalanced = 1, kPairs = 2 };

// Division of n (0 <= n < 2^32) by a per-launch constant d (1 <= d < 2^32) as
// a multiply-high, an add and two shifts (Granlund and Montgomery, "Division
// by invariant integers using multiplication", PLDI 1994, fig. 4.1): the
// workgroups' schedule arithmetic divides by a handful of launch constants,
// and a 32-bit division otherwise costs ~35 instructions with a VALU round
// trip, a 64-bit one ~100.
struct Div32 {
  unsigned d, m;
  int sh1, sh2;
};
inline Div32 make_div32(unsigned d) {
  int l = 0;  // ceil(log2 d)
  while (l < 32 && (1ull << l) < d) ++l;
  Div32 f;
  f.d = d;
  f.m = (unsigned)(((1ull << 32) * ((1ull << l) - d)) / d + 1);
  f.sh1 = l < 1 ? l : 1;
  f.sh2 = l > 1 ? l - 1 : 0;
  return f;
}
__host__ __device__ inline unsigned div32(const Div32& f, unsigned n) {
  const unsigned t = (unsigned)(((unsigned long long)f.m * n) >> 32);
  return (t + ((n - t) >> f.sh1)) >> f.sh2;
}

struct Work {
  int nqb;          // query blocks per head
  int tpb;          // key tiles added per block (QB / BN): block b has tpb (b + 1)
  int last_nt;      // key tiles of the last (possibly partial) block
  int paired;       // unit order: 1 pair order, 0 block order
  int sched;        // Sched
  int grid;         // workgroups
  long units_head;  // units per head
  long units;       // total units
  int cpb;          // balanced: cost charged at the start of every block, in units
  long cost;        // balanced: total cost, units + cpb per block
  float* part;      // balanced: partial states
  int part_bytes;   // balanced: bytes of part
  int* count;       // balanced: arrival counters [H][nqb], zero between calls
  int polls;        // balanced: poll budget of the workgroup that merges a split block (await_parts)
  // Magic divisors of the launch constants below, valid when fast is set
  // (every dividend of the schedule arithmetic fits in 32 bits): units_head,
  // the pair span tpb (nqb + 1), its cost tpb (nqb + 1) + 2 cpb, the head
  // cost, grid and cost.
  int fast;
  Div32 dv_units_head, dv_full, dv_fcost, dv_head_cost, dv_grid, dv_cost;
  Div32 dv_group;  // query heads per K/V head (set at launch)
};

// a / b for 0 <= a, 0 < b: a 32-bit division when both fit (every realistic
// shape), which is a few instructions instead of the ~100 of a 64-bit one.
__host__ __device__ __forceinline__ long udiv(long a, long b) {
  if (((unsigned long)a | (unsigned long)b) >> 32 == 0) return (long)((unsigned)a / (unsigned)b);
  return a / b;
}

// The schedule arithmetic below is written once over an integer type I: int
// when the launch's values fit (Work::fast: every dividend below 2^32, every
// quantity below 2^31), with the magic divisors, so that a workgroup's
// set-up runs a short chain of 32-bit scalar instructions; long otherwise.
// q(a, f, b) is a / b for the launch constant b whose magic divisor is f.
template <typename I>
__host__ __device__ __forceinline__ I q(I a, const Div32& f, long b);
template <>
__host__ __device__ __forceinline__ int q<int>(int a, const Div32& f, long) { return (int)div32(f, (unsigned)a); }
template <>
__host__ __device__ __forceinline__ long q<long>(long a, const Div32&, long b) { return udiv(a, b); }

__host__ __device__ __forceinline__ int block_tiles(int b, const Work& w) {
  return b == w.nqb - 1 ? w.last_nt : w.tpb * (b + 1);
}
// Block order: units of a head before block b.
template <typename I = long>
__host__ __device__ __forceinline__ I plain_before(int b, const Work& w) { return (I)w.tpb * b * (b + 1) / 2; }
// Pair order: units of a head before pair k (blocks k and n-1-k).  Every pair
// but the first holds tpb (n + 1) units; the first lacks the last block's
// missing tiles (tpb n - last_nt).
template <typename I = long>
__host__ __device__ __forceinline__ I pair_before(int k, const Work& w) {
  const I full = (I)w.tpb * (w.nqb + 1);
  const I delta = (I)w.tpb * w.nqb - w.last_nt;
  return k == 0 ? 0 : k * full - delta;
}

// Balanced ranges split a cost line evenly: the units in pair order, with
// cpb units of cost in front of every block (a segment's fixed work: the
// hand-over inside the workgroup, the output or partial-state stores, the
// next segment's first loads), so a workgroup whose range starts more blocks
// gets fewer units.  Per head, pair k (blocks k and n-1-k) spans cost
// [k F - delta, (k + 1) F - delta) with F = tpb (n + 1) + 2 cpb (pair 0 from 0):
// cpb, block k's units, cpb, block n-1-k's units.  A range of more than cpb
// cost holds at least one unit, which the planner guarantees.
template <typename I = long>
__host__ __device__ __forceinline__ I head_cost(const Work& w) { return (I)w.units_head + (I)w.nqb * w.cpb; }

// Units (in pair order) whose cost position is below c.
template <typename I>
__host__ __device__ __forceinline__ I units_below_cost_t(I c, const Work& w) {
  const I hc = head_cost<I>(w);
  const I hh = q<I>(c, w.dv_head_cost, hc);
  const I r = c - hh * hc;
  const I F = (I)w.tpb * (w.nqb + 1) + 2 * (I)w.cpb;
  const I delta = (I)w.tpb * w.nqb - w.last_nt;
  const I kq = q<I>(r + delta, w.dv_fcost, F);
  const int k = (int)(kq < (I)((w.nqb - 1) / 2) ? kq : (I)((w.nqb - 1) / 2));
  const I o = r - (k == 0 ? 0 : k * F - delta);
  const I na = block_tiles(k, w);
  const I in_pair = o < w.cpb + na ? (o > w.cpb ? o - w.cpb : 0) : na + (o > 2 * (I)w.cpb + na ? o - 2 * (I)w.cpb - na : 0);
  return hh * (I)w.units_head + pair_before<I>(k, w) + in_pair;
}

// Cost position of unit u.
template <typename I>
__host__ __device__ __forceinline__ I cost_of_unit_t(I u, const Work& w) {
  const I hh = q<I>(u, w.dv_units_head, w.units_head);
  const I r = u - hh * (I)w.units_head;
  const I full = (I)w.tpb * (w.nqb + 1);
  const I delta = (I)w.tpb * w.nqb - w.last_nt;
  const I kq = q<I>(r + delta, w.dv_full, full);
  const int k = (int)(kq < (I)((w.nqb - 1) / 2) ? kq : (I)((w.nqb - 1) / 2));
  const I starts = r - pair_before<I>(k, w) < block_tiles(k, w) ? 2 * k + 1 : 2 * k + 2;
  return hh * head_cost<I>(w) + r + starts * w.cpb;
}

// First unit of balanced range v (v = grid: the end of the last range).
template <typename I>
__host__ __device__ __forceinline__ I range_start_t(I v, const Work& w) {
  return units_below_cost_t<I>(q<I>(v * (I)w.cost, w.dv_grid, w.grid), w);
}
__host__ __device__ __forceinline__ long range_start(long v, const Work& w) {
  return w.fast ? (long)range_start_t<int>((int)v, w) : range_start_t<long>(v, w);
}

// The balanced range that holds unit u: the one whose cost interval
// [v cost / grid, (v + 1) cost / grid) holds u's cost position.
template <typename I>
__host__ __device__ __forceinline__ int range_of_t(I u, const Work& w) {
  return (int)q<I>((cost_of_unit_t<I>(u, w) + 1) * (I)w.grid - 1, w.dv_cost, w.cost);
}
__host__ __device__ __forceinline__ int range_of(long u, const Work& w) {
  return w.fast ? range_of_t<int>((int)u, w) : range_of_t<long>(u, w);
}

// This workgroup's range index and unit range [u0, u1).  Balanced ranges are
// numbered XCD-contiguously: workgroups are dispatched to the eight XCDs
// round-robin, so workgroup b takes range (b % 8) (grid / 8) + b / 8 and
// neighbouring ranges -- which share split blocks and K/V heads -- run on one
// XCD and share its L2.
__device__ __forceinline__ int wg_range(const Work& w, int H, long& u0, long& u1) {
  int vidx = blockIdx.x;
  if (w.sched == kBalanced) {
    if (w.grid % 8 == 0) vidx = (blockIdx.x % 8) * (w.grid / 8) + blockIdx.x / 8;
    u0 = range_start(vidx, w);
    u1 = range_start(vidx + 1, w);
  } else if (w.sched == kPairs) {
    const int hh = blockIdx.x % H, k = blockIdx.x / H;
    u0 = hh * w.units_head + pair_before(k, w);
    u1 = 2 * k + 2 <= w.nqb ? hh * w.units_head + pair_before(k + 1, w) : (hh + 1) * w.units_head;
  } else {
    const int hh = blockIdx.x % H;
    const int b = w.nqb - 1 - blockIdx.x / H;  // heaviest first
    u0 = hh * w.units_head + plain_before(b, w);
    u1 = u0 + block_tiles(b, w);
  }
  return vidx;
}

// wg_range with 32-bit arithmetic throughout (Work::fast must hold): no
// 64-bit paths, whose division set-up the compiler would otherwise hoist to
// the kernel's start.
__device__ __forceinline__ int wg_range_fast(const Work& w, int H, int& u0, int& u1) {
  int vidx = blockIdx.x;
  if (w.sched == kBalanced) {
    if (w.grid % 8 == 0) vidx = (blockIdx.x % 8) * (w.grid / 8) + blockIdx.x / 8;
    u0 = range_start_t<int>(vidx, w);
    u1 = range_start_t<int>(vidx + 1, w);
  } else if (w.sched == kPairs) {
    const int hh = blockIdx.x % H, k = blockIdx.x / H;
    u0 = hh * (int)w.units_head + pair_before<int>(k, w);
    u1 = 2 * k + 2 <= w.nqb ? hh * (int)w.units_head + pair_before<int>(k + 1, w) : (hh + 1) * (int)w.units_head;
  } else {
    const int hh = blockIdx.x % H;
    const int b = w.nqb - 1 - blockIdx.x / H;  // heaviest first
    u0 = hh * (int)w.units_head + plain_before<int>(b, w);
    u1 = u0 + block_tiles(b, w);
  }
  return vidx;
}

// The schedule arithmetic with the unit type chosen at compile time: F true
// (the plan's Work::fast holds: every value fits in 32 bits) takes the 32-bit
// paths only, so that a kernel instantiated for it carries no 64-bit
// division code (which the compiler would otherwise set up at the kernel's
// start and keep in registers throughout).
template <bool F>
__device__ __forceinline__ int wg_range_x(const Work& w, int H, long& u0, long& u1) {
  if constexpr (F) {
    int a, b;
    const int v = wg_range_fast(w, H, a, b);
    u0 = a;
    u1 = b;
    return v;
  } else {
    return wg_range(w, H, u0, u1);
  }
}
template <bool F>
__device__ __forceinline__ int range_of_x(long u, const Work& w) {
  if constexpr (F)
    return range_of_t<int>((int)u, w);
  else
    return range_of(u, w);
}
template <bool F>
__device__ __forceinline__ long range_start_x(long v, const Work& w) {
  if constexpr (F)
    return range_start_t<int>((int)v, w);
  else
    return range_start(v, w);
}

// A segment: head hh, query block b, tiles [t0, t1) of the block's nt tiles,
// whose first unit is bstart.
struct Seg {
  int hh, b, t0, t1, nt;
  long bstart;
};

// The segment of the range [u0, ..) that ends with unit u.  Ranges are walked
// from their last segment to their first: the first segment in unit order is
// often the tail of a block whose head other workgroups hold, and taking it
// last leaves the merge of that block's partial states to this workgroup,
// the last to arrive, after its other segments rather than before them.
template <typename I>
__host__ __device__ __forceinline__ Seg decode_seg_t(I u, I u0, const Work& w) {
  Seg sg;
  sg.hh = (int)q<I>(u, w.dv_units_head, w.units_head);
  const I r = u - (I)sg.hh * (I)w.units_head;
  I before;
  if (w.paired) {
    const I full = (I)w.tpb * (w.nqb + 1);
    const I delta = (I)w.tpb * w.nqb - w.last_nt;
    const I kq = q<I>(r + delta, w.dv_full, full);
    const int k = (int)(kq < (I)((w.nqb - 1) / 2) ? kq : (I)((w.nqb - 1) / 2));
    before = pair_before<I>(k, w);
    const int na = block_tiles(k, w);
    if (r - before < na) {
      sg.b = k;
    } else {
      sg.b = w.nqb - 1 - k;
      before += na;
    }
  } else {
    int b = (int)((sqrtf(1.0f + 8.0f * (float)r / (float)w.tpb) - 1.0f) * 0.5f);
    b = max(0, min(b, w.nqb - 1));
    while (b + 1 <= w.nqb - 1 && plain_before<I>(b + 1, w) <= r) ++b;
    while (b > 0 && plain_before<I>(b, w) > r) --b;
    sg.b = b;
    before = plain_before<I>(b, w);
  }
  const I bstart = (I)sg.hh * (I)w.units_head + before;
  sg.bstart = bstart;
  sg.nt = block_tiles(sg.b, w);
  sg.t0 = (int)((u0 > bstart ? u0 : bstart) - bstart);
  sg.t1 = (int)(u - bstart + 1);
  return sg;
}
__host__ __device__ __forceinline__ Seg decode_seg(long u, long u0, const Work& w) {
  return w.fast ? decode_seg_t<int>((int)u, (int)u0, w) : decode_seg_t<long>(u, u0, w);
}
template <bool F>
__device__ __forceinline__ Seg decode_seg_x(long u, long u0, const Work& w) {
  if constexpr (F)
    return decode_seg_t<int>((int)u, (int)u0, w);
  else
    return decode_seg_t<long>(u, u0, w);
}

// The workgroup holding a split block's last range merges it.  It walks that
// segment last, long after the block's other parts -- walked first by their
// ranges -- have stored their states and arrived, so rather than store its own
// state and arrive it polls the block's counter until the other nparts - 1
// have arrived (their arrivals never reach nparts - 1 without it) and sets
// `arrival` to nparts - 1.  The poll is bounded (Work::polls polls, each an
// atomic load and ~512 cycles of sleep, ~0.5 us; the planner gives 256, or 0
// when blocks are split into many parts); past that `arrival` is -1 and the
// workgroup stores its state and arrives like the others, the last of which
// merges.  Either way the states are folded in the
// same order, so the result does not depend on which workgroup merges.  (The
// teams kernel's 128-query form has its own protocol, which folds each part
// as it arrives; see flash_bf16.hip.)
__device__ __forceinline__ void await_parts(int* count, int nparts, int polls, int& arrival) {
  if (threadIdx.x == 0) {
    int n = 0;
    for (int it = 0; it < polls; ++it) {
      n = __hip_atomic_load(count, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (n == nparts - 1) break;
      __builtin_amdgcn_s_sleep(8);
    }
    arrival = n == nparts - 1 ? nparts - 1 : -1;
  }
  __syncthreads();
}

// s_waitcnt with vmcnt <= n and the other counters left alone (gfx9 encoding).
template <int n>
__device__ __forceinline__ void wait_vm() {
  static_assert(n >= 0 && n < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Swizzle of 256-byte K/V rows in LDS: logical 16-byte chunk c of row r sits
// at chunk c ^ row_swz(r), row_swz(r) = 4 (r % 4) + 2 ((r / 4) % 2) + (r / 8) % 2.
// The 16 rows of a K-fragment read (b128, one chunk each, also as rows 0-7 x
// chunks 2f, 2f+1) and the 4 aligned rows x 4 aligned chunks of a transposed
// V read (b64) then all fall in distinct bank groups.  It depends on r % 16
// only.
__device__ __forceinline__ int row_swz(int r) { return ((r & 3) << 2) | (((r >> 2) & 1) << 1) | ((r >> 3) & 1); }

}  // namespace fsched
}  // namespace nkl
