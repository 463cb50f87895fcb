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
};

// a / b for 0 <= a, 0 < b: a 32-bit division when both fit (every realistic
// shape), which is a few instructions instead of the ~100 of a 64-bit one.
__device__ __forceinline__ long udiv(long a, long b) {
  if (((unsigned long)a | (unsigned long)b) >> 32 == 0) return (long)((unsigned)a / (unsigned)b);
  return a / b;
}

__device__ __forceinline__ int block_tiles(int b, const Work& w) {
  return b == w.nqb - 1 ? w.last_nt : w.tpb * (b + 1);
}
// Block order: units of a head before block b.
__device__ __forceinline__ long plain_before(int b, const Work& w) { return (long)w.tpb * b * (b + 1) / 2; }
// Pair order: units of a head before pair k (blocks k and n-1-k).  Every pair
// but the first holds tpb (n + 1) units; the first lacks the last block's
// missing tiles (tpb n - last_nt).
__device__ __forceinline__ long pair_before(int k, const Work& w) {
  const long full = (long)w.tpb * (w.nqb + 1);
  const long delta = (long)w.tpb * w.nqb - w.last_nt;
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
__device__ __forceinline__ long head_cost(const Work& w) { return w.units_head + (long)w.nqb * w.cpb; }

// Units (in pair order) whose cost position is below c.
__device__ __forceinline__ long units_below_cost(long c, const Work& w) {
  const long hc = head_cost(w);
  const long hh = udiv(c, hc);
  const long r = c - hh * hc;
  const long F = (long)w.tpb * (w.nqb + 1) + 2L * w.cpb;
  const long delta = (long)w.tpb * w.nqb - w.last_nt;
  const int k = (int)min(udiv(r + delta, F), (long)((w.nqb - 1) / 2));
  const long o = r - (k == 0 ? 0 : k * F - delta);
  const long na = block_tiles(k, w);
  const long in_pair = o < w.cpb + na ? max(0L, o - w.cpb) : na + max(0L, o - 2L * w.cpb - na);
  return hh * w.units_head + pair_before(k, w) + in_pair;
}

// Cost position of unit u.
__device__ __forceinline__ long cost_of_unit(long u, const Work& w) {
  const long hh = udiv(u, w.units_head);
  const long r = u - hh * w.units_head;
  const long full = (long)w.tpb * (w.nqb + 1);
  const long delta = (long)w.tpb * w.nqb - w.last_nt;
  const int k = (int)min(udiv(r + delta, full), (long)((w.nqb - 1) / 2));
  const long starts = r - pair_before(k, w) < block_tiles(k, w) ? 2 * k + 1 : 2 * k + 2;
  return hh * head_cost(w) + r + starts * w.cpb;
}

// First unit of balanced range v (v = grid: the end of the last range).
__device__ __forceinline__ long range_start(long v, const Work& w) { return units_below_cost(udiv(v * w.cost, w.grid), w); }

// The balanced range that holds unit u: the one whose cost interval
// [v cost / grid, (v + 1) cost / grid) holds u's cost position.
__device__ __forceinline__ int range_of(long u, const Work& w) {
  return (int)udiv((cost_of_unit(u, w) + 1) * w.grid - 1, w.cost);
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
__device__ __forceinline__ Seg decode_seg(long u, long u0, const Work& w) {
  Seg sg;
  sg.hh = (int)udiv(u, w.units_head);
  const long r = u - (long)sg.hh * w.units_head;
  long before;
  if (w.paired) {
    const long full = (long)w.tpb * (w.nqb + 1);
    const long delta = (long)w.tpb * w.nqb - w.last_nt;
    const int k = min((int)udiv(r + delta, full), (w.nqb - 1) / 2);
    before = pair_before(k, w);
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
    while (b + 1 <= w.nqb - 1 && plain_before(b + 1, w) <= r) ++b;
    while (b > 0 && plain_before(b, w) > r) --b;
    sg.b = b;
    before = plain_before(b, w);
  }
  sg.bstart = (long)sg.hh * w.units_head + before;
  sg.nt = block_tiles(sg.b, w);
  sg.t0 = (int)(max(u0, sg.bstart) - sg.bstart);
  sg.t1 = (int)(u - sg.bstart + 1);
  return sg;
}

// The workgroup holding a split block's last range merges it.  It walks that
// segment last, long after the block's other parts -- walked first by their
// ranges -- have stored their states and arrived, so rather than store its own
// state and arrive it polls the block's counter until the other nparts - 1
// have arrived (their arrivals never reach nparts - 1 without it) and sets
// `arrival` to nparts - 1.  The poll is bounded (4096 polls, each followed by
// ~512 cycles of sleep: ~1 ms); past that `arrival` is -1 and the workgroup
// stores its state and arrives like the others, the last of which merges.
__device__ __forceinline__ void await_parts(int* count, int nparts, int& arrival) {
  if (threadIdx.x == 0) {
    int n = 0;
    for (int it = 0; it < 4096; ++it) {
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
