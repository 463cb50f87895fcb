// Shared declarations of the causal attention kernels.
#pragma once

#include "common.h"

namespace nkl {

struct AttnArgs {
  const void* q;
  const void* k;
  const void* v;
  void* o;
  int H, S, d;
  long q_sh, q_ss, k_sh, k_ss, v_sh, v_ss, o_sh, o_ss;
  float c;    // softmax scale * log2(e): p = exp2(s * c - m)
  int group;  // query heads per K/V head (grouped-query attention; 1 for multi-head)
  int f16;    // 16-bit kernels: 1 for fp16 q, k, v, o (P rounded to fp16), 0 for bf16
};

// bf16 (and fp16: AttnArgs::f16) flash attention (flash_bf16.hip).  With a workspace of
// flash_bf16_workspace_bytes() bytes for partial states and a zeroed counter
// array of flash_bf16_counter_bytes() bytes (left zero by every call), the
// work is balanced over one workgroup per CU (stream-K); without them, each
// workgroup takes one whole query block.
size_t flash_bf16_workspace_bytes(int H, int S, int d, bool f16 = false);
size_t flash_bf16_counter_bytes(int H, int S);
int flash_bf16_launch(const AttnArgs& a, void* workspace, size_t workspace_bytes, int* counters,
                      size_t counter_bytes, hipStream_t st);

namespace fsched {
struct Work;
}
// The 64-key-tile bf16 kernel (flash_fwd.hip) for 64 < d <= 128: launch over
// a planned Work (128-query blocks, 64-key tiles), and the bytes of one
// workgroup's partial state of a block (the workspace holds two per range).
// pingpong: the two key-half wavefronts of a SIMD half an iteration apart
// (matrix-core work of one beside vector work of the other).
void launch_flash_fwd(const AttnArgs& a, const fsched::Work& w, bool pingpong, hipStream_t st);
size_t flash_fwd_part_bytes();
// The key-split kernel (flash_ks.hip) for 64 < d <= 128: launch over a
// planned Work (64-query blocks, 32-key tiles, four wavefronts that each take
// every fourth tile of a segment), and the bytes of one part's state of a
// block (the workspace holds two per range).
void launch_flash_ks(const AttnArgs& a, const fsched::Work& w, hipStream_t st);
size_t flash_ks_part_bytes();
// The one-pass kernel for short sequences (flash_tiny.hip): 64 < d <= 128,
// S <= kTinyMaxS, scale > 0; one workgroup per (head, 128-query block) with
// every key row of the block staged in LDS at once.  No scratch.
constexpr int kTinyMaxS = 256;
bool flash_tiny_fits(const AttnArgs& a);
void launch_flash_tiny(const AttnArgs& a, hipStream_t st);
// Process-wide kernel / schedule / block / start-cost overrides (-1: automatic).
int flash_bf16_configure(int kern, int sched, int qb, int cpb);
// Process-wide poll budget of the workgroup that merges a split block (-1: the
// planner's choice).
int flash_bf16_configure_polls(int polls);
// Host-side check of the launch plan's work split (flash_bf16.hip).
int flash_bf16_plan_check(int H, int S, int d, bool f16, long* info);

}  // namespace nkl
