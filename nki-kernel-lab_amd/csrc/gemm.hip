// GEMM: C = A . op(B) (+ R) on 32x32 MFMA tiles with fp32 accumulation.
//
// bf16 operands take the LDS-DMA kernel further down (gemm_dma_kernel: the
// hot path, tiles from 64x64 to 256x256).
//
// Register-staged blocked kernel (fp32 operands, and bf16 operands the DMA
// kernel's buffer offsets cannot address): a 256-thread workgroup owns a
// BM x BN tile of C; its four wavefronts are laid out 2 x 2 and each owns a
// (BM/2) x (BN/2) sub-tile of 32x32 MFMA accumulators.  Per K step of BK
// elements (64 bytes of each operand row) the workgroup stages an A tile
// [BM][BK] and a B tile [BN][BK] in LDS, both K-contiguous so that every MFMA
// operand fragment is one 16-byte LDS read.  B given as [K, N] (the
// reference's `rhs`) is transposed while it is written to LDS; B given as
// [N, K] (nn.Linear.weight) is copied as is.  LDS is double-buffered and the
// next K step's global loads are in flight while the current one computes.
//
// Naive kernel (variant "naive", and the fallback for shapes the blocked
// kernel's 16-byte loads cannot address): each wavefront computes one 32x32
// tile of C reading its operands straight from global memory at every K step
// -- no on-chip reuse, like the reference's matmul_naive.
#include <atomic>
#include <cstdlib>
#include <cstring>
#include <type_traits>

#include "common.h"

namespace nkl {

// Epilogues of the LDS-DMA kernel.
enum Epi {
  kEpiElem = 0,    // one element per lane per store (any alignment)
  kEpiStaged = 1,  // tile staged in LDS, 16 bytes per lane per store
  kEpiSwiglu = 2,  // staged; adjacent 32-column tiles are gate and up: C = silu(gate) * up, N / 2 columns
};

struct GemmArgs {
  const void* A;
  const void* B;
  void* C;
  const void* R;
  int M, N, K;
  long lda, ldb, ldc, ldr;
  long sA, sB, sC, sR;
  int epi;  // Epi (the LDS-DMA kernel; the other kernels store elements)
};

template <typename T>
struct GemmBK { static constexpr int value = 64 / sizeof(T); };

// Workgroup tile index -> (tile_m, tile_n).  Consecutive workgroup ids are
// dispatched round-robin over the 8 XCDs; the remap gives each XCD a
// contiguous range of tiles, walked in groups of GROUP_M tile-rows so the
// A and B stripes a group touches stay in that XCD's L2.
__device__ __forceinline__ void tile_coords(int bid, int tiles_m, int tiles_n, int& tm, int& tn) {
  const int total = tiles_m * tiles_n;
  int id = bid;
  if (total % 8 == 0) id = (bid % 8) * (total / 8) + bid / 8;
  constexpr int GROUP_M = 8;
  const int group_size = GROUP_M * tiles_n;
  const int group = id / group_size;
  const int first_m = group * GROUP_M;
  const int gm = min(tiles_m - first_m, GROUP_M);
  const int in_group = id - group * group_size;
  tm = first_m + in_group % gm;
  tn = in_group / gm;
}

template <typename T, typename TO, int BM, int BN, bool BT>
__global__ __launch_bounds__(256) void gemm_blocked_kernel(GemmArgs p) {
  using MF = Mfma32<T>;
  constexpr int E = VecE<T>::value;           // elements per 16-byte chunk
  constexpr int BK = GemmBK<T>::value;        // K elements per stage (64 bytes)
  constexpr int PAD = E;                      // 16 bytes of row padding
  constexpr int LDK = BK + PAD;               // LDS row stride (elements)
  constexpr int CPR = BK / E;                 // 16-byte chunks per LDS row (4)
  constexpr int WM = BM / 2, WN = BN / 2;     // wave sub-tile
  constexpr int TM = WM / 32, TN = WN / 32;   // 32x32 MFMA tiles per wave
  constexpr int A_CH = BM * CPR / 256;        // A chunks per thread
  constexpr int B_CH = BN * CPR / 256;        // B chunks per thread
  static_assert(A_CH >= 1 && B_CH >= 1, "tile too small for 256 threads");

  __shared__ T As[2][BM * LDK];
  __shared__ T Bs[2][BN * LDK];

  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int wm = wid >> 1, wn = wid & 1;
  const int tiles_m = (p.M + BM - 1) / BM, tiles_n = (p.N + BN - 1) / BN;
  int tm, tn;
  tile_coords(blockIdx.x, tiles_m, tiles_n, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const int bz = blockIdx.z;
  const T* A = static_cast<const T*>(p.A) + (long)bz * p.sA;
  const T* B = static_cast<const T*>(p.B) + (long)bz * p.sB;
  TO* C = static_cast<TO*>(p.C) + (long)bz * p.sC;
  const TO* R = p.R ? static_cast<const TO*>(p.R) + (long)bz * p.sR : nullptr;

  uint4 ra[A_CH], rb[B_CH];
  auto gload = [&](int k0) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < A_CH; ++i) {
      const int c = tid + 256 * i, row = c / CPR, kc = (c % CPR) * E;
      const int gm = m0 + row, gk = k0 + kc;
      ra[i] = ld16_or_zero(A, (long)gm * p.lda + gk, gm < p.M && gk < p.K);
    }
    if constexpr (BT) {
#pragma unroll
      for (int i = 0; i < B_CH; ++i) {
        const int c = tid + 256 * i, row = c / CPR, kc = (c % CPR) * E;
        const int gn = n0 + row, gk = k0 + kc;
        rb[i] = ld16_or_zero(B, (long)gn * p.ldb + gk, gn < p.N && gk < p.K);
      }
    } else {
      constexpr int NCH = BN / E;  // 16-byte chunks per B row of the tile
#pragma unroll
      for (int i = 0; i < B_CH; ++i) {
        const int c = tid + 256 * i, kr = c / NCH, nc = (c % NCH) * E;
        const int gk = k0 + kr, gn = n0 + nc;
        rb[i] = ld16_or_zero(B, (long)gk * p.ldb + gn, gk < p.K && gn < p.N);
      }
    }
  };

  auto lstore = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < A_CH; ++i) {
      const int c = tid + 256 * i, row = c / CPR, kc = (c % CPR) * E;
      *reinterpret_cast<uint4*>(&As[buf][row * LDK + kc]) = ra[i];
    }
    if constexpr (BT) {
#pragma unroll
      for (int i = 0; i < B_CH; ++i) {
        const int c = tid + 256 * i, row = c / CPR, kc = (c % CPR) * E;
        *reinterpret_cast<uint4*>(&Bs[buf][row * LDK + kc]) = rb[i];
      }
    } else {
      constexpr int NCH = BN / E;
#pragma unroll
      for (int i = 0; i < B_CH; ++i) {
        const int c = tid + 256 * i, kr = c / NCH, nc = (c % NCH) * E;
        const T* v = reinterpret_cast<const T*>(&rb[i]);
#pragma unroll
        for (int e = 0; e < E; ++e) Bs[buf][(nc + e) * LDK + kr] = v[e];
      }
    }
  };

  floatx16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  const int nk = (p.K + BK - 1) / BK;
  gload(0);
  lstore(0);
  __syncthreads();
  const int lr = lane & 31, lg = lane >> 5;
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < nk) gload((kt + 1) * BK);
#pragma unroll
    for (int ks = 0; ks < BK / MF::MK; ++ks) {
      const int kk = ks * MF::MK + lg * MF::KPER;
      typename MF::frag af[TM], bfr[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) af[i] = load_frag(&As[buf][(wm * WM + i * 32 + lr) * LDK + kk]);
#pragma unroll
      for (int j = 0; j < TN; ++j) bfr[j] = load_frag(&Bs[buf][(wn * WN + j * 32 + lr) * LDK + kk]);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = MF::mma(af[i], bfr[j], acc[i][j]);
    }
    if (kt + 1 < nk) lstore(buf ^ 1);
    __syncthreads();
  }

  // Epilogue: accumulator element e of tile (i, j) is C[row][col] with
  // row = 8 * (e / 4) + 4 * (lane / 32) + e % 4, col = lane % 32.
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int col = n0 + wn * WN + j * 32 + lr;
      if (col >= p.N) continue;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int row = m0 + wm * WM + i * 32 + 8 * (e / 4) + 4 * lg + (e % 4);
        if (row < p.M) {
          float vv = acc[i][j][e];
          if (R) vv += to_f32(R[(long)row * p.ldr + col]);
          C[(long)row * p.ldc + col] = from_f32<TO>(vv);
        }
      }
    }
}

// One wavefront per 32x32 tile of C, four per workgroup; operands are read
// from global memory at every K step with per-element bounds checks.
template <typename T, typename TO, bool BT>
__global__ __launch_bounds__(256) void gemm_naive_kernel(GemmArgs p) {
  using MF = Mfma32<T>;
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int tiles_n = (p.N + 31) / 32;
  const int tile = blockIdx.x * 4 + wid;
  const int tm = tile / tiles_n, tn = tile % tiles_n;
  if (tm * 32 >= p.M) return;
  const int bz = blockIdx.z;
  const T* A = static_cast<const T*>(p.A) + (long)bz * p.sA;
  const T* B = static_cast<const T*>(p.B) + (long)bz * p.sB;
  TO* C = static_cast<TO*>(p.C) + (long)bz * p.sC;
  const TO* R = p.R ? static_cast<const TO*>(p.R) + (long)bz * p.sR : nullptr;
  const int lr = lane & 31, lg = lane >> 5;
  const int arow = tm * 32 + lr, bcol = tn * 32 + lr;
  floatx16 acc;
#pragma unroll
  for (int e = 0; e < 16; ++e) acc[e] = 0.f;
  for (int k0 = 0; k0 < p.K; k0 += MF::MK) {
    T av[MF::KPER], bv[MF::KPER];
#pragma unroll
    for (int j = 0; j < MF::KPER; ++j) {
      const int k = k0 + lg * MF::KPER + j;
      const bool kin = k < p.K;
      av[j] = (kin && arow < p.M) ? A[(long)arow * p.lda + k] : from_f32<T>(0.f);
      if constexpr (BT)
        bv[j] = (kin && bcol < p.N) ? B[(long)bcol * p.ldb + k] : from_f32<T>(0.f);
      else
        bv[j] = (kin && bcol < p.N) ? B[(long)k * p.ldb + bcol] : from_f32<T>(0.f);
    }
    typename MF::frag af, bfr;
    if constexpr (MF::KPER == 1) {
      af = av[0];
      bfr = bv[0];
    } else {
#pragma unroll
      for (int j = 0; j < MF::KPER; ++j) {
        af[j] = av[j];
        bfr[j] = bv[j];
      }
    }
    acc = MF::mma(af, bfr, acc);
  }
  const int col = tn * 32 + lr;
  if (col >= p.N) return;
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    const int row = tm * 32 + 8 * (e / 4) + 4 * lg + (e % 4);
    if (row < p.M) {
      float vv = acc[e];
      if (R) vv += to_f32(R[(long)row * p.ldr + col]);
      C[(long)row * p.ldc + col] = from_f32<TO>(vv);
    }
  }
}

// ------------------------------------------------ bf16 GEMM, LDS-DMA staged --
//
// The bf16 path.  Operand tiles are copied global -> LDS by the buffer unit
// (buffer_load ... lds, lane l's 16 bytes at the instruction's LDS base + 16 l)
// into a ring of NS stages, NS - 1 K-steps ahead of use, so that even a small
// GEMM (1024^3, 256 workgroups of 64x64) keeps enough loads in flight to cover
// the memory latency.  Every staged tile is made of 128-byte rows (64 bf16 of
// K for A and for B given as [N, K]; 64 columns of N for B given as [K, N],
// in sub-tiles of 64 columns) whose 16-byte chunks are swizzled: chunk c of
// row r sits at chunk c ^ g_swz(r).  The swizzle keeps the 16-row b128
// fragment reads (A, B^T) and the 4-row transposed b64 reads (B as [K, N],
// read with ds_read_b64_tr_b16) free of bank conflicts.  One barrier per
// K-step; WGM x WGN wavefronts of 32x32x16 MFMA tiles.
//
// 2 x 2 wavefronts (256 threads, one per SIMD) for tiles up to 128 x 128;
// 2 x 4 (512 threads, two per SIMD) for 256-row tiles.  A 128 x 128 tile
// stages 32 KB per K-step for 2 MFLOP, ~64 B/clk per CU at the MFMA rate --
// all an L2 channel set delivers; a 256 x 256 tile stages half that per flop.
// With two 64 KB stages the next K-step's copies have one K-step (32 MFMAs
// per wavefront, two wavefronts per SIMD) to land.

namespace {

constexpr int G_BK = 64;  // K elements per stage

__device__ __forceinline__ int g_swz(int r) { return (((r >> 1) & 1) << 2) | (((r >> 2) & 1) << 1) | ((r >> 3) & 1); }
// Byte offset of 16-byte chunk c of row r in a tile of 128-byte rows.
__device__ __forceinline__ int g_pos(int r, int c) { return r * 128 + ((c ^ g_swz(r)) << 4); }

template <int n>
__device__ __forceinline__ void g_wait_vm() {
  static_assert(n >= 0 && n < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8));
}

__device__ __forceinline__ void g_wait_lgkm0() { __builtin_amdgcn_s_waitcnt((15) | (3 << 14) | (7 << 4)); }

constexpr unsigned kOOB = 0x80000000u;  // a buffer offset past every range: the lane reads zeros

}  // namespace

template <typename TI, typename TO, int BM, int BN, bool BT, int NS, int WGM = 2, int WGN = 2, int KG = 1>
__global__ __launch_bounds__(64 * WGM * WGN * KG) void gemm_dma_kernel(GemmArgs p) {
  // TI: the 16-bit operand format (bf16 or fp16); operands move as raw 16-bit
  // values, the format only picks the MFMA.
  // KG > 1: KG groups of WGM x WGN wavefronts share the tile; group g takes
  // K-steps g, g + KG, ... through its own part of each stage, and the groups'
  // accumulators are added in group order at the end.  Each SIMD then runs KG
  // wavefronts whose copy and fragment-read latencies hide each other's.
  constexpr bool H = std::is_same<TI, f16>::value;
  static_assert(H || std::is_same<TI, bf16>::value, "16-bit operands");
  constexpr int NW = WGM * WGN;
  constexpr int A_BYTES = BM * 128;
  constexpr int B_BYTES = BN * 128;  // BN rows of 128 B (B^T) or BN / 64 sub-tiles of 64 x 128 B
  constexpr int STAGE = A_BYTES + B_BYTES;
  constexpr int A_PW = A_BYTES / 1024 / NW, B_PW = B_BYTES / 1024 / NW;  // DMA instructions per wavefront
  constexpr int LPT = A_PW + B_PW;
  constexpr int WM = BM / WGM, WN = BN / WGN, TM = WM / 32, TN = WN / 32;
  static_assert(A_PW >= 1 && B_PW >= 1 && A_PW * NW * 1024 == A_BYTES && B_PW * NW * 1024 == B_BYTES,
                "tile too small");
  static_assert(TM >= 1 && TN >= 1 && TM * 32 * WGM == BM && TN * 32 * WGN == BN, "wavefront tiles");
  static_assert((NS - 2) * LPT < 64, "vmcnt range");
  static_assert(KG >= 1, "K groups");
  constexpr int SSET = KG * STAGE;  // one stage of every group
  __shared__ __align__(16) unsigned char lds[NS * SSET];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wall = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int kg = wall / NW, wid = wall % NW;  // K group, wavefront within it
  const int wm = wid / WGN, wn = wid % WGN;
  const int tiles_m = (p.M + BM - 1) / BM, tiles_n = (p.N + BN - 1) / BN;
  int tm, tn;
  tile_coords(blockIdx.x, tiles_m, tiles_n, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const int bz = blockIdx.z;
  const bf16* A = static_cast<const bf16*>(p.A) + (long)bz * p.sA;
  const bf16* B = static_cast<const bf16*>(p.B) + (long)bz * p.sB;
  TO* C = static_cast<TO*>(p.C) + (long)bz * p.sC;
  const TO* R = p.R ? static_cast<const TO*>(p.R) + (long)bz * p.sR : nullptr;
  const int K = p.K;

  // ---- DMA: instruction q of a 128-byte-row tile covers rows 8 q .. 8 q + 7;
  // lane l fills row 8 q + l / 8, physical chunk l % 8.
  const int dr = lane >> 3, dpc = lane & 7;
  // A rows m (B^T rows n): byte offset of the lane's chunk at K-step 0, or kOOB.
  const int rows_a = min(BM, p.M - m0);
  const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(A + (long)m0 * p.lda), (short)0, (int)min(2L * ((rows_a - 1) * p.lda + K), 0x7fffffffL), 0x00020000);
  unsigned aoff[A_PW];
  int akc[A_PW];
#pragma unroll
  for (int u = 0; u < A_PW; ++u) {
    const int row = 8 * (wid * A_PW + u) + dr;
    const int lc = dpc ^ g_swz(row);
    akc[u] = 8 * lc;
    aoff[u] = row < rows_a ? (unsigned)(2 * ((long)row * p.lda + 8 * lc)) : kOOB;
  }
  __amdgpu_buffer_rsrc_t rb;
  unsigned boff[B_PW];
  int bkc[B_PW], brow[B_PW];
  if constexpr (BT) {
    const int rows_b = min(BN, p.N - n0);
    rb = __builtin_amdgcn_make_buffer_rsrc((void*)(B + (long)n0 * p.ldb), (short)0,
                                           (int)min(2L * ((rows_b - 1) * p.ldb + K), 0x7fffffffL), 0x00020000);
#pragma unroll
    for (int u = 0; u < B_PW; ++u) {
      const int row = 8 * (wid * B_PW + u) + dr;
      const int lc = dpc ^ g_swz(row);
      bkc[u] = 8 * lc;
      brow[u] = 0;
      boff[u] = row < rows_b ? (unsigned)(2 * ((long)row * p.ldb + 8 * lc)) : kOOB;
    }
  } else {
    // [K, N]: instruction q -> sub-tile q / 8 (64 columns), k rows 8 (q % 8) + dr.
    const int cols_b = min(BN, p.N - n0);
    rb = __builtin_amdgcn_make_buffer_rsrc((void*)(B + n0), (short)0,
                                           (int)min(2L * ((long)(K - 1) * p.ldb + cols_b), 0x7fffffffL), 0x00020000);
#pragma unroll
    for (int u = 0; u < B_PW; ++u) {
      const int q = wid * B_PW + u;
      const int sub = q / 8, row = 8 * (q % 8) + dr;
      const int col = 64 * sub + 8 * (dpc ^ g_swz(row));
      brow[u] = row;
      bkc[u] = 0;
      boff[u] = col < cols_b ? (unsigned)(2 * ((long)row * p.ldb + col)) : kOOB;
    }
  }
  // Copy instruction u (A for u < A_PW, then B) of K-step s into stage st
  // (K-steps past K copy zeros).
  auto dma1 = [&](int s, int st, int u) __attribute__((always_inline)) {
    const int k0 = (KG * s + kg) * G_BK;
    unsigned char* sb = lds + st * SSET + kg * STAGE;
    if (u < A_PW) {
      const unsigned off = (aoff[u] != kOOB && k0 + akc[u] < K) ? aoff[u] + 2u * k0 : kOOB;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (__attribute__((address_space(3))) void*)(sb + (wid * A_PW + u) * 1024),
                                               16, (int)off, 0, 0, 0);
    } else {
      const int w = u - A_PW;
      unsigned off;
      if constexpr (BT)
        off = (boff[w] != kOOB && k0 + bkc[w] < K) ? boff[w] + 2u * k0 : kOOB;
      else
        off = (boff[w] != kOOB && k0 + brow[w] < K) ? boff[w] + (unsigned)(2L * k0 * p.ldb) : kOOB;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rb, (__attribute__((address_space(3))) void*)(sb + A_BYTES + (wid * B_PW + w) * 1024), 16, (int)off, 0, 0,
          0);
    }
  };
  auto dma = [&](int s, int st) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < LPT; ++u) dma1(s, st, u);
  };

  // ---- fragment offsets within a stage (K-step sub-step ks = 0..3)
  const int lr = lane & 31, lg = lane >> 5;
  // The swizzle depends on row bits 1..3 only, so the 32-row tiles of a
  // wavefront sit 4096 bytes apart: one offset per sub-step, plus 4096 i.
  int afo[4], bto[4], bfo[TN][4][2];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    afo[ks] = g_pos(wm * WM + lr, 2 * ks + lg);
    bto[ks] = A_BYTES + g_pos(wn * WN + lr, 2 * ks + lg);
  }
  if constexpr (!BT) {
    const int i16 = lane & 15, g2 = (lane >> 4) & 1;
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        // lane i of a 16-lane group reads row k (4 per read) at columns n .. n + 3
        const int n = wn * WN + j * 32 + 16 * g2 + 4 * (i16 & 3);
        const int sub = n / 64, nc = n % 64;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int krow = 16 * ks + 8 * lg + 4 * h + (i16 >> 2);
          bfo[j][ks][h] = A_BYTES + sub * 8192 + g_pos(krow, nc / 8) + (nc % 8) * 2;
        }
      }
  }

  floatx16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  // Fragments of sub-step ks (16 K) of the stage at sb.
  auto frags = [&](const unsigned char* sb, int ks, bf16x8 (&af)[TM], bf16x8 (&bfr)[TN])
                   __attribute__((always_inline)) {
    // With B as [K, N] every fragment read is untracked (see
    // ds_read_tr16_b64_async); lds_wait_tie on the B fragments orders them all.
#pragma unroll
    for (int i = 0; i < TM; ++i)
      af[i] = BT ? *reinterpret_cast<const bf16x8*>(sb + afo[ks] + 4096 * i)
                 : ds_read_b128_async(sb + afo[ks] + 4096 * i);
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      if constexpr (BT) {
        bfr[j] = *reinterpret_cast<const bf16x8*>(sb + bto[ks] + 4096 * j);
      } else {
        // (untracked reads: tied by lds_wait_tie before the MFMAs use them)
        const shortx4 x = ds_read_tr16_b64_async(sb + bfo[j][ks][0]);
        const shortx4 y = ds_read_tr16_b64_async(sb + bfo[j][ks][1]);
        bfr[j] = __builtin_bit_cast(bf16x8, __builtin_shufflevector(x, y, 0, 1, 2, 3, 4, 5, 6, 7));
      }
    }
  };
  auto mmas = [&](const bf16x8 (&af)[TM], const bf16x8 (&bfr)[TN]) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) acc[i][j] = mma32_16b<H>(af[i], bfr[j], acc[i][j]);
  };
  // Every wavefront's copies of a stage have landed once each waited for its
  // own (vmcnt) and all passed the barrier.  A bare s_barrier, not
  // __syncthreads(): the latter's fence makes the compiler wait for every
  // outstanding copy (vmcnt(0)), which would leave one stage in flight
  // instead of NS - 1.  The signal fences keep the compiler from moving LDS
  // accesses across the barrier; they emit no instruction.
  auto barrier = [&]() __attribute__((always_inline)) {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
  };

  // Software pipeline: the fragments of sub-step ks + 1 are read while the
  // MFMAs of sub-step ks run; the stage hand-over (wait, barrier) sits between
  // the reads and the MFMAs of the last sub-step, so the barrier wait overlaps
  // MFMAs already issued.  The copies go out interleaved with MFMAs, never in
  // a burst (each holds the wavefront's issue while the address unit drains
  // it, ~35 cycles).  With three or more stages, the copies of K-step s+NS-1
  // (into the stage freed at the end of step s-1) are spread over the four
  // sub-steps of step s, NS-2 steps ahead of use; with two stages, the copies
  // of K-step s+NS go out in two parts, the first H2 with the last sub-step,
  // right after the barrier that frees their stage, the rest with the first
  // sub-step of step s+1, and must land by the end of step s+1.
  constexpr bool SPREAD = NS >= 3;
  constexpr int NMMA = TM * TN;
  constexpr int Q = (LPT + 3) / 4;  // copies per sub-step when spread
  constexpr int H2 = (LPT + 1) / 2;  // two stages: copies issued right after the barrier
  // Copies issued after K-step s+1's last one when step s waits for it: with
  // SPREAD, K-steps s+2 .. s+NS-2 and the first 3 Q copies of K-step s+NS-1
  // (its last ones go out after the wait); with two stages, none (the wait
  // takes every copy in flight).
  constexpr int WAITN = SPREAD ? (NS - 3) * LPT + 3 * Q : (NS - 2) * LPT;
  static_assert(!SPREAD || 3 * Q <= LPT, "the last sub-step's share of the copies is not negative");
  // The MFMAs of one sub-step with copies u0 .. u1-1 of K-step sd between them.
  auto mma_copy = [&](const bf16x8 (&af)[TM], const bf16x8 (&bfr)[TN], int sd, int u0, int u1)
                      __attribute__((always_inline)) {
    const int per = (u1 - u0 + NMMA - 1) / NMMA;
#pragma unroll
    for (int k = 0; k < NMMA; ++k) {
      acc[k / TN][k % TN] = mma32_16b<H>(af[k / TN], bfr[k % TN], acc[k / TN][k % TN]);
#pragma unroll
      for (int u = u0 + k * per; u < u0 + (k + 1) * per && u < u1; ++u) dma1(sd, sd % NS, u);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  // Steps of the loop: KG K-steps each (a group's K-steps past K copy zeros).
  const int nk = ((K + G_BK - 1) / G_BK + KG - 1) / KG;
  const unsigned char* const glds = lds + kg * STAGE;  // this group's part of stage 0
  // K-steps 0 .. NS-2, and with two stages the first H2 copies of K-step
  // NS-1 (step 0 issues the rest, as every step does for the K-step after it).
#pragma unroll
  for (int s = 0; s < NS - 1; ++s) dma(s, s);
  if constexpr (!SPREAD) {
#pragma unroll
    for (int u = 0; u < H2; ++u) dma1(NS - 1, NS - 1, u);
  }
  g_wait_vm<(NS - 2) * LPT + (SPREAD ? 0 : H2)>();  // K-step 0 has landed
  barrier();
  bf16x8 fa[2][TM], fb[2][TN];
  frags(glds, 0, fa[0], fb[0]);
#pragma unroll 1
  for (int s = 0; s < nk; ++s) {
    const unsigned char* sb = glds + (s % NS) * SSET;
#pragma unroll
    for (int ks = 0; ks < 3; ++ks) {
      if constexpr (!BT) {  // B^T fragments of sub-step ks have landed (read one sub-step ago)
#pragma unroll
        for (int j = 0; j < TN; ++j) lds_wait_tie(fb[ks & 1][j]);
      }
      frags(sb, ks + 1, fa[(ks + 1) & 1], fb[(ks + 1) & 1]);
      __builtin_amdgcn_sched_barrier(0);  // the reads stay ahead of the MFMAs
      if constexpr (SPREAD)
        mma_copy(fa[ks & 1], fb[ks & 1], s + NS - 1, ks * Q, min((ks + 1) * Q, LPT));
      else if (ks == 0)
        mma_copy(fa[0], fb[0], s + NS - 1, H2, LPT);  // the rest of K-step s+1
      else
        mmas(fa[ks & 1], fb[ks & 1]);
      __builtin_amdgcn_sched_barrier(0);
    }
    g_wait_vm<WAITN>();  // K-step s+1 has landed
    g_wait_lgkm0();      // this wavefront's reads of K-step s are done
    if constexpr (!BT) {
#pragma unroll
      for (int j = 0; j < TN; ++j) lds_wait_tie(fb[1][j]);
    }
    barrier();                    // ... for every wavefront
    // The next K-step's first fragment reads come first in program order
    // (the copies may alias them), then the last sub-step's MFMAs, whose
    // fragments are already in registers.
    frags(glds + ((s + 1) % NS) * SSET, 0, fa[0], fb[0]);
    if constexpr (SPREAD)
      mma_copy(fa[1], fb[1], s + NS - 1, 3 * Q, LPT);
    else
      mma_copy(fa[1], fb[1], s + NS, 0, H2);  // into K-step s's stage
  }
  __builtin_amdgcn_s_waitcnt(0);  // the copies of K-steps past K have landed

  // Epilogue staging (staged path): NW wavefronts x RP rows of PITCH floats.
  constexpr int OE = 16 / sizeof(TO);  // output elements per 16-byte store
  constexpr int WC_MAX = WN;           // staged columns per wavefront (SwiGLU: WN / 2)
  constexpr int PITCH = WC_MAX + 4;    // staged row pitch, floats
  constexpr int RP = NW * WM * PITCH * 4 <= NS * SSET ? WM : 32;  // rows per pass
  constexpr int TP = RP / 32;                                      // tiles per pass
  static_assert(NW * RP * PITCH * 4 <= NS * SSET, "the staged rows fit the stages");
  if constexpr (KG > 1) {
    // Groups 1 .. KG-1 leave their accumulators in LDS past the staging
    // area (lane-major float4 chunks); group 0 adds them in group order and
    // writes the tile alone.  The second barrier is the last one any
    // wavefront takes part in.
    constexpr int NCH = TM * TN * 4;  // float4 chunks per lane
    constexpr int ROFF = (NW * RP * PITCH * 4 + 15) / 16 * 16;
    static_assert(ROFF + (KG - 1) * NW * NCH * 1024 <= NS * SSET, "the partial sums fit the stages");
    float4* red = reinterpret_cast<float4*>(lds + ROFF);
    __syncthreads();  // every wavefront is done with the stages
    if (kg > 0) {
#pragma unroll
      for (int c = 0; c < NCH; ++c) {
        const floatx16& a = acc[c / 4 / TN][c / 4 % TN];
        red[(((kg - 1) * NW + wid) * NCH + c) * 64 + lane] =
            make_float4(a[4 * (c % 4)], a[4 * (c % 4) + 1], a[4 * (c % 4) + 2], a[4 * (c % 4) + 3]);
      }
    }
    __syncthreads();
    if (kg > 0) return;
#pragma unroll
    for (int g = 1; g < KG; ++g)
#pragma unroll
      for (int c = 0; c < NCH; ++c) {
        const float4 v = red[(((g - 1) * NW + wid) * NCH + c) * 64 + lane];
        floatx16& a = acc[c / 4 / TN][c / 4 % TN];
        a[4 * (c % 4)] += v.x;
        a[4 * (c % 4) + 1] += v.y;
        a[4 * (c % 4) + 2] += v.z;
        a[4 * (c % 4) + 3] += v.w;
      }
  }

  // Epilogue: accumulator element e of tile (i, j) is C[row][col] with
  // row = 8 * (e / 4) + 4 * (lane / 32) + e % 4, col = lane % 32.
  if (p.epi != kEpiElem) {
    // Staged: the wavefront writes RP rows of its WM x WC block (fp32) to its
    // own LDS rows, then each lane reads OE consecutive values of a row, adds
    // the residual in fp32 and stores them as one 16-byte vector; WM / RP
    // passes.  With the SwiGLU pairing, tiles 2k and 2k+1 of the wavefront
    // hold gate and up for the same 32 output columns (the weight rows are
    // interleaved in groups of 32), and the block written is
    // silu(TO(gate)) * TO(up): the values a gate and an up GEMM with TO
    // outputs would hand the SwiGLU kernel.
    if constexpr (KG == 1) __syncthreads();  // every wavefront is done with the stages (KG > 1: above)
    float* stg = reinterpret_cast<float*>(lds) + wid * (RP * PITCH);
    const bool sw = p.epi == kEpiSwiglu;
    const int wc = sw ? WN / 2 : WN;
    // Rows of the block go to rows m0 + wm WM ..; columns to c0 ...
    const int c0 = sw ? (n0 + wn * WN) / 2 : n0 + wn * WN;
    const int ncols = sw ? p.N / 2 : p.N;
    const int cpr = wc / OE;  // 16-byte chunks per staged row
#pragma unroll
    for (int ip = 0; ip < TM / TP; ++ip) {
      if (sw) {
        if constexpr (TN % 2 == 0) {  // gate/up tiles come in pairs (the host picks such a tile)
#pragma unroll
          for (int t = 0; t < TP; ++t)
#pragma unroll
            for (int k = 0; k < TN / 2; ++k)
#pragma unroll
              for (int e = 0; e < 16; ++e) {
                const float g = to_f32<TO>(from_f32<TO>(acc[ip * TP + t][2 * k][e]));
                const float u = to_f32<TO>(from_f32<TO>(acc[ip * TP + t][2 * k + 1][e]));
                stg[(t * 32 + 8 * (e / 4) + 4 * lg + (e % 4)) * PITCH + k * 32 + lr] = silu(g) * u;
              }
        }
      } else {
#pragma unroll
        for (int t = 0; t < TP; ++t)
#pragma unroll
          for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e)
              stg[(t * 32 + 8 * (e / 4) + 4 * lg + (e % 4)) * PITCH + j * 32 + lr] = acc[ip * TP + t][j][e];
      }
#pragma unroll 4
      for (int c = lane; c < RP * cpr; c += 64) {
        const int rl = c / cpr, cl = (c % cpr) * OE;
        const int row = m0 + wm * WM + ip * RP + rl, col = c0 + cl;
        if (row < p.M && col < ncols) {
          float v[OE];
#pragma unroll
          for (int e = 0; e < OE; e += 4) {
            const float4 x = *reinterpret_cast<const float4*>(stg + rl * PITCH + cl + e);
            v[e] = x.x;
            v[e + 1] = x.y;
            v[e + 2] = x.z;
            v[e + 3] = x.w;
          }
          if (R) {
            float r[OE];
            load16(R + (long)row * p.ldr + col, r);
#pragma unroll
            for (int e = 0; e < OE; ++e) v[e] += r[e];
          }
          store_vec<OE>(C + (long)row * p.ldc + col, v);
        }
      }
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int col = n0 + wn * WN + j * 32 + lr;
      if (col >= p.N) continue;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int row = m0 + wm * WM + i * 32 + 8 * (e / 4) + 4 * lg + (e % 4);
        if (row < p.M) {
          float vv = acc[i][j][e];
          if (R) vv += to_f32(R[(long)row * p.ldr + col]);
          C[(long)row * p.ldc + col] = from_f32<TO>(vv);
        }
      }
    }
}

static bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// The staged epilogue stores 16-byte vectors: C (and R) rows, batch strides
// and N must keep every vector 16-byte aligned.
template <typename TO>
static bool staged_ok(const GemmArgs& a) {
  constexpr long OE = 16 / sizeof(TO);
  const bool c_ok = aligned16(a.C) && a.ldc % OE == 0 && a.sC % OE == 0 && a.N % OE == 0;
  const bool r_ok = !a.R || (aligned16(a.R) && a.ldr % OE == 0 && a.sR % OE == 0);
  return c_ok && r_ok;
}

// Tiles of the LDS-DMA kernel.
// K2: two K groups of four wavefronts per tile.
enum DmaTile { kT64x64, kT64x128, kT128x128, kT128x256, kT256x128, kT256x192, kT256x256, kT64x64K2, kT64x128K2,
               kTileCount };

template <typename TI, typename TO, bool BT>
static void launch_dma(DmaTile t, const GemmArgs& g, int batch, hipStream_t st) {
  auto grid = [&](int bm, int bn) {
    return dim3((unsigned)((long)((g.M + bm - 1) / bm) * ((g.N + bn - 1) / bn)), 1, (unsigned)batch);
  };
  switch (t) {
    case kT256x256: gemm_dma_kernel<TI, TO, 256, 256, BT, 2, 2, 4><<<grid(256, 256), dim3(512), 0, st>>>(g); break;
    case kT256x192: gemm_dma_kernel<TI, TO, 256, 192, BT, 2, 4, 2><<<grid(256, 192), dim3(512), 0, st>>>(g); break;
    case kT256x128: gemm_dma_kernel<TI, TO, 256, 128, BT, 3, 4, 2><<<grid(256, 128), dim3(512), 0, st>>>(g); break;
    case kT128x256: gemm_dma_kernel<TI, TO, 128, 256, BT, 3, 2, 4><<<grid(128, 256), dim3(512), 0, st>>>(g); break;
    case kT128x128: gemm_dma_kernel<TI, TO, 128, 128, BT, 4><<<grid(128, 128), dim3(256), 0, st>>>(g); break;
    case kT64x128: gemm_dma_kernel<TI, TO, 64, 128, BT, 6><<<grid(64, 128), dim3(256), 0, st>>>(g); break;
    case kT64x128K2: gemm_dma_kernel<TI, TO, 64, 128, BT, 3, 2, 2, 2><<<grid(64, 128), dim3(512), 0, st>>>(g); break;
    case kT64x64K2: gemm_dma_kernel<TI, TO, 64, 64, BT, 4, 2, 2, 2><<<grid(64, 64), dim3(512), 0, st>>>(g); break;
    default: gemm_dma_kernel<TI, TO, 64, 64, BT, 8><<<grid(64, 64), dim3(256), 0, st>>>(g); break;
  }
}

// NKL_GEMM_TILE=64x64|64x128|128x128|128x256|256x128|256x192|256x256|64x64k2|64x128k2
// forces a tile (for measurements); -1 when unset or unknown.
static int forced_tile() {
  static const int forced = [] {
    const char* f = getenv("NKL_GEMM_TILE");
    if (!f) return -1;
    static const char* names[kTileCount] = {"64x64",   "64x128",   "128x128",  "128x256", "256x128",
                                            "256x192", "256x256", "64x64k2", "64x128k2"};
    for (int i = 0; i < kTileCount; ++i)
      if (!strcmp(f, names[i])) return i;
    return -1;
  }();
  return forced;
}

static long tiles_of(const GemmArgs& a, int bm, int bn, int batch) {
  return (long)((a.M + bm - 1) / bm) * ((a.N + bn - 1) / bn) * batch;
}

// Tile choice.  With a 128x128 tile or larger for every CU, the tile whose
// rounds of 256 workgroups (one per CU) cost least, at the time per K-step
// of a round measured on MI355X (bf16, K-contiguous B): 256x256 1.9 us,
// 256x192 1.75 us, 256x128 1.25 us, 128x128 0.8 us.  256x192 fills the CUs
// where 256x256 leaves a quarter idle (2048 x 6144: 256 tiles against 192).
// Smaller GEMMs: the largest tile that still gives every CU a workgroup, with
// two K groups (64x64: 1024^3 9.0 -> 8.4 us; 64x128: 2-6% on 1024-2048-row
// shapes).
static DmaTile choose_tile(const GemmArgs& a, int batch) {
  if (forced_tile() >= 0) return (DmaTile)forced_tile();
  const long t128 = tiles_of(a, 128, 128, batch);
  if (t128 >= 256) {
    auto rounds = [](long t) { return (double)((t + 255) / 256); };
    const struct { DmaTile t; double c; } cand[] = {
        {kT256x256, 1.9 * rounds(tiles_of(a, 256, 256, batch))},
        {kT256x192, 1.75 * rounds(tiles_of(a, 256, 192, batch))},
        {kT256x128, 1.25 * rounds(tiles_of(a, 256, 128, batch))},
        {kT128x128, 0.8 * rounds(t128)}};
    DmaTile best = kT256x256;
    double cb = 1e30;
    for (const auto& c : cand)
      if (c.c < cb) cb = c.c, best = c.t;
    return best;
  }
  if (tiles_of(a, 64, 128, batch) >= 256) return kT64x128K2;
  return kT64x64K2;
}

// CUs of the current device (256 on MI355X), read once per device (threads
// that race to read it store the same value).
static int gemm_cus() {
  static std::atomic<int> cus[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = cus[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cus[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

// Rows and columns of a tile.
static void tile_dims(DmaTile t, int& bm, int& bn) {
  switch (t) {
    case kT256x256: bm = 256, bn = 256; break;
    case kT256x192: bm = 256, bn = 192; break;
    case kT256x128: bm = 256, bn = 128; break;
    case kT128x256: bm = 128, bn = 256; break;
    case kT128x128: bm = 128, bn = 128; break;
    case kT64x128:
    case kT64x128K2: bm = 64, bn = 128; break;
    default: bm = 64, bn = 64; break;
  }
}

// Time per K-step of a round of one-per-CU workgroups (the tile choice's
// figures), 0 for the tiles it does not price.
static double round_step_us(DmaTile t) {
  return t == kT256x256 ? 1.9 : t == kT256x192 ? 1.75 : t == kT256x128 ? 1.25 : t == kT128x128 ? 0.8 : 0.0;
}

// Column split of a launch whose 256-row tiles leave a partial last round:
// the columns of the whole rounds go to a first launch, the rest to a second
// launch with the tile chosen for them alone (2048 x 11264: 352 tiles of
// 256 x 256 make a round and then 96 -- instead, 256 such tiles over the first
// 8192 columns and 192 tiles of 256 x 128 over the last 3072).  The plan is
// the cheapest, at the round times above plus 2 us for a second launch, of
// the chosen tile over all columns and the column splits of the 256-row
// tiles.  n1 = 0: one launch with t1.  swiglu: the gate/up GEMM, whose
// wavefronts own 64 columns (no 256 x 192 tile).
struct TilePlan {
  DmaTile t1;
  int n1;
  DmaTile t2;
};
static TilePlan plan_tiles(const GemmArgs& a, DmaTile t, int batch, bool swiglu) {
  TilePlan best{t, 0, t};
  if (batch != 1 || forced_tile() >= 0 || round_step_us(t) == 0.0) return best;
  const long cus = gemm_cus();
  const double nk = (a.K + G_BK - 1) / G_BK;
  auto cost = [&](DmaTile x, int n) {
    int bm, bn;
    tile_dims(x, bm, bn);
    const long tiles = (long)((a.M + bm - 1) / bm) * ((n + bn - 1) / bn);
    return round_step_us(x) * (double)((tiles + cus - 1) / cus) * nk;
  };
  double cb = cost(t, a.N);
  for (DmaTile x : {kT256x256, kT256x192, kT256x128}) {
    if (swiglu && x == kT256x192) continue;
    int bm, bn;
    tile_dims(x, bm, bn);
    const long tm = (a.M + 255) / 256, tiles = tm * ((a.N + bn - 1) / bn);
    if (tiles <= cus || tiles % cus == 0 || tm > cus) continue;
    const long n1 = (tiles / cus) * cus / tm * bn;  // the columns of the whole rounds
    if (n1 <= 0 || n1 >= a.N) continue;
    GemmArgs rest = a;
    rest.N = (int)(a.N - n1);
    DmaTile t2 = choose_tile(rest, 1);
    if (swiglu && t2 == kT256x192) t2 = kT256x256;
    if (round_step_us(t2) == 0.0) continue;
    const double c = cost(x, (int)n1) + cost(t2, rest.N) + 2.0;
    if (c < cb) cb = c, best = TilePlan{x, (int)n1, t2};
  }
  return best;
}

// launch_dma after plan_tiles: one launch, or two over a column split.
template <typename TI, typename TO, bool BT>
static void launch_dma_cols(DmaTile t, const GemmArgs& g, int batch, bool swiglu, hipStream_t st) {
  const TilePlan pl = plan_tiles(g, t, batch, swiglu);
  if (pl.n1 == 0) {
    launch_dma<TI, TO, BT>(pl.t1, g, batch, st);
    return;
  }
  GemmArgs g1 = g, g2 = g;
  g1.N = pl.n1;
  g2.N = g.N - pl.n1;
  const uint16_t* B = static_cast<const uint16_t*>(g.B);
  g2.B = BT ? B + (long)pl.n1 * g.ldb : B + pl.n1;
  const long coff = swiglu ? pl.n1 / 2 : pl.n1;
  g2.C = static_cast<TO*>(g.C) + coff;
  if (g.R) g2.R = static_cast<const TO*>(g.R) + coff;
  launch_dma<TI, TO, BT>(pl.t1, g1, 1, st);
  launch_dma<TI, TO, BT>(pl.t2, g2, 1, st);
}

template <typename T, typename TO, bool BT>
static int gemm_dispatch(const GemmArgs& a, int batch, int variant, hipStream_t st) {
  constexpr int E = VecE<T>::value;
  const bool vec = aligned16(a.A) && aligned16(a.B) && a.K % E == 0 && a.lda % E == 0 && a.ldb % E == 0 &&
                   a.sA % E == 0 && a.sB % E == 0 && (BT || a.N % E == 0);
  constexpr bool half = std::is_same<T, f16>::value;
  if constexpr (half) {
    // fp16 operands: the LDS-DMA kernel, or for the naive variant, unaligned
    // operands, K or leading dimensions off a multiple of 8 and operands over
    // 2 GiB, the one-tile-per-wavefront kernel.
    const long a_bytes = 2L * ((long)(a.M - 1) * a.lda + a.K), b_bytes = BT ? 2L * ((long)(a.N - 1) * a.ldb + a.K)
                                                                        : 2L * ((long)(a.K - 1) * a.ldb + a.N);
    if (variant == NKL_GEMM_NAIVE || !vec || a_bytes >= (1L << 31) || b_bytes >= (1L << 31)) {
      const long tiles = (long)((a.M + 31) / 32) * ((a.N + 31) / 32);
      gemm_naive_kernel<T, TO, BT><<<dim3((unsigned)((tiles + 3) / 4), 1, batch), dim3(256), 0, st>>>(a);
      return check_launch("nkl_gemm(naive)");
    }
    GemmArgs g = a;
    g.epi = staged_ok<TO>(a) ? kEpiStaged : kEpiElem;
    launch_dma_cols<f16, TO, BT>(choose_tile(a, batch), g, batch, false, st);
    return check_launch("nkl_gemm(blocked)");
  } else {
  if (variant == NKL_GEMM_NAIVE || !vec) {
    const long tiles = (long)((a.M + 31) / 32) * ((a.N + 31) / 32);
    gemm_naive_kernel<T, TO, BT><<<dim3((unsigned)((tiles + 3) / 4), 1, batch), dim3(256), 0, st>>>(a);
    return check_launch("nkl_gemm(naive)");
  }
  const long t128 = (long)((a.M + 127) / 128) * ((a.N + 127) / 128) * batch;
  const long t64x128 = (long)((a.M + 63) / 64) * ((a.N + 127) / 128) * batch;
  if constexpr (std::is_same<T, bf16>::value) {
    // bf16: the LDS-DMA kernel, whose buffer offsets need operands under 2 GB.
    const long a_bytes = 2L * ((long)(a.M - 1) * a.lda + a.K), b_bytes = BT ? 2L * ((long)(a.N - 1) * a.ldb + a.K)
                                                                        : 2L * ((long)(a.K - 1) * a.ldb + a.N);
    if (a_bytes < (1L << 31) && b_bytes < (1L << 31)) {
      GemmArgs g = a;
      g.epi = staged_ok<TO>(a) ? kEpiStaged : kEpiElem;
      launch_dma_cols<bf16, TO, BT>(choose_tile(a, batch), g, batch, false, st);
      return check_launch("nkl_gemm(blocked)");
    }
  }
  if (t128 >= 256) {
    const long tiles = (long)((a.M + 127) / 128) * ((a.N + 127) / 128);
    gemm_blocked_kernel<T, TO, 128, 128, BT><<<dim3((unsigned)tiles, 1, batch), dim3(256), 0, st>>>(a);
  } else if (t64x128 >= 256) {
    const long tiles = (long)((a.M + 63) / 64) * ((a.N + 127) / 128);
    gemm_blocked_kernel<T, TO, 64, 128, BT><<<dim3((unsigned)tiles, 1, batch), dim3(256), 0, st>>>(a);
  } else {
    const long tiles = (long)((a.M + 63) / 64) * ((a.N + 63) / 64);
    gemm_blocked_kernel<T, TO, 64, 64, BT><<<dim3((unsigned)tiles, 1, batch), dim3(256), 0, st>>>(a);
  }
  return check_launch("nkl_gemm(blocked)");
  }
}

template <typename T, typename TO>
static int gemm_layout(const GemmArgs& a, int b_trans, int batch, int variant, hipStream_t st) {
  return b_trans ? gemm_dispatch<T, TO, true>(a, batch, variant, st)
                 : gemm_dispatch<T, TO, false>(a, batch, variant, st);
}

}  // namespace nkl

using namespace nkl;

extern "C" int nkl_gemm(const void* A, const void* B, void* C, const void* R, int M, int N, int K, long lda,
                        long ldb, long ldc, long ldr, int b_trans, int batch, long strideA, long strideB,
                        long strideC, long strideR, int dtype_in, int dtype_out, int variant, void* stream) {
  if (M < 0 || N < 0 || K < 0 || batch < 0)
    return set_error(NKL_EINVAL, "nkl_gemm: negative shape M=%d N=%d K=%d batch=%d", M, N, K, batch);
  if (variant != NKL_GEMM_BLOCKED && variant != NKL_GEMM_NAIVE)
    return set_error(NKL_EINVAL, "nkl_gemm: unknown variant %d", variant);
  if (M == 0 || N == 0 || batch == 0) return NKL_OK;
  if (lda < K || ldc < N || (R && ldr < N) || (b_trans ? ldb < K : ldb < N))
    return set_error(NKL_EINVAL, "nkl_gemm: leading dimension too small (lda=%ld ldb=%ld ldc=%ld)", lda, ldb, ldc);
  if (!A || !B || !C) return set_error(NKL_EINVAL, "nkl_gemm: null operand pointer");
  GemmArgs a{A, B, C, R, M, N, K, lda, ldb, ldc, ldr, strideA, strideB, strideC, strideR};
  hipStream_t st = (hipStream_t)stream;
  if (dtype_in == NKL_F32 && dtype_out == NKL_F32) return gemm_layout<float, float>(a, b_trans, batch, variant, st);
  if (dtype_in == NKL_BF16 && dtype_out == NKL_BF16) return gemm_layout<bf16, bf16>(a, b_trans, batch, variant, st);
  if (dtype_in == NKL_BF16 && dtype_out == NKL_F32) return gemm_layout<bf16, float>(a, b_trans, batch, variant, st);
  if (dtype_in == NKL_F16 && dtype_out == NKL_F16) return gemm_layout<f16, f16>(a, b_trans, batch, variant, st);
  if (dtype_in == NKL_F16 && dtype_out == NKL_F32) return gemm_layout<f16, float>(a, b_trans, batch, variant, st);
  return set_error(NKL_EDTYPE, "nkl_gemm: unsupported dtype pair (%d -> %d)", dtype_in, dtype_out);
}

extern "C" int nkl_gemm_swiglu(const void* A, const void* Bgu, void* C, int M, int N, int K, long lda, long ldb,
                               long ldc, int dtype, void* stream) {
  if (M < 0 || N < 0 || K < 0)
    return set_error(NKL_EINVAL, "nkl_gemm_swiglu: negative shape M=%d N=%d K=%d", M, N, K);
  if (dtype != NKL_BF16 && dtype != NKL_F16)
    return set_error(NKL_EDTYPE, "nkl_gemm_swiglu: only bf16 and fp16 are supported (dtype %d)", dtype);
  if (M == 0 || N == 0) return NKL_OK;
  if (N % 32 != 0) return set_error(NKL_EINVAL, "nkl_gemm_swiglu: N=%d must be a multiple of 32", N);
  if (!A || !Bgu || !C) return set_error(NKL_EINVAL, "nkl_gemm_swiglu: null operand pointer");
  if (lda < K || ldb < K || ldc < N)
    return set_error(NKL_EINVAL, "nkl_gemm_swiglu: leading dimension too small (lda=%ld ldb=%ld ldc=%ld)", lda, ldb,
                     ldc);
  if (!aligned16(A) || !aligned16(Bgu) || !aligned16(C) || K % 8 != 0 || lda % 8 != 0 || ldb % 8 != 0 ||
      ldc % 8 != 0)
    return set_error(NKL_EINVAL, "nkl_gemm_swiglu: operands must be 16-byte aligned with K and leading dimensions "
                     "multiples of 8");
  const long a_bytes = 2L * ((long)(M - 1) * lda + K), b_bytes = 2L * ((long)(2L * N - 1) * ldb + K);
  if (a_bytes >= (1L << 31) || b_bytes >= (1L << 31))
    return set_error(NKL_EINVAL, "nkl_gemm_swiglu: operands must be under 2 GiB");
  GemmArgs a{A, Bgu, C, nullptr, M, 2 * N, K, lda, ldb, ldc, 0, 0, 0, 0, 0, kEpiSwiglu};
  hipStream_t st = (hipStream_t)stream;
  // A tile whose wavefronts own 64 columns (one gate/up pair), summing the
  // K-steps in the order the separate M x N gate and up GEMMs would: in two
  // K groups where their tile has them.
  GemmArgs half = a;
  half.N = N;
  const DmaTile th = choose_tile(half, 1);
  DmaTile t = th == kT64x64K2 || th == kT64x128K2 ? kT64x128K2 : choose_tile(a, 1);
  if (t == kT64x64) t = kT64x128;
  if (t == kT64x64K2) t = kT64x128K2;
  if (t == kT256x192) t = kT256x256;
  if (dtype == NKL_F16)
    launch_dma_cols<f16, f16, true>(t, a, 1, true, st);
  else
    launch_dma_cols<bf16, bf16, true>(t, a, 1, true, st);
  return check_launch("nkl_gemm_swiglu");
}

extern "C" int nkl_check_blocks(int BM, int BN) {
  if (BM < 1 || BN < 1) return set_error(NKL_EINVAL, "nkl_check_blocks: BM=%d BN=%d must be positive", BM, BN);
  if (BM * BN > 8)
    return set_error(NKL_ELIMIT,
                     "BM*BN = %d fp32 [128,512] accumulators exceed the 8 PSUM banks the blocked matmul may hold",
                     BM * BN);
  return NKL_OK;
}
