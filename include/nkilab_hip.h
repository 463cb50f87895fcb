/*
 * nkilab_hip.h -- C ABI of libnkilab_hip.so, the gfx950 (MI355X) kernel set
 * behind nkilab.ops / nkilab.model.
 *
 * Every entry point replaces one `nki.simulate(kernel)(...)` call of the
 * reference host layer (nkilab/ops.py) and is bound from Python with ctypes
 * (nkilab/_lib.py).  Conventions shared by all entry points:
 *
 *   - Pointers are device pointers allocated by the caller.  The library never
 *     allocates or frees memory; kernels that need scratch space (the unfused
 *     softmax, the naive attention) take a caller-provided workspace whose
 *     size is reported by the matching *_workspace_bytes() function.
 *   - Strides (ld*, *_sh, *_ss, batch strides) are in ELEMENTS, not bytes.
 *   - dtype codes: NKL_F32 = 0 (float32), NKL_BF16 = 1 (bfloat16),
 *     NKL_F16 = 2 (float16: the 16-bit operand format with 11 significant
 *     bits, taken by the GEMMs, the RMSNorm output, the gate/up SwiGLU GEMM
 *     and the causal attention; see each entry point).
 *   - `stream` is a hipStream_t passed as void* (0 = the null stream).  Every
 *     call only enqueues work and returns; it is asynchronous with respect to
 *     the host.  State kept across calls: the per-thread error string; the
 *     process-wide attention configuration (nkl_flash_attn_configure and
 *     nkl_flash_attn_configure_polls, and the NKL_FLASH_* / NKL_GEMM_TILE
 *     environment read once); a per-device cache of the CU count; and the
 *     per-device static scratch of nkl_flash_attn_causal_noalloc.  Calls are
 *     safe from several threads at once, except that a configuration change
 *     must not overlap attention calls that size or launch under it, and
 *     noalloc calls that may overlap on one device race on its scratch.
 *   - Return value: NKL_OK (0) on success, a negative NKL_E* code otherwise;
 *     nkl_last_error_string() describes the last failure on this thread.
 */
#ifndef NKILAB_HIP_H
#define NKILAB_HIP_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NKL_ABI_VERSION 1

enum { NKL_F32 = 0, NKL_BF16 = 1, NKL_F16 = 2 };

enum {
  NKL_OK = 0,
  NKL_EINVAL = -1,      /* bad shape / stride / argument */
  NKL_EDTYPE = -2,      /* unsupported dtype combination */
  NKL_ELAUNCH = -3,     /* the HIP launch failed */
  NKL_EWORKSPACE = -4,  /* workspace missing or too small */
  NKL_ELIMIT = -5       /* an on-chip accumulator budget is exceeded */
};

/* GEMM variants: the reference's two matmul kernels. */
enum { NKL_GEMM_BLOCKED = 0, NKL_GEMM_NAIVE = 1 };

/* Version of this ABI (NKL_ABI_VERSION). */
int nkl_abi_version(void);

/* Human-readable description of the last error returned on this thread. */
const char* nkl_last_error_string(void);

/*
 * C[b] = A[b] . op(B[b]) (+ R[b]),  b in [0, batch)
 *
 * Replaces nkilab/kernels/matmul.py:46 (matmul_blocked, variant
 * NKL_GEMM_BLOCKED) and nkilab/kernels/matmul.py:24 (matmul_naive, variant
 * NKL_GEMM_NAIVE), called from nkilab/ops.py:48 and :51.
 *   A: [M, K] row-major (lda >= K).
 *   B: b_trans == 0 -> [K, N] row-major (ldb >= N), the reference's `rhs`;
 *      b_trans == 1 -> [N, K] row-major (ldb >= K), e.g. nn.Linear.weight.
 *   C: [M, N] row-major (ldc >= N), dtype_out.
 *   R: optional residual added in the fp32 epilogue ([M, N], ldr, dtype_out);
 *      NULL for none.
 * Products accumulate in fp32; C is rounded once (round-to-nearest-even) to
 * dtype_out.  dtype_in in {F32, BF16, F16}; dtype_out in {F32, dtype_in}.
 * BF16 and F16 operands take the LDS-DMA kernel when A and B are 16-byte
 * aligned, K, lda, ldb (and N when b_trans == 0) are multiples of 8 and the
 * operands are under 2 GiB; other shapes, and variant NKL_GEMM_NAIVE, take a
 * one-tile-per-wavefront kernel (the same fp32 accumulation).
 * The work is enqueued on `stream` as one kernel launch, or as two over
 * column ranges when the large tiles would leave a partial last round of
 * workgroups; nothing is allocated, and the call can be captured in a graph.
 */
int nkl_gemm(const void* A, const void* B, void* C, const void* R,
             int M, int N, int K, long lda, long ldb, long ldc, long ldr,
             int b_trans, int batch, long strideA, long strideB, long strideC,
             long strideR, int dtype_in, int dtype_out, int variant,
             void* stream);

/*
 * C = silu(A . Wg^T) * (A . Wu^T): the decoder's gate and up projections and
 * the SwiGLU between them in one GEMM (the fusion docs/STUDY_GUIDE.md:57
 * suggests for nkilab/model.py:88, which calls ops.swiglu, nkilab/ops.py:64,
 * on two matmul outputs).
 *   A:   [M, K] dtype (lda >= K), dtype in {BF16, F16}.
 *   Bgu: [2N, K] dtype (ldb >= K), the rows of Wg and Wu ([N, K] each)
 *        interleaved in groups of 32: rows 64 j .. 64 j + 31 are Wg rows
 *        32 j .., rows 64 j + 32 .. 64 j + 63 are Wu rows 32 j ...
 *   C:   [M, N] dtype (ldc >= N).
 * N must be a multiple of 32; pointers 16-byte aligned; K, lda, ldb, ldc
 * multiples of 8.  The gate and up accumulators are rounded to dtype before
 * silu(gate) * up is formed in fp32 and rounded once, so C equals what two
 * dtype GEMMs followed by a SwiGLU in dtype produce.  Like nkl_gemm, one or
 * two kernel launches on `stream`.
 */
int nkl_gemm_swiglu(const void* A, const void* Bgu, void* C, int M, int N,
                    int K, long lda, long ldb, long ldc, int dtype,
                    void* stream);

/*
 * The reference's PSUM block check (nkilab/kernels/matmul.py:58): returns
 * NKL_OK when a BM x BN block of fp32 accumulator tiles fits the 8-tile
 * budget, NKL_ELIMIT (with a message naming PSUM) otherwise.  Used by the
 * kernel-level mirror nkilab.kernels.matmul.matmul_blocked.
 */
int nkl_check_blocks(int BM, int BN);

/*
 * y = softmax(x) over the last dimension, fused single pass.
 * Replaces nkilab/kernels/norm.py:65 (softmax_fused), nkilab/ops.py:57.
 * x: [rows, cols] (ldx), y: [rows, cols] (ldy), same dtype.  Row max and sum
 * in fp32, exp(x - max) * (1 / sum) rounded once to dtype.
 */
int nkl_softmax(const void* x, void* y, int rows, int cols, long ldx,
                long ldy, int dtype, void* stream);

/*
 * Three-pass softmax through HBM (max -> exp & sum -> divide).
 * Replaces nkilab/kernels/norm.py:22 (softmax_unfused), nkilab/ops.py:56-57
 * with fused=False.  The fp32 intermediates live in `workspace`
 * (nkl_softmax_unfused_workspace_bytes(rows, cols) bytes, 256-byte aligned).
 */
size_t nkl_softmax_unfused_workspace_bytes(int rows, int cols);
int nkl_softmax_unfused(const void* x, void* y, void* workspace,
                        size_t workspace_bytes, int rows, int cols, long ldx,
                        long ldy, int dtype, void* stream);

/*
 * y = x * rsqrt(mean(x^2) + eps) * w.
 * Replaces nkilab/kernels/norm.py:92 (rmsnorm_fused), nkilab/ops.py:61.
 * x: [rows, cols] (ldx, dtype_in); w: [cols] (dtype_in); y: (ldy, dtype_out).
 * dtype_out in {dtype_in, BF16, F16 (dtype_in F32 only)}: an fp32 residual
 * stream can be normalised straight into a 16-bit GEMM operand.
 */
int nkl_rmsnorm(const void* x, const void* w, void* y, int rows, int cols,
                long ldx, long ldy, float eps, int dtype_in, int dtype_out,
                void* stream);

/*
 * The same RMSNorm with the weight in its own dtype (dtype_w in {F32, BF16},
 * independent of dtype_in): the fp32 normalised row is multiplied by the
 * weight as stored, then rounded once, as nkilab/kernels/norm.py:116 does
 * with the weight tile it loads.  nkl_rmsnorm is this call with
 * dtype_w = dtype_in.  Same reference lines as nkl_rmsnorm.
 */
int nkl_rmsnorm_ex(const void* x, const void* w, void* y, int rows, int cols,
                   long ldx, long ldy, float eps, int dtype_in, int dtype_w,
                   int dtype_out, void* stream);

/*
 * y = silu(g) * u, element-wise over n contiguous elements (fp32, bf16 or
 * fp16; silu and the product in fp32, one rounding).
 * Replaces nkilab/kernels/norm.py:121 (swiglu_fused), nkilab/ops.py:65.
 */
int nkl_swiglu(const void* g, const void* u, void* y, long n, int dtype,
               void* stream);

/*
 * hi/lo split of an fp32 matrix into bf16: y[r, c] = bf16(x[r, c]) and
 * y[r, cols + c] = bf16(x[r, c] - y[r, c]) (round-to-nearest-even), so that
 * hi + lo carries x to 16 significand bits.  A bf16 GEMM over y (K = 2 cols)
 * against a weight stacked twice along K accumulates x . w in fp32 to about
 * 2^-17 relative: the decoder block's fp32-accurate projections on bf16 MFMA.
 * No counterpart in the reference (nkilab/model.py:70-89 runs its block in
 * one dtype).  x: [rows, cols] fp32 (ldx), y: [rows, 2 cols] bf16 (ldy);
 * cols, ldx, ldy multiples of 4; x 16-byte, y 8-byte aligned.
 */
int nkl_split_bf16(const void* x, void* y, int rows, int cols, long ldx,
                   long ldy, void* stream);

/*
 * y = x over nbytes (a multiple of 16; both pointers 16-byte aligned): 16-byte
 * loads (2 in flight per lane, the fastest count on MI355X) and non-temporal
 * stores, the row kernels' loads and stores with none of their arithmetic.
 * A 16-byte call launches one workgroup: the launch cost alone.  No counterpart in the
 * reference: a measurement entry point that gives the HBM ceiling the row
 * kernels' roofline is read against, at their size and in the same run.
 */
int nkl_stream_copy(const void* x, void* y, long nbytes, void* stream);

/*
 * Causal attention O = softmax(Q K^T * scale + causal mask) V, flash style:
 * online softmax over key tiles, key tiles wholly above the diagonal are
 * skipped, the diagonal tiles are masked (key > query).
 * Replaces nkilab/kernels/attention.py:280 (flash_attention_pipelined, the
 * default of nkilab/ops.py:77) and its numerically identical siblings
 * attention.py:155, :179, :249; called from nkilab/ops.py:90.
 * q, k, v, o: [H, S, d] with element strides (*_sh between heads, at most
 * 2^24; *_ss between positions, at most 2^21) and unit stride along d; any
 * S >= 1, 1 <= d <= 128.
 * bf16: P is rounded to bf16 before P.V, statistics and O accumulate in fp32,
 * O is rounded once.  f16: the same with fp16 operands, P and O (the teams,
 * key-split or one-pass kernel).  f32: everything in fp32.
 */
int nkl_flash_attn_causal(const void* q, const void* k, const void* v,
                          void* o, int H, int S, int d, long q_sh, long q_ss,
                          long k_sh, long k_ss, long v_sh, long v_ss,
                          long o_sh, long o_ss, float scale, int dtype,
                          void* stream);

/*
 * The same causal attention with caller-provided scratch, which lets the bf16
 * kernel balance the causal triangle over every CU: query blocks may be split
 * across workgroups and finished by the last one to arrive.
 *   workspace: partial (max, sum, output) states of split blocks,
 *     nkl_flash_attn_causal_workspace_bytes() bytes, no initialisation.
 *   counters: one arrival counter per query block,
 *     nkl_flash_attn_causal_counter_bytes() bytes.  They must be zero before
 *     the first call; every call leaves them zero, so one zeroed array (of
 *     the largest size needed) can serve successive calls of any shape on
 *     one stream.  Calls that may overlap need separate arrays.
 * Both sizes are 0 exactly when the schedule chosen for the shape is not the
 * balanced one: f32, and the largest bf16 shapes (about 1024 key tiles of
 * 128 queries per CU and up, e.g. 32 x 16384 on 256 CUs), which run as
 * nkl_flash_attn_causal does and ignore the scratch.  Most shapes, including
 * ones with more query blocks than CUs (16 x 2048), need it: query the two
 * sizes for every shape rather than predicting them.  Same reference lines
 * as nkl_flash_attn_causal.
 */
size_t nkl_flash_attn_causal_workspace_bytes(int H, int S, int d, int dtype);
size_t nkl_flash_attn_causal_counter_bytes(int H, int S, int dtype);
int nkl_flash_attn_causal_ws(const void* q, const void* k, const void* v,
                             void* o, void* workspace, size_t workspace_bytes,
                             int* counters, size_t counter_bytes, int H, int S,
                             int d, long q_sh, long q_ss, long k_sh, long k_ss,
                             long v_sh, long v_ss, long o_sh, long o_ss,
                             float scale, int dtype, void* stream);

/*
 * Process-wide choice of the bf16 causal-attention kernel and schedule, for
 * tests and tuning (no counterpart in the reference).  Each argument is -1
 * for the automatic choice, or:
 *   kernel:   0 teams, 1 one wavefront per SIMD (32 queries), 2 (64 queries,
 *             2 wavefronts), 3 (64 queries, 4 wavefronts), 4 4-wavefront
 *             teams, 5 one-wavefront kernel at two per SIMD, 6 the
 *             64-key-tile kernel, 7 the same with its two key-half
 *             wavefronts half an iteration apart, 8 the key-split kernel
 *             (64-query blocks, four wavefronts that each take every
 *             fourth key tile), 9 the one-pass kernel for short sequences
 *             (S <= 256: one workgroup per 128-query block with every key
 *             row staged in LDS at once; the default up to S = 224, and
 *             up to 256 for launches of fewer than 12 units of 128 queries
 *             x 32 keys per CU); kernels
 *             6-9 for 64 < d <= 128 only, others fall back to kernel 0;
 *   schedule: 0 block, 1 balanced (needs the scratch of
 *             nkl_flash_attn_causal_ws), 2 pairs;
 *   qb:       64 or 128 queries per block (kernels 0 and 4);
 *   cpb:      balanced schedule, cost charged per block start, 0..4096.
 * Without a call the choice is read once from NKL_FLASH_KERNEL,
 * NKL_FLASH_SCHEDULE, NKL_FLASH_QB and NKL_FLASH_CPB.  The workspace sizes
 * follow the configuration in force when they are queried; do not change it
 * while another thread sizes or launches attention.
 */
int nkl_flash_attn_configure(int kernel, int schedule, int qb, int cpb);

/*
 * Test and tuning control, process-wide, of the balanced schedule: the poll
 * budget (0 .. 2^20; -1 for the automatic choice: 256, or 0 when the longest
 * block spans six or more ranges) of the workgroup that merges a split query
 * block while it waits for the block's other parts (the 128-query teams
 * kernel folds each part as it arrives).  Past the budget it stores its own
 * state (or what it has folded so far) and arrives like the others, and the
 * last to arrive merges the rest; the parts are folded in the same order
 * either way, so every budget gives the same bits.  No counterpart in the reference (its kernels
 * have no split blocks).
 */
int nkl_flash_attn_configure_polls(int polls);

/*
 * Test hook, host only (no GPU work): checks the work split the 16-bit
 * attention kernels would walk for an H x S x d call (dtype NKL_BF16 or
 * NKL_F16) under the configuration in force.  Balanced ranges tile the
 * units in order and none is empty; walking each range from its last
 * segment to its first, as the kernels do, covers it exactly; every split
 * block's parts are the ranges that hold its units and its last range is
 * the one that merges; no range puts two parts in one of its two partial-
 * state slots; the pairs and block schedules take every block whole, once.
 * Returns NKL_OK, NKL_EDTYPE for other dtypes, or NKL_EINVAL naming the
 * first violated invariant (or a shape outside d <= 128).  info
 * (NULL or 5 longs): workgroups, units, split blocks, most parts of a block,
 * and the merging workgroup's poll budget (-1 without the balanced schedule).
 * No counterpart in the reference (its kernels have no work split).
 */
int nkl_flash_attn_plan_check(int H, int S, int d, int dtype, long* info);

/*
 * Unfused causal attention: scores (fp32, [H, S, S]) and probabilities
 * ([H, S, S], dtype) are materialised in `workspace`, then O = P V.
 * Replaces nkilab/kernels/attention.py:35 (attention_naive), selected by
 * variant "naive" at nkilab/ops.py:68-74.
 */
size_t nkl_attention_naive_workspace_bytes(int H, int S, int dtype);
int nkl_attention_naive(const void* q, const void* k, const void* v, void* o,
                        void* workspace, size_t workspace_bytes, int H, int S,
                        int d, long q_sh, long q_ss, long k_sh, long k_ss,
                        long v_sh, long v_ss, long o_sh, long o_ss,
                        float scale, int dtype, void* stream);

/*
 * Grouped-query (and multi-query) forms of the two entry points above: q and
 * o have H heads, k and v have Hkv heads (H a multiple of Hkv), and query
 * head h attends with K/V head h / (H / Hkv).  No counterpart in the
 * reference, whose README lists GQA/MQA among the features it does not
 * implement (README.md:89); with Hkv == H they equal nkl_flash_attn_causal_ws
 * and nkl_attention_naive.  Scratch sizes are those of the H-head call.
 */
int nkl_flash_attn_causal_gqa(const void* q, const void* k, const void* v,
                              void* o, void* workspace, size_t workspace_bytes,
                              int* counters, size_t counter_bytes, int H,
                              int Hkv, int S, int d, long q_sh, long q_ss,
                              long k_sh, long k_ss, long v_sh, long v_ss,
                              long o_sh, long o_ss, float scale, int dtype,
                              void* stream);
int nkl_attention_naive_gqa(const void* q, const void* k, const void* v,
                            void* o, void* workspace, size_t workspace_bytes,
                            int H, int Hkv, int S, int d, long q_sh, long q_ss,
                            long k_sh, long k_ss, long v_sh, long v_ss,
                            long o_sh, long o_ss, float scale, int dtype,
                            void* stream);

/*
 * nkl_flash_attn_causal_gqa without the scratch arguments, for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  No counterpart in the reference.
 * The partial states and arrival counters live in a static device array of
 * 64 MiB + 1 MiB that each GPU holds from its first call until the process
 * ends; a shape whose nkl_flash_attn_causal_workspace_bytes() exceeds 64 MiB
 * (or whose counters, 4 H ceil(S / 64) bytes, exceed 1 MiB) is rejected with
 * NKL_EWORKSPACE.  The call allocates nothing and clears the counters with a
 * kernel (no memset node), so it may be captured; make the first call on each
 * device outside capture (it looks the array's address up).  Every call on a
 * GPU shares that GPU's array: calls that may overlap on one GPU (other
 * streams, other threads) race and must be serialised by the caller.
 */
int nkl_flash_attn_causal_noalloc(const void* q, const void* k, const void* v,
                                  void* o, int H, int Hkv, int S, int d,
                                  long q_sh, long q_ss, long k_sh, long k_ss,
                                  long v_sh, long v_ss, long o_sh, long o_ss,
                                  float scale, int dtype, void* stream);

/*
 * Rotary position embedding, rotate-half layout (RoFormer, as GPT-NeoX and
 * Llama apply it): for each head h and row s of x [H, S, d] (strides x_sh,
 * x_ss; d even), element i < d/2 and element i + d/2 rotate by the angle
 * (pos0 + s) * base^(-2 i / d).  fp32, bf16 or fp16 x and y; fp32
 * arithmetic, one rounding per output;
 * y may be x (in place).  No counterpart in the reference (README.md:89 lists
 * rotary embeddings as not implemented); applied to q and k before attention.
 */
int nkl_rope(const void* x, void* y, int H, int S, int d, long x_sh, long x_ss,
             long y_sh, long y_ss, int pos0, float base, int dtype,
             void* stream);

#ifdef __cplusplus
}
#endif

#endif /* NKILAB_HIP_H */
