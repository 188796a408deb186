/*
 * dfmi -- MI355X (gfx950) kernels for the dflash-mlx target-verify hot path.
 *
 * C ABI of libdfmi.so.  Plain pointers and sizes only: every pointer argument
 * marked "device" is HIP device memory; `stream` is a hipStream_t (NULL = the
 * null stream).  All launches are stream-ordered and asynchronous; a return of
 * DFMI_OK means the work was enqueued.  No function allocates or frees device
 * memory and none keeps a pointer past its return (dfmi_qmm_prepare writes
 * the pointers it is given into the caller's record buffer, which
 * dfmi_qmm_run then reads).  Functions are reentrant;
 * the process state is the thread-local error string and, for
 * dfmi_qmm_affine_noalloc only, its static device scratch array and the
 * per-device address of it (set once, under a lock).
 *
 * Packed-weight layout (the bytes dflash-mlx and MLX hand to the kernels,
 * dflash_mlx/verify_qmm.py:97-115): w_q uint32 [N, K*bits/32] row-major,
 * word j of row n holding k = j*(32/bits) .. , the first k in the lowest
 * bits; scales and biases [N, K/group_size] in the activation dtype.
 * Dequantised weight: w[n,k] = q[n,k]*scales[n,k/gs] + biases[n,k/gs].
 *
 * Workspaces: functions taking (workspace, workspace_bytes) need a device
 * buffer of at least the size their *_workspace_bytes query returns.  The
 * buffer must be zero-filled once when it is created; the kernels leave every
 * counter and key they use back at zero when they finish, so one workspace
 * serves any sequence of calls on ONE stream.  Calls that overlap in time
 * (different streams) must not share a workspace.
 */
#ifndef DFMI_H
#define DFMI_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes. */
#define DFMI_OK 0
#define DFMI_EINVAL (-1)   /* unsupported shape / dtype / alignment: caller falls back */
#define DFMI_ELAUNCH (-2)  /* HIP launch error */
#define DFMI_ENOSPC (-3)   /* workspace too small */

/* Activation / scale dtypes. */
#define DFMI_BF16 0
#define DFMI_F16 1
#define DFMI_F32 2

/* Library version string and the message of the last failed call on this thread. */
const char *dfmi_version(void);
const char *dfmi_last_error(void);

/* Optional launch-shape override for the affine qmm (tuning sweeps).  Zero
 * fields mean "automatic".
 *   path: 1 = general kernel, 2 = streaming kernel (DFMI_EINVAL if the shape
 *         is outside it: M <= 32, K % 256 == 0, K % (8*group_size) == 0;
 *         checked for both weight widths); any other value is DFMI_EINVAL;
 *   tiles_per_wave: general kernel, 16-row weight tiles per wavefront (1, 2,
 *         4); the streaming kernel always covers 64 rows per workgroup;
 *   waves_per_block: general kernel, wavefronts of a workgroup that split K
 *         (1..8; the reference's K_PARTS); streaming kernel, 4 or 8
 *         wavefronts (8 needs M <= 16 and K % 512 == 0);
 *   k_splits: streaming kernel, workgroups that split K of one output block
 *         (raised if a split's K range would exceed one scale / bias window
 *         of 120 groups);
 *   rows_per_block: streaming kernel, 64 or 128 weight rows per workgroup
 *         (128: the pair-streaming plan of 4-bit gs 64 / 128 shapes with
 *         M <= 16 and N a multiple of 128, waves_per_block 0; DFMI_EINVAL
 *         otherwise); 0 automatic. */
typedef struct dfmi_qmm_tuning {
  int path;
  int tiles_per_wave;
  int waves_per_block;
  int k_splits;
  int rows_per_block;
} dfmi_qmm_tuning;

/*
 * y[M, N] = x[M, K] . dequant(W)^T  (affine, transpose=True).
 *
 * Replaces the reference's M=16 / M=4 verify kernels AND the stock
 * mx.quantized_matmul they fall back to:
 *   dflash_mlx/verify_qmm.py:905-1022  verify_matmul (combo_ktmpl,
 *     super_tree_fp16_ktmpl, mma2big, mma2big_pipe, m4_ksplit_np launches at
 *     941-949, 961-973, 982-1002, 1009-1022)
 *   dflash_mlx/verify_linear.py:166-175, 190-211, 223-232  per-module _run
 *   mx.quantized_matmul(x, w, scales, biases, transpose=True, group_size, bits)
 *     (verify_qmm.py:915-919 and every fallback site)
 * x, scales, biases: dtype x_dtype (DFMI_BF16 or DFMI_F16); y: same dtype.
 * Supported: bits 4 or 8 (8-bit: w_q [N, K/4], byte i of word j = k 4j+i,
 * the reference's mma2big_8bit layout, verify_qmm.py:549-650, 767-884),
 * group_size in {32, 64, 128}, K % 32 == 0, K % group_size == 0, any M >= 1,
 * any N >= 1; 16-byte aligned x / w_q / scales / biases.  fp32 accumulation,
 * output rounded to nearest even.
 * Anything else returns DFMI_EINVAL without launching.  Results do not depend
 * on scheduling: every K split is summed in a fixed order.  Shapes that split
 * K across workgroups need the workspace dfmi_qmm_workspace_bytes reports
 * (0 bytes -> workspace may be NULL); it must be zero-filled when created.
 */
int dfmi_qmm_affine(const void *x, int x_dtype, const uint32_t *w_q, const void *scales,
                    const void *biases, void *y, int64_t M, int64_t K, int64_t N,
                    int group_size, int bits, void *workspace, size_t workspace_bytes,
                    void *stream);
int dfmi_qmm_affine_ex(const void *x, int x_dtype, const uint32_t *w_q, const void *scales,
                       const void *biases, void *y, int64_t M, int64_t K, int64_t N,
                       int group_size, int bits, void *workspace, size_t workspace_bytes,
                       const dfmi_qmm_tuning *tuning, void *stream);
size_t dfmi_qmm_workspace_bytes(int64_t M, int64_t K, int64_t N, int group_size, int bits);

/*
 * The whole stock quantized matmul: mx.quantized_matmul, which dflash-mlx
 * calls for every input its verify kernels decline (verify_qmm.py:915-919,
 * 936-938, 957-959, 984-986, 1005-1007), for 4- and 8-bit affine weights at
 * group size 32 / 64 / 128:
 *   transpose != 0: y[M, N] = x[M, K] . dequant(w)^T, w_q [N, K*bits/32]
 *     (16-byte aligned), scales / biases [N, K/gs]; K % gs == 0;
 *   transpose == 0: y[M, N] = x[M, K] . dequant(w), w_q [K, N*bits/32]
 *     quantised along N, scales / biases [K, N/gs]; N % gs == 0, any K >= 1.
 * x_dtype and s_dtype (scales and biases) are DFMI_BF16, DFMI_F16 or
 * DFMI_F32; y has their common dtype when they are the same, else float32
 * (MLX's promotion).  transpose with x and scales of one 16-bit dtype is
 * dfmi_qmm_affine_ex (same kernels and results; workspace as
 * dfmi_qmm_workspace_bytes reports); every other case runs fp32 VALU
 * kernels, needs no workspace (NULL, 0) and is deterministic.
 */
int dfmi_qmm_general(const void *x, int x_dtype, const uint32_t *w_q, const void *scales,
                     const void *biases, int s_dtype, void *y, int64_t M, int64_t K, int64_t N,
                     int group_size, int bits, int transpose, void *workspace,
                     size_t workspace_bytes, void *stream);

/*
 * dfmi_qmm_affine_ex with the layer's pair table as well: sb_pairs
 * [K/group_size][N] uint32, pair[g][n] = scales[n][g] | biases[n][g] << 16
 * (built once per weight by dfmi_sb_pairs; 16-byte aligned).  Same call
 * sites replaced as dfmi_qmm_affine (verify_qmm.py:905-1022,
 * verify_linear.py:166-175, 190-211, 223-232); the reference's
 * VerifyQuantizedLinear likewise precomputes per-module launch state
 * (verify_linear.py:118-223).  With the table, 4-bit gs 64 / 128 calls with
 * M <= 32 and whole 256-k steps stream the pairs with every step instead of
 * holding a scale / bias window in LDS, so three workgroups share a CU.  The
 * launch plan does not depend on sb_pairs: the result is bit-identical to
 * dfmi_qmm_affine_ex (tuning included) on the same inputs; sb_pairs may be
 * NULL.
 */
int dfmi_qmm_affine_pairs(const void *x, int x_dtype, const uint32_t *w_q, const void *scales,
                          const void *biases, const uint32_t *sb_pairs, void *y, int64_t M,
                          int64_t K, int64_t N, int group_size, int bits, void *workspace,
                          size_t workspace_bytes, const dfmi_qmm_tuning *tuning, void *stream);
/*
 * Pair table for dfmi_qmm_affine_pairs / dfmi_qmm_affine_multi: from scales
 * and biases [N, groups] (dtype DFMI_BF16 or DFMI_F16, the layer's 16-bit
 * values) to sb_pairs [groups][N] uint32 (scale in the low half, bias in the
 * high half), on `stream`.  No reference counterpart: a one-time re-layout of
 * a loaded layer's scales (the reference reads them in place).
 */
int dfmi_sb_pairs(const void *scales, const void *biases, int dtype, int64_t N, int64_t groups,
                  uint32_t *sb_pairs, void *stream);
/* Host-only plan query (no reference counterpart; for tests, benchmarks
 * and profiles): the streaming launch dfmi_qmm_affine_ex (nseg = 1, Ns[0] =
 * N, tuning as given) or dfmi_qmm_affine_multi (nseg 2..4, tuning NULL)
 * makes for this shape.  streaming = 0 when another kernel runs (the other
 * fields are then 0).  blocks: 64-row blocks of the grid; whole_blocks: the
 * first blocks run unsplit, the rest are split k_splits ways; workgroups:
 * the grid; pair_streaming: the plan runs on the pair-streaming kernel when
 * pair tables are given; rows_per_block: 64 or 128 (a 128-row plan runs as
 * its 64-row equivalent, same results, when the pair tables are missing). */
typedef struct dfmi_qmm_plan_info {
  int streaming;
  int waves;
  int k_splits;
  int whole_blocks;
  int blocks;
  int workgroups;
  int pair_streaming;
  int rows_per_block;
} dfmi_qmm_plan_info;
int dfmi_qmm_plan(int64_t M, int64_t K, const int64_t *Ns, int nseg, int group_size, int bits,
                  const dfmi_qmm_tuning *tuning, dfmi_qmm_plan_info *out);
/* Host-only plan query (no reference counterpart; for benchmarks and
 * profiles): name of the kernel dfmi_qmm_affine_ex would launch for this
 * shape, "qmm_stream_kernel", "qmm_dense_kernel" or
 * (bits 8) "qmm8_stream_kernel" / "qmm8_kernel";
 * NULL if unsupported. */
const char *dfmi_qmm_kernel_name(int64_t M, int64_t K, int64_t N, int group_size, int bits,
                                 const dfmi_qmm_tuning *tuning);
size_t dfmi_qmm_workspace_bytes_ex(int64_t M, int64_t K, int64_t N, int group_size, int bits,
                                   const dfmi_qmm_tuning *tuning);

/*
 * dfmi_qmm_affine that allocates nothing and takes no workspace.  No
 * counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  The split-K workspace (block counters, then fp32
 * partials) lives in a static device array of dfmi_qmm_noalloc_scratch_bytes()
 * bytes (64 KiB + 8 MiB) that every GPU the library runs on holds until the
 * process ends.  The automatic plan of the shape must fit it, else
 * DFMI_ENOSPC (nothing launched); the same plan and kernels as
 * dfmi_qmm_affine, so the result is bit-identical to it.  The first call on a
 * device clears the array's counters with a kernel on `stream`.  All calls on
 * one GPU share the array: calls that overlap in time on one GPU (different
 * streams, or host threads) race on it and must be serialised by the caller.
 */
int dfmi_qmm_affine_noalloc(const void *x, int x_dtype, const uint32_t *w_q, const void *scales,
                            const void *biases, void *y, int64_t M, int64_t K, int64_t N,
                            int group_size, int bits, void *stream);
size_t dfmi_qmm_noalloc_scratch_bytes(void);

/*
 * Several matmuls that share their activations, in one launch:
 *   y_i[M, N_i] = x[M, K] . dequant(W_i)^T,  i < nseg (1..4),
 * each W_i in the same packed layout as dfmi_qmm_affine (w_q [N_i, K*bits/32],
 * scales / biases [N_i, K/group_size], 16-byte aligned; y_i [M, N_i]).
 *
 * No reference counterpart as one call: it replaces the separate per-module
 * verify_matmul launches of sibling projections that read the same input in
 * the reference's verify forward -- q/k/v of an attention block, gate/up of
 * an MLP (dflash_mlx/verify_linear.py:266-286, one call per
 * VerifyQuantizedLinear) -- so that the layer pays one launch, one pipeline
 * fill and one grid for them: the row blocks of all W_i form one streaming
 * grid.  Shapes outside the streaming kernel (M > 32, K % 256 != 0, ...) run
 * as nseg dfmi_qmm_affine calls on the stream, in order.  Each y_i is within
 * fp32 summation order of what dfmi_qmm_affine returns for W_i alone (the two
 * may split K differently); the result does not depend on scheduling.  The
 * workspace is dfmi_qmm_multi_workspace_bytes bytes, zero-filled when
 * created.
 */
typedef struct dfmi_qmm_segment {
  const uint32_t *w_q;
  const void *scales;
  const void *biases;
  void *y;
  int64_t N;
  const uint32_t *sb_pairs; /* pair table (see dfmi_qmm_affine_pairs) or NULL */
} dfmi_qmm_segment;
int dfmi_qmm_affine_multi(const void *x, int x_dtype, const dfmi_qmm_segment *segs, int nseg,
                          int64_t M, int64_t K, int group_size, int bits, void *workspace,
                          size_t workspace_bytes, void *stream);
/*
 * dfmi_qmm_affine_multi for two or three matrices whose pair tables are
 * given side by side: sb_pairs [K/group_size][N_0 + N_1 (+ N_2)] uint32, the
 * matrices' dfmi_sb_pairs tables concatenated along the columns (built once
 * per sibling group; 16-byte aligned).  The segments' own sb_pairs are used
 * only where the launch cannot take the combined table (another count of
 * matrices, an N of 2^16 or more, a plan without pair streaming).  Same call
 * sites and the same sums as dfmi_qmm_affine_multi (bit-identical y_i); the
 * kernel then finds every value its first loads need in the arguments the
 * hardware preloads into registers, instead of reading a segment table
 * first.
 */
int dfmi_qmm_affine_multi_fused(const void *x, int x_dtype, const dfmi_qmm_segment *segs,
                                int nseg, const uint32_t *sb_pairs, int64_t M, int64_t K,
                                int group_size, int bits, void *workspace,
                                size_t workspace_bytes, void *stream);
size_t dfmi_qmm_multi_workspace_bytes(int64_t M, int64_t K, const int64_t *Ns, int nseg,
                                      int group_size, int bits);

/*
 * Prepared launches of a verify linear: the reference's VerifyQuantizedLinear
 * computes its route once per module in _build_dispatch and its per-call
 * closure only launches (dflash_mlx/verify_linear.py:118-309, calls at
 * 266-286); dfmi_qmm_prepare likewise plans one call shape -- one matrix
 * (dfmi_qmm_affine_pairs) or 2..4 sibling matrices sharing x
 * (dfmi_qmm_affine_multi / _multi_fused) -- into the caller's record
 * buffer, and dfmi_qmm_run launches it on new activations and outputs.
 * Same kernels, plans and results as those entry points (bit-identical).
 *   segs: the matrices (their y fields are ignored); fused_pairs: for nseg
 *     >= 2, their pair tables side by side, or NULL;
 *   sb_stride: the row length (in pairs) of the table that every
 *     segment's sb_pairs points into when each is its matrix's column slice
 *     of one wider table (a sibling group's combined table: sb_pairs =
 *     column 0 of the slice, 16-byte aligned; sb_stride and every N a
 *     multiple of 4; fused_pairs NULL), else 0;
 *   workspace: as the matching one-shot entry point needs
 *     (dfmi_qmm_workspace_bytes_ex / dfmi_qmm_multi_workspace_bytes).
 * The record (DFMI_QMM_RECORD_BYTES bytes, 16-byte aligned, caller-owned
 * host memory) keeps the weight, table and workspace pointers: they must
 * stay valid while the record is used, and calls that run a record (or use
 * its workspace) concurrently on different streams race.
 * dfmi_qmm_run: y0..y3 are the outputs of segments 0..nseg-1 ([M, N_i],
 * x's dtype; unused ones NULL); x 16-byte aligned [M, K].
 */
#define DFMI_QMM_RECORD_BYTES 1024
int dfmi_qmm_prepare(int x_dtype, const dfmi_qmm_segment *segs, int nseg,
                     const uint32_t *fused_pairs, int64_t sb_stride, int64_t M, int64_t K,
                     int group_size, int bits, void *workspace, size_t workspace_bytes,
                     void *record, size_t record_bytes);
int dfmi_qmm_run(const void *record, const void *x, void *y0, void *y1, void *y2, void *y3,
                 void *stream);
/* Host-only plan query (no reference counterpart; for benchmarks and
 * profiles): the kernel of the single launch dfmi_qmm_affine_multi makes,
 * "qmm_stream_multi_kernel" (nseg >= 2) or "qmm_stream_kernel"; NULL when it
 * makes one dfmi_qmm_affine call per matrix instead (or the shape is
 * invalid). */
const char *dfmi_qmm_multi_kernel_name(int64_t M, int64_t K, const int64_t *Ns, int nseg,
                                       int group_size, int bits);

/*
 * Routed-expert matmul: for each pair p < P,
 *   y[p, N] = x[lhs_rows[p], K] . dequant(W[rhs_experts[p]])^T
 * with w_q [E, N, K*bits/32], scales / biases [E, N, K/gs].
 * Replaces mx.gather_qmm(x, w, scales, biases, rhs_indices=..., transpose=True,
 * group_size, bits, sorted_indices=...) as called by mlx-lm's
 * QuantizedSwitchLinear (reached from dflash_mlx/engine/target_qwen_gdn.py:865,874),
 * with the lhs broadcast resolved to explicit row ids.  lhs_rows may be NULL
 * (row p for pair p).  Pair order is free (sorted or not); results are
 * per pair.  Expert ids outside [0, E) and row ids outside [0, x_rows) are
 * checked on the device: that pair's output row is filled with NaN (the call
 * still returns DFMI_OK; validate on the host when it matters).  P <= 65535.
 * P == 0 (or N == 0) is a no-op, and then x_rows may be 0.
 */
int dfmi_gather_qmm_affine(const void *x, int x_dtype, int64_t x_rows, const uint32_t *w_q,
                           const void *scales, const void *biases, const int32_t *lhs_rows,
                           const int32_t *rhs_experts, void *y, int64_t P, int64_t K, int64_t N,
                           int64_t E, int group_size, int bits, void *stream);

/*
 * SwitchGLU front half, fused: for each pair p,
 *   h[p, N] = silu(gate_p) * up_p,  gate_p = rnd(x_p . dequant(Wg[e])^T),
 *   up_p = rnd(x_p . dequant(Wu[e])^T)   (rnd = round to x_dtype)
 * i.e. mlx-lm SwitchGLU's gate_proj / up_proj gather_qmm pair plus its
 * SwiGLU activation, one weight pass.  Same index conventions as above.
 */
int dfmi_gather_qmm_swiglu(const void *x, int x_dtype, int64_t x_rows,
                           const uint32_t *wg_q, const void *g_scales, const void *g_biases,
                           const uint32_t *wu_q, const void *u_scales, const void *u_biases,
                           const int32_t *lhs_rows, const int32_t *rhs_experts, void *h,
                           int64_t P, int64_t K, int64_t N, int64_t E, int group_size, int bits,
                           void *stream);

/*
 * The two gathers above with the experts' (scale, bias) pair table
 * (dfmi_moe_pairs): the same results within the gathers' tolerance, from a
 * main loop that streams the pairs per 256-k step (128-row work units, two
 * workgroups per CU).  Taken when sb_pairs != NULL (16-byte aligned), gs is
 * 64 or 128, K % 256 == 0, N % 128 == 0 (affine) or N % 64 == 0 (SwiGLU),
 * P <= 256, x_rows <= 32767 and E < 65535; otherwise the call is exactly the
 * plain entry point's.  Same call sites as dfmi_gather_qmm_affine /
 * dfmi_gather_qmm_swiglu (mlx-lm QuantizedSwitchLinear / SwitchGLU, reached
 * from dflash_mlx/engine/target_qwen_gdn.py:865,874), with the per-layer
 * table built once, as the reference's VerifyQuantizedLinear precomputes
 * per-module state (dflash_mlx/verify_linear.py:118-223).
 * workspace (16-byte aligned, dfmi_gather_workspace_bytes() bytes: 4 KiB
 * of counters, zero when first used and left zero by every call, then the
 * pieces' fp32 partials, which need no clearing) lets the units of the last
 * partial round split along K; NULL runs them whole.  Calls that overlap
 * on one workspace race.
 */
int dfmi_gather_qmm_affine_pairs(const void *x, int x_dtype, int64_t x_rows,
                                 const uint32_t *w_q, const void *scales, const void *biases,
                                 const uint32_t *sb_pairs, const int32_t *lhs_rows,
                                 const int32_t *rhs_experts, void *y, int64_t P, int64_t K,
                                 int64_t N, int64_t E, int group_size, int bits,
                                 void *workspace, size_t workspace_bytes, void *stream);
int dfmi_gather_qmm_swiglu_pairs(const void *x, int x_dtype, int64_t x_rows,
                                 const uint32_t *wg_q, const void *g_scales,
                                 const void *g_biases, const uint32_t *wu_q,
                                 const void *u_scales, const void *u_biases,
                                 const uint32_t *sb_pairs, const int32_t *lhs_rows,
                                 const int32_t *rhs_experts, void *h, int64_t P, int64_t K,
                                 int64_t N, int64_t E, int group_size, int bits,
                                 void *workspace, size_t workspace_bytes, void *stream);
size_t dfmi_gather_workspace_bytes(void);

/*
 * Pair table of routed experts for the *_pairs gathers: from scales / biases
 * [E, N, groups] (16-bit, dtype DFMI_BF16 or DFMI_F16), sb_pairs
 * [E][groups][N] uint32 = scale | bias << 16.  With up_scales / up_biases
 * (the SwiGLU's up projection; N a multiple of 32) the table is
 * [E][groups][2N], gate and up interleaved 32 columns at a time: column
 * 64 (n / 32) + 32 u + n % 32 holds row n of the gate (u = 0) or up (u = 1)
 * set.  Asynchronous on `stream`.
 */
int dfmi_moe_pairs(const void *scales, const void *biases, const void *up_scales,
                   const void *up_biases, int dtype, int64_t E, int64_t N, int64_t groups,
                   uint32_t *sb_pairs, void *stream);

/*
 * Weighted sum over each token's top-k expert outputs (the Qwen MoE block's
 * `(y * scores[..., None]).sum(axis=-2)`, reached from
 * dflash_mlx/engine/target_qwen_gdn.py:865,874), with the unsort mlx-lm's
 * SwitchGLU applies to expert-sorted outputs folded in:
 *   out[t, D] = rnd(sum_j scores[t, j] * y[r(t*k + j), D])   (fp32 accumulate)
 * r(p) = y_rows[p] when y_rows != NULL (y in expert-sorted pair order,
 * y_rows = the inverse of the sort permutation), else p.  A row id outside
 * [0, T*k) gives NaN outputs for that token.  y and out in y_dtype; scores
 * fp32 [T, k].
 */
int dfmi_moe_combine(const void *y, int y_dtype, const int32_t *y_rows, const float *scores,
                     void *out, int64_t T, int64_t k, int64_t D, void *stream);

/*
 * Greedy verify over given logits: posterior[m] = argmax_v masked(logits[m, v])
 * with masked ids set to dtype(-1e9) (dflash_mlx/engine/sampling.py:48-55),
 * lowest index on ties, NaN never selected unless the row is all NaN.
 * When verify_ids != NULL (M >= 1):
 *   accept_len[0] = match_acceptance_length(verify_ids[1:], posterior[:-1])
 *     (dflash_mlx/engine/acceptance.py:9-16, engine/spec_epoch.py:2070-2072)
 *   bonus[0] = posterior[accept_len]            (engine/spec_epoch.py:2129)
 * suppress_mask: uint8 [V] (nonzero = suppressed) or NULL.
 * logits dtype: DFMI_BF16, DFMI_F16 or DFMI_F32.
 */
int dfmi_greedy_accept(const void *logits, int logits_dtype, const uint8_t *suppress_mask,
                       const uint32_t *verify_ids, int64_t M, int64_t V, uint32_t *posterior,
                       int32_t *accept_len, uint32_t *bonus, void *workspace,
                       size_t workspace_bytes, void *stream);
size_t dfmi_greedy_workspace_bytes(int64_t M);

/*
 * Fused lm_head + greedy + accept: the logits rnd(h . dequant(W_lm)^T)
 * (optionally Gemma-softcapped: rnd(rnd(tanh(rnd(l / cap))) * cap), cap > 0)
 * are reduced to the per-row argmax inside the matmul epilogue and never
 * written unless logits_out != NULL.  Replaces the stock lm_head
 * (dflash_mlx/engine/target_qwen_gdn.py:774-778, engine/target_gemma4.py:336-355)
 * followed by greedy_tokens_with_mask and match_acceptance_length
 * (engine/spec_epoch.py:2067-2072, 2129).  Outputs as dfmi_greedy_accept.
 * M <= 32.
 */
int dfmi_lmhead_greedy_accept(const void *h, int h_dtype, const uint32_t *w_q, const void *scales,
                              const void *biases, const uint8_t *suppress_mask, float softcap,
                              const uint32_t *verify_ids, int64_t M, int64_t K, int64_t V,
                              int group_size, int bits, uint32_t *posterior, int32_t *accept_len,
                              uint32_t *bonus, void *logits_out, void *workspace,
                              size_t workspace_bytes, void *stream);
size_t dfmi_lmhead_workspace_bytes(int64_t M);
/*
 * dfmi_lmhead_greedy_accept with the lm_head's pair table (sb_pairs
 * [K/group_size][V], see dfmi_sb_pairs; 16-byte aligned; may be NULL): with
 * it, M <= 16, gs 64 / 128 and K / group_size <= 120 sweep the vocabulary in
 * 128-row blocks on the pair-streaming loop.  Same call sites replaced;
 * identical outputs (the same logits, summed in the same order) for every
 * shape, with or without the table.
 */
int dfmi_lmhead_greedy_accept_pairs(const void *h, int h_dtype, const uint32_t *w_q,
                                    const void *scales, const void *biases,
                                    const uint32_t *sb_pairs, const uint8_t *suppress_mask,
                                    float softcap, const uint32_t *verify_ids, int64_t M,
                                    int64_t K, int64_t V, int group_size, int bits,
                                    uint32_t *posterior, int32_t *accept_len, uint32_t *bonus,
                                    void *logits_out, void *workspace, size_t workspace_bytes,
                                    void *stream);

/*
 * Gated-delta recurrence recording the innovation tape, over T steps
 * (dflash_mlx/kernels.py:11-219 gated_delta_kernel_with_tape; called from
 * dflash_mlx/engine/target_qwen_gdn.py:615-625 while the rollback cache is
 * armed).  Per batch b, value head hv (key head hv / (Hv/Hk)), state row dv,
 * unmasked step t:  S *= g;  d = (v[dv] - S.k) * beta;  S += d k;
 * y[dv] = S.q;  tape[dv] = d  (masked steps: S kept, y = 0, tape = 0).
 *   q, k [B, T, Hk, Dk], v / y [B, T, Hv, Dv] in qkv_dtype;
 *   g [B, T, Hv] (g_per_key = 0) or [B, T, Hv, Dk] in g_dtype;
 *   beta [B, T, Hv] in beta_dtype; mask uint8 [B, T] (nonzero = live) or NULL;
 *   state_in / state_out [B, Hv, Dv, Dk] in state_dtype (may alias);
 *   tape [B, T, Hv, Dv] fp32.
 * The state is carried in fp32 across the steps.  Dk in {32, 64, 128, 256,
 * 512}, Hv a multiple of Hk, B*Hv <= 65535.
 */
int dfmi_gated_delta_tape(const void *q, const void *k, const void *v, const void *g,
                          const void *beta, const void *state_in, const uint8_t *mask, void *y,
                          void *state_out, float *tape, int64_t B, int64_t T, int64_t Hk,
                          int64_t Hv, int64_t Dk, int64_t Dv, int qkv_dtype, int g_dtype,
                          int beta_dtype, int state_dtype, int g_per_key, void *stream);

/*
 * Tape replay over the accepted steps (dflash_mlx/kernels.py:691-866
 * tape_replay_kernel; called by dflash_mlx/recurrent_rollback_cache.py:142-165
 * with the first accepted+1 steps): per unmasked step
 * S = round(S * g + tape[dv] * k) to state_dtype.
 *   tape fp32 [B, T, Hv, Dv]; k [B, T, Hk, Dk] in k_dtype; g as above;
 *   state_in / state_out [B, Hv, Dv, Dk] in state_dtype (may alias).
 */
int dfmi_tape_replay(const float *tape, const void *k, const void *g, const void *state_in,
                     const uint8_t *mask, void *state_out, int64_t B, int64_t T, int64_t Hk,
                     int64_t Hv, int64_t Dk, int64_t Dv, int k_dtype, int g_dtype,
                     int state_dtype, int g_per_key, void *stream);

/*
 * match_acceptance_length on device arrays (dflash_mlx/engine/acceptance.py:9-16):
 * out[0] = length of the longest prefix with drafted[i] == posterior[i]; 0 for L == 0.
 */
int dfmi_match_acceptance_length(const uint32_t *drafted, const uint32_t *posterior, int64_t L,
                                 int32_t *out, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* DFMI_H */
