/*
 * switchyard for MI355X -- C ABI of the Block AttnRes operator.
 *
 * One token (b, t) of the operator, with N sources v_0..v_{N-1} of width D and
 * a pseudo-query w:
 *
 *     r_n     = 1 / sqrt(mean_d(v_n[d]^2) + eps)
 *     logit_n = r_n * sum_d w[d] * v_n[d]          (no 1/sqrt(D) factor)
 *     alpha   = softmax_n(logit)                   (over the source axis)
 *     out[d]  = sum_n alpha_n * v_n[d]              (weighted sum of RAW sources)
 *
 * Layout (all element counts, not bytes):
 *   v        [N][n_tok][D]  row n of token t at v + n*src_stride + t*D
 *   out      [n_tok][D]     contiguous
 *   grad_out [n_tok][D]     contiguous, same dtype as v
 *   dv       [N][n_tok][D]  contiguous (source stride n_tok*D)
 *   w, dw    [D]
 *   queries  [S][D], batched out [S][n_tok][D]
 *   m, l     [n_tok] fp32 (batched: [S][n_tok]): max logit, sum of exp(logit - m)
 * The *_table entry points take the sources as a host array of N device
 * pointers instead, each source [n_tok][D] contiguous (dv likewise), so
 * separately allocated sources need no stacking copy.
 * n_tok is B*T: the batch and sequence axes are flattened because tokens are
 * independent.
 *
 * Conventions shared by every entry point:
 *   - Launches are asynchronous on `stream` (a hipStream_t; NULL = the null
 *     stream). Nothing synchronises the host.
 *   - The library never allocates device memory: the caller owns every buffer,
 *     including the backward workspace sized by sy_bwd_workspace_bytes().
 *   - Return value 0 = success; < 0 = an sy_status argument error detected
 *     before any device work; > 0 = the hipError_t the HIP runtime returned.
 *   - Entry points are reentrant; concurrent calls on different streams are
 *     safe as long as they do not share output or workspace buffers.
 */
#ifndef SWITCHYARD_H
#define SWITCHYARD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SY_ABI_VERSION 4

/* Most sources a per-source pointer list (the *_table entry points) may hold. */
#define SY_MAX_TABLE_ROWS 16

/* Element types. Reference: tensors may be bf16/fp16/fp32 and all arithmetic is
 * fp32 (src/switchyard/triton_op.py:36, :66-67). */
typedef enum sy_dtype { SY_F32 = 0, SY_F16 = 1, SY_BF16 = 2 } sy_dtype;

typedef enum sy_status {
  SY_OK = 0,
  SY_ERR_NULL = -1,        /* a required pointer is NULL                       */
  SY_ERR_SHAPE = -2,       /* a size is out of range (N < 1, D < 1, ...)       */
  SY_ERR_DTYPE = -3,       /* unknown dtype code or unsupported combination    */
  SY_ERR_WORKSPACE = -4,   /* workspace NULL or smaller than required          */
  SY_ERR_STRIDE = -5,      /* src_stride < n_tok * D                           */
  SY_ERR_DEVICE = -6,      /* no usable HIP device                             */
  SY_ERR_OP = -7           /* unknown operation or probe kind                  */
} sy_status;

/* Operations known to sy_plan(). */
typedef enum sy_op {
  SY_OP_FWD = 0,
  SY_OP_BWD = 1,
  SY_OP_BATCHED = 2,
  SY_OP_SOL = 3,
  SY_OP_BWD_BATCHED = 4
} sy_op;

/* Kernel families a plan can select. */
typedef enum sy_family {
  SY_FAMILY_RESIDENT = 0,  /* the whole [N, D] token tile lives in registers       */
  SY_FAMILY_CHUNKED = 1,   /* register tile of NR rows, online softmax over chunks */
  SY_FAMILY_GENERIC = 2,   /* element-wise loads, two passes per token             */
  SY_FAMILY_PER_QUERY = 3, /* batched op answered by one forward launch per query  */
  SY_FAMILY_MATRIX = 4     /* batched op on the matrix cores: 4 waves per token,
                              [N, D] staged in LDS, queries in registers         */
} sy_family;

/* How a call will be executed: which kernel family and which compile-time tile.
 * Pure host arithmetic on shapes -- no device is touched. */
typedef struct sy_plan {
  int32_t family;          /* sy_family                                          */
  int32_t waves_per_token; /* wavefronts that share one token's D axis           */
  int32_t chunks_per_lane; /* 16-byte chunks per lane per source row             */
  int32_t rows_per_tile;   /* compile-time rows held in registers (NR)           */
  int32_t elems_per_chunk; /* elements in one 16-byte chunk (8 for 16-bit types) */
  int32_t block_threads;   /* threads per workgroup                              */
  int32_t tokens_per_block;/* tokens a workgroup handles at once                 */
  int32_t n_chunks;        /* softmax chunks per token (1 = resident)            */
} sy_plan;

/* Fill *out with the execution plan for op at the given shape. `aligned` says
 * whether every pointer and row start is 16-byte aligned (the vector paths need
 * it). SY_OP_BWD plans assume the forward's stats are passed (the operator's
 * path); a backward without stats may run a thinner tile. The forward and
 * backward launches also take the token count into account: with at most two
 * tokens per CU (16-bit rows of four chunks a lane, 3 <= N <= 16) they run
 * tiles of four or two waves per token, and the backward does so also at
 * N = 2, for fp32 rows, and (up to four tokens per CU) where a wave's row
 * slice is two chunks a lane; the forward over 10-16 rows keeps four-row
 * chunks on four waves up to three tokens per CU and on two up to six, and
 * fp32 forwards take four waves a token up to one token per CU (10-16 rows:
 * two), and 16-bit D = 4096 up to one token per CU runs the forward on four
 * waves and the backward on eight;
 * sy_kernel_info and sy_plan_for_tokens report
 * the launched tile, this function, having no token count, does not.
 * Replaces the dispatch helpers _launch_config, _bwd_launch and
 * _batched_launch (src/switchyard/triton_op.py:130-150, :267-276, :420-435). */
int sy_plan_for(int op, int64_t n_src, int64_t n_q, int64_t d, int v_dtype, int w_dtype,
                int aligned, sy_plan* out);

/* sy_plan_for for a launch of n_tok tokens on the current device: for the
 * forward and the backward, the tile sy_fwd / sy_bwd run, with the token-count
 * rule and any sy_tuning_set tile override applied; other ops as
 * sy_plan_for. Without a device the token-count rule is skipped. No
 * counterpart in the reference, whose launch configuration ignores the token
 * count (src/switchyard/triton_op.py:130-150); it serves benchmarks and
 * callers that report the launched tile. */
int sy_plan_for_tokens(int op, int64_t n_src, int64_t n_q, int64_t n_tok, int64_t d, int v_dtype,
                       int w_dtype, int aligned, sy_plan* out);

/* Forward of the autograd operator: out = AttnRes(v, w).
 * Replaces _BlockAttnResTriton.forward and its _fwd_resident/_fwd_tiled
 * launches (src/switchyard/triton_op.py:505-536, :50-117).
 * `stats` may be NULL; when given it receives [2][N][n_tok] fp32: the logits,
 * then the inverse RMS r_n, which sy_bwd can reuse instead of recomputing.
 * w may have a different dtype from v (it is upcast, as in triton_op.py:67).
 * The same call on the same inputs returns the same bits. A token's result is
 * rounded once either way, but its last bit can depend on the launch it is
 * in (the tile the token count selects, and whether the persistent kernel
 * takes it as a wave's final token, whose rows are folded in as they land). */
int sy_fwd(const void* v, const void* w, void* out, float* stats, int64_t n_src, int64_t n_tok,
           int64_t d, int64_t src_stride, int v_dtype, int w_dtype, float eps, void* stream);

/* sy_fwd with the sources given as a host array of n_src <= SY_MAX_TABLE_ROWS
 * device pointers, v_rows[n] -> [n_tok][D]. The reference takes only a stacked
 * tensor and names a per-source pointer table (fla's API) as the better design
 * that removes the stacking copy (docs/report.md:401-404); this is that input.
 * SY_ERR_SHAPE when n_src > SY_MAX_TABLE_ROWS, SY_ERR_NULL for a NULL row. */
int sy_fwd_table(const void* const* v_rows, const void* w, void* out, float* stats, int64_t n_src,
                 int64_t n_tok, int64_t d, int v_dtype, int w_dtype, float eps, void* stream);

/* attn_with_stats: the unnormalised partial result of one source group,
 *     m = max_n logit_n,  l = sum_n exp(logit_n - m),  o = sum_n exp(logit_n - m) v_n,
 * so that o / l is the operator's output and two groups merge exactly with
 * sy_merge_stats. o has v's dtype; m and l are fp32 [n_tok]; stats as in sy_fwd.
 * Replaces attn_with_stats (src/switchyard/reference.py:194-215). */
int sy_attn_with_stats(const void* v, const void* w, void* o, float* m, float* l, float* stats,
                       int64_t n_src, int64_t n_tok, int64_t d, int64_t src_stride, int v_dtype,
                       int w_dtype, float eps, void* stream);

/* Phase 2 of the two-phase schedule in one pass: attn_with_stats over this
 * group's sources merged with a prior group's (o1, m1, l1) before anything is
 * written, so the group's own o is never stored and re-read:
 *     M = max(m1, max_n logit_n),  s1 = exp(m1 - M),
 *     o = s1 o1 + sum_n exp(logit_n - M) v_n,  l = s1 l1 + sum_n exp(logit_n - M).
 * normalize = 1: out = o / l (the operator's output over both groups);
 * normalize = 0: out = o, unnormalised, for a further merge. m and l always
 * receive (M, l). o1 has v's dtype [n_tok][D]; m1, l1, m, l are fp32 [n_tok].
 * Outputs must not overlap the prior's buffers. Replaces attn_with_stats
 * followed by merge_online_softmax (src/switchyard/reference.py:194-233, the
 * paper's Algorithm 1 phase 2, lines 10-12); SY_ERR_OP for normalize not 0/1. */
int sy_attn_with_stats_merge(const void* v, const void* w, const void* o1, const float* m1,
                             const float* l1, void* out, float* m, float* l, int64_t n_src,
                             int64_t n_tok, int64_t d, int64_t src_stride, int v_dtype,
                             int w_dtype, float eps, int normalize, void* stream);

/* Merge two (o, m, l) results of disjoint source groups into their union:
 * m = max(m1, m2), s_i = exp(m_i - m), o = s1 o1 + s2 o2, l = s1 l1 + s2 l2.
 * o may alias o1 or o2 (and m/l likewise). Replaces merge_online_softmax
 * (src/switchyard/reference.py:218-233). */
int sy_merge_stats(const void* o1, const float* m1, const float* l1, const void* o2,
                   const float* m2, const float* l2, void* o, float* m, float* l, int64_t n_tok,
                   int64_t d, int dtype, void* stream);

/* Gradient of sy_merge_stats: from dL/d(o, m, l) to dL/d(o1, m1, l1) and
 * dL/d(o2, m2, l2). The max goes to group 1 on a tie. Outputs must not alias
 * inputs. No reference counterpart (the reference merge is forward-only);
 * it completes the two-phase schedule's training path. */
int sy_merge_stats_bwd(const void* o1, const float* m1, const float* l1, const void* o2,
                       const float* m2, const float* l2, const void* grad_o, const float* grad_m,
                       const float* grad_l, void* do1, float* dm1, float* dl1, void* do2,
                       float* dm2, float* dl2, int64_t n_tok, int64_t d, int dtype, void* stream);

/* Bytes of device workspace sy_bwd needs for this shape on the current device
 * (per-workgroup fp32 dw partials). Returns < 0 (an sy_status) on bad input.
 * Replaces the fp32 dw buffer of triton_op.py:550. */
int64_t sy_bwd_workspace_bytes(int64_t n_src, int64_t n_tok, int64_t d, int v_dtype, int w_dtype);

/* Backward of the autograd operator: dv (v dtype, contiguous [N][n_tok][D])
 * and dw (w dtype, [D]) from grad_out (v dtype). dw is reduced
 * deterministically (per-workgroup partials + fixed-order tree), with no float
 * atomics. `stats` may be NULL (recompute) or the array sy_fwd wrote.
 * Replaces _BlockAttnResTriton.backward with _bwd_resident and
 * _bwd_stats/_bwd_apply (src/switchyard/triton_op.py:538-589, :194-375). */
int sy_bwd(const void* v, const void* w, const void* grad_out, const float* stats, void* dv,
           void* dw, void* workspace, int64_t workspace_bytes, int64_t n_src, int64_t n_tok,
           int64_t d, int64_t src_stride, int v_dtype, int w_dtype, float eps, void* stream);

/* sy_bwd over per-source pointer lists: v_rows and dv_rows each hold n_src <=
 * SY_MAX_TABLE_ROWS device pointers to [n_tok][D] rows (dv rows must not
 * overlap). Same workspace as sy_bwd. Pointer-table input as for sy_fwd_table. */
int sy_bwd_table(const void* const* v_rows, const void* w, const void* grad_out,
                 const float* stats, void* const* dv_rows, void* dw, void* workspace,
                 int64_t workspace_bytes, int64_t n_src, int64_t n_tok, int64_t d, int v_dtype,
                 int w_dtype, float eps, void* stream);

/* Largest dw partial-row buffer sy_bwd_static can use (bytes). */
#define SY_STATIC_WORKSPACE_BYTES (8 << 20)

/* sy_bwd that allocates nothing and takes no workspace: the dw partial rows
 * live in a static device array of SY_STATIC_WORKSPACE_BYTES per GPU (held
 * until the process ends), resolved once per device on the first call there.
 * No counterpart in the reference; for callers that cannot allocate device
 * memory -- code under HIP graph capture, tight serving loops, harnesses
 * that forbid allocation. Same kernels, grid and bits as sy_bwd. Returns
 * SY_ERR_WORKSPACE when sy_bwd_workspace_bytes() for the shape exceeds the
 * array. Every call on a GPU shares that GPU's array: calls that overlap on
 * one GPU (concurrent streams, or host threads) race and must be serialised
 * by the caller. */
int sy_bwd_static(const void* v, const void* w, const void* grad_out, const float* stats, void* dv,
                  void* dw, int64_t n_src, int64_t n_tok, int64_t d, int64_t src_stride, int v_dtype,
                  int w_dtype, float eps, void* stream);

/* Gradient of sy_attn_with_stats: from grad_o (v dtype [n_tok][D]) and grad_m,
 * grad_l (fp32 [n_tok]) to dv and dw, with k the first row holding the max:
 *     dlogit_n = p_n (G_n + grad_l) (n != k),  dlogit_k = grad_m - sum_{n != k} p_n (G_n + grad_l),
 *     p_n = exp(logit_n - m), G_n = <grad_o, v_n>, then dv, dw as in sy_bwd with
 *     p_n in place of alpha_n. Same workspace and stats as sy_bwd. The reference
 * has no backward for attn_with_stats (src/switchyard/reference.py:194-215). */
int sy_attn_with_stats_bwd(const void* v, const void* w, const void* grad_o, const float* grad_m,
                           const float* grad_l, const float* stats, void* dv, void* dw,
                           void* workspace, int64_t workspace_bytes, int64_t n_src, int64_t n_tok,
                           int64_t d, int64_t src_stride, int v_dtype, int w_dtype, float eps,
                           void* stream);

/* The two stages of sy_bwd, separately launchable (to time them, or to run the
 * small dw reduction later on another stream). sy_bwd == sy_bwd_main followed
 * by sy_dw_reduce over sy_bwd_partial_rows() rows of the workspace.
 * sy_bwd_partial_rows returns the row count (0 when n_tok == 0) or < 0 on bad
 * input; `aligned` as in sy_plan_for, `has_stats` whether stats will be
 * passed. sy_bwd_main writes dv and the fp32 partials [rows][D];
 * sy_dw_reduce writes dw[c] = sum_r partial[r][c] in a fixed order, cast to
 * w_dtype. Same reference interface as sy_bwd. */
int64_t sy_bwd_partial_rows(int64_t n_src, int64_t n_tok, int64_t d, int v_dtype, int w_dtype,
                            int aligned, int has_stats);
int sy_bwd_main(const void* v, const void* w, const void* grad_out, const float* stats, void* dv,
                void* workspace, int64_t workspace_bytes, int64_t n_src, int64_t n_tok, int64_t d,
                int64_t src_stride, int v_dtype, int w_dtype, float eps, void* stream);
int sy_dw_reduce(const float* partial, int64_t rows, int64_t d, void* dw, int w_dtype,
                 void* stream);

/* Output-only batched forward: out[s] = AttnRes(v, queries[s]) for S queries
 * sharing one read of v. queries has v's dtype.
 * Replaces block_attn_res_batched/_fwd_batched_resident
 * (src/switchyard/triton_op.py:438-501, :378-414). */
int sy_fwd_batched(const void* v, const void* queries, void* out, int64_t n_src, int64_t n_q,
                   int64_t n_tok, int64_t d, int64_t src_stride, int dtype, float eps,
                   void* stream);

/* sy_fwd_batched over a per-source pointer list (see sy_fwd_table). */
int sy_fwd_batched_table(const void* const* v_rows, const void* queries, void* out, int64_t n_src,
                         int64_t n_q, int64_t n_tok, int64_t d, int dtype, float eps,
                         void* stream);

/* Batched attn_with_stats: o[s] (v dtype [S][n_tok][D], unnormalised), m[s] and
 * l[s] (fp32 [S][n_tok]) for S queries sharing one read of v -- the batched
 * inter-block phase of the two-phase schedule, returning the merge statistics
 * the reference's batched API lacks (src/switchyard/reference.py:194-215,
 * triton_op.py:438-501). */
int sy_batched_with_stats(const void* v, const void* queries, void* o, float* m, float* l,
                          int64_t n_src, int64_t n_q, int64_t n_tok, int64_t d, int64_t src_stride,
                          int dtype, float eps, void* stream);

/* Bytes of workspace sy_bwd_batched needs (fp32 dq partials, one row of
 * n_q*D per workgroup of its persistent grid), or < 0 on bad input. */
int64_t sy_bwd_batched_workspace_bytes(int64_t n_src, int64_t n_q, int64_t n_tok, int64_t d,
                                       int dtype);

/* Backward of the batched forward: from grad_out [S][n_tok][D] (v dtype) to
 * dv (contiguous [N][n_tok][D]) = sum over queries of each query's source
 * gradient, and dq [S][D] (v dtype) = each query's pseudo-query gradient,
 * reduced over tokens in a fixed order (no float atomics). v is read once
 * for all S queries and dv is rounded once. The reference's batched API has no
 * backward (src/switchyard/triton_op.py:438-501, PROJECT_STATE.md:74-76 lists
 * it as next); this completes its training contract. */
int sy_bwd_batched(const void* v, const void* queries, const void* grad_out, void* dv, void* dq,
                   void* workspace, int64_t workspace_bytes, int64_t n_src, int64_t n_q,
                   int64_t n_tok, int64_t d, int64_t src_stride, int dtype, float eps,
                   void* stream);

/* Speed-of-light ceiling: out[t] = sum_n v_n[t] with the forward's geometry and
 * bytes but no softmax. Replaces speed_of_light (src/switchyard/triton_op.py:153-191). */
int sy_sol(const void* v, void* out, int64_t n_src, int64_t n_tok, int64_t d,
           int64_t src_stride, int dtype, void* stream);

/* HBM probes over `bytes` (a multiple of 16): kind 0 = read src (dst receives
 * one float per workgroup, dst must hold sy_probe_grid(bytes) floats, at most
 * 32768),
 * 1 = write dst, 2 = copy src -> dst, 3 = the forward's 9:1 read:write mix as
 * one linear stream: src holds `bytes` (a multiple of 144), read once in 36 KiB
 * steps, and dst receives bytes / 9 in 4 KiB steps, each 16-byte chunk the sum
 * (as 32-bit integers) of the chunks at the same position in the step's nine
 * 4 KiB source blocks. Replaces the copy/read/write probes of
 * bench/machine.py:41-61; kind 3 has no reference counterpart. */
int sy_bw_probe(int kind, const void* src, void* dst, int64_t bytes, void* stream);
int64_t sy_probe_grid(int64_t bytes);

/* Resources of the kernel a plan selects on the current device:
 * out[0] VGPRs per lane, out[1] static LDS bytes per workgroup, out[2] the
 * workgroups per CU the library assumes, out[3] the launch grid for n_tok
 * tokens. Diagnostics only; no reference counterpart. */
int sy_kernel_info(int op, int64_t n_src, int64_t n_tok, int64_t d, int v_dtype, int w_dtype,
                   int32_t out[4]);

/* Measurement-only overrides of the launch configuration. The library never
 * reads its environment: the kernel, tile and grid of every call are a
 * function of shape, dtype, alignment and device, unless a caller installs
 * overrides here. A tile triple {W, VPL, NR} of zeros keeps the planner's
 * choice; a triple is applied only where that tile is built, covers the row
 * and (backward, batched) holds every source, and is otherwise ignored.
 * bwd_blocks_per_cu (1..64) replaces the backward's persistent workgroups per
 * CU -- and with it the dw partial-row count and dw's bits. mx_slots (1 or 2)
 * sets the token slots of the matrix-core batched forward; bmx_waves = 4 runs
 * the four-wave matrix-core batched backward. The overrides are process-wide
 * and apply to calls issued after sy_tuning_set returns; they exist for tile
 * sweeps and for tests that force a tile. No reference counterpart (the
 * reference's tile constants are module globals, triton_op.py:120-150). */
typedef struct sy_tuning {
  int32_t fwd_tile[3];
  int32_t bwd_tile[3];
  int32_t batched_tile[3];
  int32_t sol_tile[3];
  int32_t bwd_blocks_per_cu;
  int32_t mx_slots;
  int32_t bmx_waves;
} sy_tuning;

/* Install overrides (NULL restores the defaults). SY_ERR_SHAPE for a value
 * out of range, which leaves the previous overrides in place. */
int sy_tuning_set(const sy_tuning* t);
/* Copy the installed overrides (all zeros when none). */
int sy_tuning_get(sy_tuning* out);

/* Static string for a status code (negative sy_status or positive hipError_t). */
const char* sy_strerror(int code);

/* SY_ABI_VERSION of the loaded library. */
int sy_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* SWITCHYARD_H */
