/*
 * sandmuon_amd.h -- C ABI of libsandmuon_amd.so, the MI355X (gfx950) HIP
 * implementation of the SandMuon optimizer step.
 *
 * Every entry point is extern "C", takes plain pointers and sizes, and
 * enqueues work on the explicit `stream` (a hipStream_t passed as void*).
 * No entry point allocates or frees device memory, synchronises the device
 * or copies device data to the host (smx_s8_timing_read, a benchmark aid,
 * waits for the events it reports).  Device buffers (including workspaces)
 * belong to the caller.  Descriptor tables (smx_*_desc) are HOST arrays:
 * the library copies them into kernel arguments by value at launch, so the
 * caller may reuse or free them as soon as the call returns.
 *
 * Return value: SMX_OK (0) on success; a negative SMX_E* code for invalid
 * arguments (shape, dtype, alignment, workspace size); SMX_ELAUNCH when a
 * kernel launch fails.  smx_last_error() returns a thread-local message for
 * the last failure on the calling thread.
 *
 * Threads: entry points may be called from several host threads, also on
 * one device and with different streams.  smx_matrix_step and smx_s8 fork
 * part of their launches onto a second stream of the device that the
 * library owns; the enqueue from that fork to its join is serialised by a
 * process-wide lock, so concurrent callers never share a fork.  Calls whose
 * device buffers overlap (the same workspace, slot rows or parameters)
 * must be ordered by the caller, as for any kernels.  The S8 launch
 * recorder (smx_s8_timing) and the test aids smx_s8_comp_stages,
 * smx_s8_comp_mask and smx_s8_tile_geometry are process-wide settings, not
 * thread-safe.
 *
 * The reference interface each entry point replaces is cited as
 * path:line under pxike/SandMuon.
 */
#ifndef SANDMUON_AMD_H
#define SANDMUON_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SMX_ABI_VERSION 5

enum smx_status {
  SMX_OK = 0,
  SMX_EINVAL = -1,      /* null pointer, bad count or enum          */
  SMX_ESHAPE = -2,      /* unsupported or inconsistent shape         */
  SMX_EDTYPE = -3,      /* unsupported element type                  */
  SMX_EALIGN = -4,      /* pointer or stride alignment               */
  SMX_EWORKSPACE = -5,  /* workspace too small                       */
  SMX_ELAUNCH = -6      /* kernel launch failed (see smx_last_error) */
};

/* SMX_F64 is accepted by the module-level helpers only (smx_inverse_sqrt,
 * smx_rank1_apply), which the reference also runs in float64. */
enum smx_dtype { SMX_F32 = 0, SMX_BF16 = 1, SMX_F16 = 2, SMX_F64 = 3 };

/* Arithmetic of the S8 polar map.
 * SMX_S8_FP32: every product on FP32 MFMA (v_mfma_f32_32x32x2_f32), FP32
 *   intermediates.  Restates sandmuon/optimizer.py:69-93.
 * SMX_S8_COMP_BF16: every product as three BF16 MFMAs on hi/lo splits
 *   (hi*lo + lo*hi + hi*hi, FP32 accumulation); intermediates are stored as
 *   the BF16 hi/lo pair.  The compensated-product scheme of
 *   reproduction/odl/ops/bf16_compensated_mm_fast.py:18-68, applied to all
 *   five stages.
 * SMX_S8_MIXED: stages 1 and 2 as SMX_S8_COMP_BF16 (stage 1 maps the raw
 *   input, whose range needs BF16's exponent; stage 2's rounding is the
 *   one the later stages amplify most); stages 3-5 of a matrix with
 *   rows == cols after padding (run on the iterate, X-space) on FP16
 *   operands with FP32 accumulation (v_mfma_f32_32x32x16_f16, one product
 *   per 16 K).  A wider matrix (run on r x r Gram products) stays
 *   compensated in every stage: its Gram has the square of the iterate's
 *   spectrum, which FP16 does not hold.  Direction error up to about 3e-3
 *   against the FP32 map; the S8 time falls with the share of square
 *   matrices.  No counterpart in the reference (whose historical recipe,
 *   reproduction/odl/ops/dense_s8_compensated_fast.py:53-85, runs stages
 *   2-5 as plain BF16 products). */
enum smx_s8_mode { SMX_S8_FP32 = 0, SMX_S8_COMP_BF16 = 1, SMX_S8_MIXED = 2 };

int smx_abi_version(void);
const char *smx_last_error(void);

/* ------------------------------------------------------------------ *
 * Statistics (forward hook A-capture and cotangent hook B-capture).
 * Replaces the hook bodies at sandmuon/optimizer.py:156-168 (A: sum of
 * x^2, and sum of x for the rank-one variant) and :171-177 (B: sum of
 * delta^2).
 *
 * x is a [rows, cols] view with unit column stride and row stride
 * `row_stride` elements, of type `dtype`.  The per-channel partial sums are
 * added into `n_slots` slot rows: slots_sq[p*cols + c] (and slots_first)
 * for p in [0, n_slots).  Each slot row is owned by one row chunk, so the
 * accumulation is deterministic and needs no atomics.  The slot rows are
 * folded into the running sums by smx_stats_fold / smx_stats_finish.
 * slots_first may be NULL (B side, diagonal A).
 * ------------------------------------------------------------------ */
int smx_stats_accumulate(const void *x, int dtype, int64_t rows, int64_t cols,
                         int64_t row_stride, float *slots_sq,
                         float *slots_first, int32_t n_slots, void *stream);

/* smx_stats_accumulate_batch: several hook calls of the bodies above in
 * one launch (the same sandmuon/optimizer.py:156-168 / :171-177 bodies,
 * applied to n_desc inputs at once).  Each descriptor adds exactly what
 * smx_stats_accumulate with the same arguments adds, bit for bit.  The
 * descriptors run concurrently, so no two may share slot rows (SMX_EINVAL
 * if their slot ranges overlap); the inputs must stay unmodified until the
 * launch has run on `stream`. */
typedef struct smx_stats_desc {
  const void *x;
  float *slots_sq;
  float *slots_first;   /* NULL: B side or diagonal A */
  int64_t rows, cols, row_stride;
  int32_t dtype, n_slots;
} smx_stats_desc;

int smx_stats_accumulate_batch(const smx_stats_desc *descs, int32_t n_desc,
                               void *stream);

/* smx_stats_slot_rows: how many leading slot rows (of n_slots) a call with
 * `rows` input rows adds into (the row chunks hold at least 512 rows), so
 * that the fold and finish can skip rows no call touched; -1 for invalid
 * arguments.  No counterpart in the reference (its sums have no slots). */
int32_t smx_stats_slot_rows(int64_t rows, int32_t n_slots);

/* The statistics fused into passes a mixed-precision Linear makes anyway
 * (the hook bodies above, moved; no counterpart entry point in the
 * reference).  Both add sum(x^2) to slots_sq exactly as
 * smx_stats_accumulate does, bit for bit.
 *
 * smx_stats_cast: the forward's fp32 -> bf16/f16 input cast (what autocast
 * does before the GEMM) with the A statistic of sandmuon/optimizer.py:
 * 156-168 taken from the same read.  x must be f32; out (out_dtype
 * SMX_BF16 or SMX_F16, row stride out_stride) receives x rounded to nearest
 * even.  slots_first may be NULL. */
int smx_stats_cast(const void *x, int dtype, int64_t rows, int64_t cols,
                   int64_t row_stride, float *slots_sq, float *slots_first,
                   int32_t n_slots, void *out, int out_dtype,
                   int64_t out_stride, void *stream);

/* smx_stats_gelu: out = GELU(x) (the exact form, x * 0.5 * (1 + erf(x /
 * sqrt(2))) in FP32, rounded to the input dtype) with the A statistic of
 * sandmuon/optimizer.py:156-168 of the output taken in the same pass, for
 * the Linear the GELU feeds (no reference entry point).  The
 * statistic goes to per-chunk partials, not to slot rows: part_sq (and
 * part_first, or NULL) receive smx_stats_slot_rows(rows, n_slots) rows of
 * cols FP32 sums, which smx_stats_add_partials later adds into the Linear's
 * slot rows; the result is the slot rows a smx_stats_accumulate of out
 * would leave, bit for bit.  x and out are bf16 or f16 (out in x's dtype),
 * with cols and row strides multiples of 8 elements and 16-byte aligned
 * pointers (SMX_EALIGN otherwise). */
int smx_stats_gelu(const void *x, int dtype, int64_t rows, int64_t cols,
                   int64_t row_stride, void *out, int64_t out_stride,
                   float *part_sq, float *part_first, int32_t n_slots,
                   void *stream);

/* smx_stats_relayout: the row-major copy out[b*seq + t][h*head_dim + d] =
 * x[b, t, h, d] of a [batch, seq, heads, head_dim] view with strides
 * (batch_stride, seq_stride, head_stride, 1) (an attention output handed
 * back from [batch, heads, seq, head_dim] to the Linear that projects it),
 * with the A statistic of sandmuon/optimizer.py:156-168 of the copy taken
 * in the same pass, for that Linear (no reference entry point).  The
 * statistic goes to per-chunk partials as for smx_stats_gelu
 * (smx_stats_slot_rows(batch*seq, n_slots) rows of heads*head_dim FP32
 * sums; part_first may be NULL), equal bit for bit to what a
 * smx_stats_accumulate of out would add.  x and out are bf16 or f16 (out
 * in x's dtype, contiguous); head_dim and the strides are multiples of 8
 * elements, x and out 16-byte aligned (SMX_EALIGN otherwise); seq must be a
 * multiple of the statistic's row chunk, max(ceil(batch*seq / n_slots),
 * 512) rows, so that no chunk crosses a sequence (SMX_ESHAPE otherwise). */
int smx_stats_relayout(const void *x, int dtype, int64_t batch, int64_t seq,
                       int64_t heads, int64_t head_dim, int64_t batch_stride,
                       int64_t seq_stride, int64_t head_stride, void *out,
                       float *part_sq, float *part_first, int32_t n_slots,
                       void *stream);

/* slots[p*cols + c] += part[p*cols + c] for p < n_rows (FP32), for sq and,
 * when both are given, first: the addition a statistics call makes into its
 * slot rows, applied to the partials of smx_stats_gelu and
 * smx_stats_relayout. */
int smx_stats_add_partials(float *slots_sq, const float *part_sq,
                           float *slots_first, const float *part_first,
                           int64_t cols, int32_t n_rows, void *stream);

/* smx_stats_colsum: the backward's bias gradient, colsum[c] = sum over the
 * rows of x, with the B statistic of sandmuon/optimizer.py:171-177 taken
 * from the same read.  The read writes one FP32 partial per row chunk into
 * `workspace` (smx_stats_colsum_workspace_bytes(cols, n_slots) bytes,
 * 256-byte aligned); a second, small launch folds them in a fixed order in
 * FP64.  rows may be 0 (colsum becomes zero).  Calls sharing a workspace
 * must be ordered on one stream. */
int64_t smx_stats_colsum_workspace_bytes(int64_t cols, int32_t n_slots);
int smx_stats_colsum(const void *x, int dtype, int64_t rows, int64_t cols,
                     int64_t row_stride, float *slots_sq, int32_t n_slots,
                     float *colsum, void *workspace, int64_t workspace_bytes,
                     void *stream);

/* Fold: sum[c] += sum_p slots[p*n + c] (in FP64), then zero the slots.
 * Used when the running sums must be materialised outside a step (for
 * example before state_dict()).  first_* may be NULL. */
int smx_stats_fold(float *sum_sq, float *slots_sq, float *sum_first,
                   float *slots_first, int64_t n, int32_t n_slots,
                   void *stream);

/* One vector to finish.  kind: 0 = diagonal A factor, 1 = rank-one A
 * factor, 2 = B factor (relative cotangent shape). */
typedef struct smx_finish_desc {
  float *sum_sq;      /* [n] running sum of squares; zeroed on return     */
  float *slots_sq;    /* [n_slots*n] pending slot rows; zeroed on return  */
  float *sum_first;   /* [n] running sum (kind 1) or NULL; zeroed         */
  float *slots_first; /* [n_slots*n] (kind 1) or NULL; zeroed             */
  float *ema;         /* [n] a_ema / b_ema, updated                       */
  float *mean_ema;    /* [n] a_mean_ema (kind 1) or NULL                  */
  float *inv;         /* [n] out: diagonal inverse square root            */
  float *z;           /* [n] out: rank-one vector (kind 1) or NULL        */
  float *kappa;       /* [1] out: rank-one coefficient (kind 1) or NULL   */
  int64_t n;
  int64_t count;      /* rows accumulated (host count, >= 1)              */
  int32_t n_slots;
  int32_t kind;
  int32_t first;      /* 1: EMA starts as a copy (first step)             */
  int32_t pad_;
} smx_finish_desc;

/* Batched _finish_a / _finish_b: sandmuon/optimizer.py:182-222 with
 * rank1_inverse_sqrt (:27-35) and diagonal_inverse_sqrt (:19-24).
 * Scalar hyperparameters are passed in double: the FP32 coefficients beta
 * and 1 - beta are both rounded from double, as the reference's
 * mul_(beta).add_(x, alpha=1-beta) rounds two Python floats.
 * `descs` is a host array of n_desc descriptors (device pointers inside). */
int smx_stats_finish(const smx_finish_desc *descs, int32_t n_desc,
                     double beta, void *stream);

/* smx_stats_finish in one fold and one finish launch for any n_desc (the
 * call above launches one pair per 32 descriptors, which travel by value in
 * the kernel arguments).  The descriptors are checked as there and written
 * in order on `stream` to `dev_table` (device memory of table_bytes >=
 * smx_stats_finish_table_bytes(n_desc) bytes), which the kernels read:
 * they travel in the kernel arguments of small upload launches (3840 bytes
 * each), so `descs` may be reused when the call returns and the call never
 * waits for the device.  The caller keeps dev_table for this call until its
 * launches have run (an event recorded on `stream` after the call marks
 * it).  No counterpart in the reference (the same
 * sandmuon/optimizer.py:182-222); for callers with more vectors than one
 * launch of smx_stats_finish takes. */
size_t smx_stats_finish_table_bytes(int32_t n_desc);
int smx_stats_finish_staged(const smx_finish_desc *descs, int32_t n_desc,
                            double beta, void *dev_table, size_t table_bytes,
                            void *stream);

/* ------------------------------------------------------------------ *
 * AdamW on the auxiliary parameters: sandmuon/optimizer.py:268-281.
 * ------------------------------------------------------------------ */
typedef struct smx_adamw_desc {
  void *param;         /* [n] of param_dtype                        */
  const void *grad;    /* [n] of grad_dtype                         */
  float *exp_avg;      /* [n]                                       */
  float *exp_avg_sq;   /* [n]                                       */
  int64_t n;
  int64_t offset;      /* exclusive prefix sum of n over the table   */
  float bias1;         /* 1 - beta1^step (this tensor's step)        */
  float bias2;         /* 1 - beta2^step                             */
  int32_t grad_dtype;
  int32_t param_dtype; /* SMX_F32, SMX_BF16 or SMX_F16                */
} smx_adamw_desc;

/* The state (exp_avg, exp_avg_sq) is FP32 for every parameter dtype.  A
 * 16-bit parameter is updated as the reference updates it
 * (sandmuon/optimizer.py:280-281): p = round(p * (1 - lr*wd)), then
 * p = round(p - lr * round(update)), each round to the parameter dtype. */

int smx_adamw(const smx_adamw_desc *descs, int32_t n_desc, int64_t total,
              double lr, double beta1, double beta2, double eps,
              double weight_decay, void *stream);

/* smx_adamw in one launch for any n_desc (the call above launches once per
 * 56 descriptors): the descriptors are written to `dev_table` (table_bytes
 * >= smx_adamw_table_bytes(n_desc, total) bytes) as in
 * smx_stats_finish_staged, with the same lifetimes, and each block finds
 * its first tensor in the table.  No counterpart in the reference (the same
 * sandmuon/optimizer.py:268-281); for models with more auxiliary tensors
 * than one launch of smx_adamw takes. */
size_t smx_adamw_table_bytes(int32_t n_desc, int64_t total);
int smx_adamw_staged(const smx_adamw_desc *descs, int32_t n_desc,
                     int64_t total, double lr, double beta1, double beta2,
                     double eps, double weight_decay, void *dev_table,
                     size_t table_bytes, void *stream);

/* ------------------------------------------------------------------ *
 * Matrix update: Nesterov momentum -> whiten -> S8 -> mapback -> graft ->
 * W -= lr * direction.  sandmuon/optimizer.py:244-264 and :283-315, with
 * rank1_whiten (:38-45), _s8_fp32 (:69-93), rank1_mapback (:48-60) and
 * _graft_direction (:63-66).
 *
 * In parameter layout (W is [rows, cols], input channels are columns) the
 * A factor acts on columns and the B factor on rows for both orientations:
 *   S = beta*m' + (1-beta)*g,      m' = beta*m + (1-beta)*g
 *   V = (D_b S D_a)(I + kappa z z^T)            (whiten)
 *   Q = S8(V)    (computed on the r<=c orientation of V)
 *   U = D_b Q (I + kappa z z^T) D_a             (mapback)
 *   W -= lr * sqrt(rows) * U / max(||U||_F, FLT_MIN)
 * The diagonal variant has z = NULL (kappa ignored).  The momentum is FP32
 * for every parameter dtype; a 16-bit parameter receives
 * W = round(W - lr * round(direction)) (sandmuon/optimizer.py:315, where
 * direction.to(parameter.dtype) is added with alpha -lr).
 * ------------------------------------------------------------------ */
typedef struct smx_matrix_desc {
  void *param;           /* [rows, cols] of param_dtype, row-major    */
  const void *grad;      /* [rows, cols] of grad_dtype                */
  float *momentum;       /* [rows, cols] fp32, updated in place       */
  const float *inv_row;  /* [rows] B factor                           */
  const float *inv_col;  /* [cols] A factor diagonal                  */
  const float *z;        /* [cols] A rank-one vector or NULL          */
  const float *kappa;    /* [1] A rank-one coefficient or NULL        */
  int64_t rows, cols;
  double lr;
  double momentum_beta;
  int32_t grad_dtype;
  int32_t param_dtype;   /* SMX_F32, SMX_BF16 or SMX_F16              */
} smx_matrix_desc;

/* Device workspace needed for one smx_matrix_step call over the given
 * matrices (rows[i], cols[i] are host arrays of parameter shapes). */
size_t smx_matrix_step_workspace_bytes(const int64_t *rows,
                                       const int64_t *cols, int32_t n,
                                       int mode);

/* Runs the whole matrix update for the n matrices of the host table
 * `descs`.  Either every matrix of a call has a rank-one term (z, kappa
 * set) or none has (SMX_EINVAL otherwise); an optimizer is one or the
 * other.  The workspace (256-byte aligned, at least
 * smx_matrix_step_workspace_bytes) holds the S8 iterates; its contents on
 * entry are irrelevant.  Everything is ordered on `stream`: the S8 map
 * runs part of its matrices on a second stream of the device (created by
 * the library, default priority), which waits for `stream` at the start
 * and which `stream` waits for before the call's later launches, so to
 * the caller the call behaves as if every launch were on `stream`. */
int smx_matrix_step(const smx_matrix_desc *descs, int32_t n, int mode,
                    void *workspace, size_t workspace_bytes, void *stream);

/* smx_matrix_step_static: smx_matrix_step with its workspace in a static
 * device array of SMX_MATRIX_STEP_STATIC_BYTES instead of a caller buffer.
 * No counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid allocation).  It allocates nothing; the array is
 * placed on a GPU by the first call there and held until the process ends.
 * Matrices whose workspace (smx_matrix_step_workspace_bytes) exceeds the
 * array are refused with SMX_EWORKSPACE before any launch.  Every call on
 * one GPU uses that GPU's one array: calls that overlap on one GPU race. */
#define SMX_MATRIX_STEP_STATIC_BYTES ((size_t)1 << 30)
int smx_matrix_step_static(const smx_matrix_desc *descs, int32_t n, int mode,
                           void *stream);

/* ------------------------------------------------------------------ *
 * Stand-alone S8 polar map on a batch: _s8_fp32, sandmuon/optimizer.py:
 * 69-93.  x and out are [batch, rows, cols] fp32 with the given strides
 * (elements); out may alias x.  A matrix that is entirely zero maps to
 * zero.  (The reference returns zeros only when the whole batch is zero
 * and NaN for a zero matrix inside a non-zero batch.)  Ordered on
 * `stream` as smx_matrix_step is (a batch of 4 or more matrices runs half
 * of them on the library's second stream).
 * ------------------------------------------------------------------ */
size_t smx_s8_workspace_bytes(int64_t batch, int64_t rows, int64_t cols,
                              int mode);
int smx_s8(const float *x, float *out, int64_t batch, int64_t rows,
           int64_t cols, int64_t batch_stride, int64_t row_stride,
           int64_t col_stride, int mode, void *workspace,
           size_t workspace_bytes, void *stream);

/* ------------------------------------------------------------------ *
 * Launch timing of the S8 kernels (no counterpart in the reference; a
 * measurement aid for benchmarks).  smx_s8_timing(1) discards earlier
 * records and starts recording a HIP event pair around every S8 phase
 * launch (by smx_matrix_step and smx_s8) and around every whole S8 run,
 * on its stream; smx_s8_timing(2) records whole runs only (two events per
 * run, so the launches inside it run back to back); smx_s8_timing(0)
 * stops recording.  smx_s8_timing_read waits for the recorded launches
 * and writes up to `capacity` records in the order they were opened:
 * duration (ms), phase (0 Gram, 1 square, 2 apply, 3 stage-1 polynomial,
 * 4 a whole S8 run, first launch to last, 5 the symmetric r x r products
 * of Gram-space classes, which are iterated on r x r matrices when their
 * padded columns exceed their padded rows)
 * and the MFMA FLOPs the launch (or run) issues (tiles computed x
 * 2*256*256*K, x3 in SMX_S8_COMP_BF16 mode, plus the square phase's
 * one-hot MFMAs).  It returns the number of records or a negative status.
 * The recorder is process-wide, not thread-safe.
 * ------------------------------------------------------------------ */
int smx_s8_timing(int32_t enable);
int32_t smx_s8_timing_read(float *ms, int32_t *phase, double *flops,
                           int32_t capacity);

/* ------------------------------------------------------------------ *
 * Module-level helpers (sandmuon/optimizer.py:19-66), in the dtype of their
 * inputs as the reference computes them: SMX_F32 or SMX_F64.
 *
 * smx_inverse_sqrt: the factor of one statistics vector of n channels.
 *   kind 0, diagonal_inverse_sqrt (:19-24): inv = rsqrt(max(max(v, m*1e-6) /
 *     max(m, tiny), 1e-6)) with m = mean(v) (`second` is v; mean, z and
 *     kappa are unused and may be NULL).
 *   kind 1, rank1_inverse_sqrt (:27-35): q = max(mean(second), tiny),
 *     inv = rsqrt(max(max(second - mean^2, 0) / q, 1e-6)),
 *     z = inv * (mean / sqrt(q)), rho = sqrt(1 + |z|^2),
 *     kappa = -1 / (rho (rho + 1)) (kappa: one element).
 *   Every pointer is a device pointer of `dtype`; n >= 1.
 * smx_rank1_apply: rank1_whiten (:38-45, order 0) and rank1_mapback
 *   (:48-60, order 1) on a contiguous batch [batch, rows, cols] of `dtype`;
 *   both sides may carry a rank-one term.  li/lz are [batch, rows], ri/rz
 *   [batch, cols], lc/rc [batch] (device, `dtype`).  `work` holds
 *   batch*(rows+cols) doubles.  out must not alias x.
 * smx_graft: _graft_direction (:63-66) on n contiguous fp32 values (the
 *   reference grafts in float32 whatever the input dtype):
 *   out = x*sqrt(output_rows)/max(||x||_F, FLT_MIN); a zero input gives a
 *   zero output (the reference returns NaN for a zero input once
 *   sqrt(rows)/FLT_MIN overflows).  `work` holds work_len doubles (>= 1).
 * ------------------------------------------------------------------ */
int smx_inverse_sqrt(int kind, int dtype, const void *second,
                     const void *mean, int64_t n, void *inv, void *z,
                     void *kappa, void *stream);

int smx_rank1_apply(int dtype, const void *x, void *out, int64_t batch,
                    int64_t rows, int64_t cols, const void *li,
                    const void *lz, const void *lc, const void *ri,
                    const void *rz, const void *rc, int order, double *work,
                    void *stream);

int smx_graft(const float *x, float *out, int64_t n, int64_t output_rows,
              double *work, int32_t work_len, void *stream);

/* ------------------------------------------------------------------ *
 * Compensated stages of SMX_S8_COMP_BF16 (no counterpart in the
 * reference; a measurement aid for choosing the recipe).  Stages 1..k use
 * the compensated product hi*lo + lo*hi + hi*hi, stages k+1..5 the plain
 * BF16 product hi*hi of the same stored operands.  The default, 5, is the
 * production recipe; 1 is the historical one
 * (reproduction/odl/ops/dense_s8_compensated_fast.py:53-85).  Process-wide,
 * read at each S8 launch; returns the previous value, or SMX_EINVAL for k
 * outside [0, 5] (then nothing changes).
 * ------------------------------------------------------------------ */
int smx_s8_comp_stages(int32_t k);

/* smx_s8_comp_mask: the same choice per stage (no counterpart in the
 * reference; a measurement aid): bit k-1 set compensates stage k, a clear
 * bit makes it the plain BF16 product hi*hi (whose one-hot linear term
 * keeps the scalar's hi and lo).  0x1f is the production recipe.  Returns
 * the previous mask, or SMX_EINVAL outside [0, 0x1f]. */
int smx_s8_comp_mask(int32_t mask);

/* ------------------------------------------------------------------ *
 * MFMA peak probe (no counterpart in the reference; a measurement aid for
 * the roofline denominators).  `blocks` blocks of 512 threads (8 waves,
 * two per SIMD) each issue `iters` rounds of 4 independent dense MFMAs on
 * register operands, no memory traffic: v_mfma_f32_32x32x16_bf16 (dtype
 * SMX_BF16) or _f16 (SMX_F16), 32768 FLOP each, or
 * v_mfma_f32_32x32x2_f32 (SMX_F32), 4096 FLOP each.  Lane 0 of each block
 * writes times[4*b .. 4*b+3] = s_memtime at start and end (engine clock
 * cycles), then s_memrealtime at start and end (a 100 MHz counter), from
 * which the caller derives the clock held under the load; sink receives
 * blocks*512 floats that depend on every MFMA.  Enqueues on `stream`; the
 * caller times it (events).
 * ------------------------------------------------------------------ */
int smx_mfma_peak(int32_t dtype, int32_t blocks, int64_t iters,
                  uint64_t *times, float *sink, void *stream);

/* ------------------------------------------------------------------ *
 * Tile geometry of the S8 GEMM launches (no counterpart in the reference;
 * a test and measurement aid).  0 (the default): each launch picks its
 * tiles from its size (256 x 256 blocks of 8 waves for launches that fill
 * the device with a long K loop, else 256 x 128 or 128 x 128 blocks of 4
 * waves); 1: 256 x 256 tiles for every launch; 2: never 256 x 256.  The
 * results agree to rounding across geometries.  Process-wide, read at each
 * S8 launch; returns the previous value, or SMX_EINVAL for a value outside
 * [0, 2] (then nothing changes).
 * ------------------------------------------------------------------ */
int smx_s8_tile_geometry(int32_t policy);

#ifdef __cplusplus
}
#endif

#endif /* SANDMUON_AMD_H */
