/*
 * purin_cp.h -- C ABI of the MI355X Chambolle--Pock projection library
 * (libpurin_cp.so).
 *
 * Plain C: opaque plan handle, device pointers passed as void*, sizes as
 * int64_t, HIP streams as void* (hipStream_t).  No torch / JAX types.
 * Every array argument is a device pointer in batch-major row-major layout
 * ((B, n) means sample-major, like the reference), of the plan's dtype unless
 * stated otherwise.  The library never frees caller buffers.
 *
 * Reference interfaces each entry point replaces (paths are into the
 * reference repository, SOULS-TAMU/Purin 1.0.2):
 *   plan_create  <- PreparedChambollePockProjection.__post_init__ +
 *                   prepare_bounds + BoundProjection.__init__
 *                   (src/purin/solvers/chambolle_pock/solver.py:32-65,
 *                    src/purin/solvers/chambolle_pock/bounds.py:18-33, 320-326)
 *   spmm         <- _batched_local_jacobian_matvec / _transpose_matvec
 *                   (src/purin/linalg/sparse/operators.py:507-533)
 *   solve        <- the jitted custom_vjp ``solve`` -> sparse_cp
 *                   (src/purin/solvers/chambolle_pock/bounds.py:42-78,
 *                    src/purin/solvers/chambolle_pock/kernels.py:178-305)
 *   project      <- BoundProjection.solve / PreparedChambollePockProjection._solve
 *                   (src/purin/solvers/chambolle_pock/bounds.py:170-317,
 *                    src/purin/solvers/chambolle_pock/solver.py:277-366)
 *   adjoint      <- custom_vjp ``bwd`` (src/purin/solvers/chambolle_pock/bounds.py:80-165)
 *                   with _batched_restarted_gmres
 *                   (src/purin/solvers/primal_dual_interior_point/operators.py:792-1125)
 *   project_values / adjoint_values <- the same with per-sample coefficients
 *                   (bounds.py:192-239)
 *   qp_solve / qp_adjoint <- PreparedDiagonalQP (src/purin/solvers/diagonal_qp.py:69-319)
 *
 * Errors: entry points return PURIN_CP_OK or an error code for invalid
 * arguments / HIP failures (the reference raises ValueError for shape and
 * configuration errors, bounds.py:176-188, config.py:50-61).  Numerical
 * outcomes are never errors: they are reported per sample through status,
 * finite, converged and valid arrays, as in the reference.
 * purin_cp_last_error() returns a message for the calling thread's last error.
 *
 * Workspaces and threading (the reference's layer is pure functional under
 * jax.jit, bounds.py:33, 68-167): every compute entry point takes its device
 * scratch either from the caller (the ``workspace`` / ``workspace_bytes``
 * fields of its options struct; size from purin_cp_workspace_bytes) or, when
 * that is NULL, from a workspace the plan owns.
 *   - With a caller workspace a call allocates nothing and changes no plan
 *     state its results depend on: calls on one plan may then run
 *     concurrently, on different streams and from different threads, each
 *     with its own workspace (and its own saved-state buffer).  The plan's
 *     data is read-only to them.
 *   - With the plan's workspace, calls on one plan must be ordered (same
 *     stream or externally synchronised).  A workspace that must grow is
 *     replaced stream-ordered (hipMallocAsync / hipFreeAsync on the call's
 *     stream).
 * All kernels are enqueued on the given stream.  project/solve read a device
 * stop flag (a stream synchronisation) only on the streaming passes with
 * early stop, every check_every iterations; the adjoints read their per-step
 * counts likewise.  Such a call on a stream under capture returns
 * PURIN_CP_ERR_ARG instead of breaking the capture; so does a call that would
 * allocate (a plan workspace that must grow) or time itself under capture.
 * A call of more than the 65536 iterations the resident kernel's step
 * schedule holds extends the schedule once: it uploads the longer schedule on
 * a stream of the plan's own and waits for that upload only.  No entry point
 * synchronises the device or the caller's other streams (plan creation,
 * destruction and set_metric are set-up calls and may).  The last_* queries
 * report the last call that recorded them (timing: opts.timing; adjoint
 * iterations: calls on the plan's workspace).
 */
#ifndef PURIN_CP_H
#define PURIN_CP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PURIN_CP_ABI_VERSION 2

enum purin_cp_dtype { PURIN_CP_F32 = 0, PURIN_CP_F64 = 1 };

enum purin_cp_error {
  PURIN_CP_OK = 0,
  PURIN_CP_ERR_ARG = 1,          /* invalid argument (ValueError in the reference) */
  PURIN_CP_ERR_HIP = 2,          /* HIP runtime error */
  PURIN_CP_ERR_UNSUPPORTED = 3,  /* option this build does not implement */
  PURIN_CP_ERR_NOMEM = 4         /* device allocation failed */
};

/* SolveStatus codes (src/purin/solvers/types.py:36-43). */
enum purin_cp_status {
  PURIN_CP_CONVERGED = 0,
  PURIN_CP_MAX_ITERATIONS = 1,
  PURIN_CP_LINEAR_SOLVE_FAILURE = 2,
  PURIN_CP_NONFINITE = 3
};

typedef struct purin_cp_plan purin_cp_plan;

/* The ChambollePockConfig knobs fixed at preparation
 * (src/purin/solvers/chambolle_pock/config.py:34-48). */
typedef struct {
  int32_t accelerated;              /* accelerated CP update (default 0) */
  int32_t row_scaling;              /* constraint-row normalisation (default 1) */
  int32_t norm_bound;               /* sparse norm bound for the steps (default 1) */
  int32_t norm_iterations;          /* power iterations for the adjoint steps (default 20) */
  int32_t norm_seed;                /* start-vector seed (default 42) */
  int32_t diagonal_preconditioning; /* per-row/per-column steps when not accelerated
                                       (kernels.py:76-88, 209-210; default 0) */
  double safety;                    /* step safety factor in (0,1) (default 0.95) */
  int32_t bound_presolve;           /* 1: singleton inequality rows become variable
                                       bounds (bounds.py:320-326; default 1); 0: every
                                       row is kept, as the diagonal-QP layer does
                                       (diagonal_qp.py:96-123) */
  int32_t reserved;
} purin_cp_options;

/* Fill *opts with the reference defaults. */
void purin_cp_default_options(purin_cp_options* opts);

/*
 * Prepare a plan for one shared constraint matrix.
 *   rows 0..me-1        equalities      K y == rhs
 *   rows me..me+mi-1    inequalities    K y <= rhs
 * given as a host CSR (indptr[me+mi+1], indices, values in float64; columns
 * ascending within a row, as the reference's row supports).  Structural zeros
 * are kept: a row's support decides whether it is a singleton bound row.
 * Inequality rows with exactly one stored entry are presolved into variable
 * bounds (bounds.py:320-326); the remaining rows ("kept rows", equalities
 * first) enter the CP iteration.
 */
int purin_cp_plan_create(purin_cp_plan** plan, int32_t dtype, int64_t n, int64_t me,
                         int64_t mi, const int64_t* indptr, const int32_t* indices,
                         const double* values, const purin_cp_options* opts);

void purin_cp_plan_destroy(purin_cp_plan* plan);

typedef struct {
  int32_t dtype;
  int64_t n, me, mi;
  int64_t kept_rows;        /* m: rows that enter the iteration (me + general inequalities) */
  int64_t bound_rows;       /* presolved singleton inequality rows */
  int64_t nnz_kept;
  double norm;              /* L used by the forward steps */
  double tau0, sigma0;      /* initial forward steps */
  double adjoint_norm;      /* power-iteration L of the adjoint (bounds.py:88-101) */
  double adjoint_tau, adjoint_sigma;
  double tolerance_factor;  /* min(1, min_i scale_i): forward tolerance = tol * factor */
  /* Measurement figures of the resident (on-chip) kernel, 0 when it does not
   * apply (no reference counterpart): the bytes of the shared matrix's chunk
   * streams one workgroup (one tile of samples) reads from L2 per iteration in
   * the fixed-iteration and the early-stop kernels, and the row and column
   * slots of a workgroup (each slot reads or writes its own 16-byte LDS entry
   * once per pass). */
  int64_t resident_stream_bytes;
  int64_t resident_stream_bytes_early;
  int64_t resident_row_slots;
  int64_t resident_col_slots;
  /* Bytes the plan's own workspaces hold now (forward, adjoint); no reference
   * counterpart.  Calls with a caller workspace, and the no-allocation entry,
   * leave them unchanged. */
  int64_t workspace_bytes;
  int64_t adjoint_workspace_bytes;
  /* Samples of one resident workgroup (tile): 2 in fp64, 4 in fp32, or 8 in
   * fp32 where n and m fit one slot per thread (two LDS planes); 0 when the
   * resident kernel does not apply.  No reference counterpart. */
  int64_t resident_tile_samples;
} purin_cp_plan_info;

int purin_cp_plan_get_info(const purin_cp_plan* plan, purin_cp_plan_info* info);

/* Host copies of the kept-row indices (int64[m], original row numbers) and
 * their row scales (double[m], 1/||K_i||_2 or 1). */
int purin_cp_plan_kept_rows(const purin_cp_plan* plan, int64_t* rows, double* scale);

/*
 * Optional diagonal metric (WeightedDistance, src/purin/solvers/metric.py:87-182):
 * the plan's matrix must already be the scaled one (coefficients times
 * 1/sqrt(D_j)); this stores sqrt(D) (host, double[n]) so that project()
 * multiplies targets by sqrt(D) on entry and divides y by it on exit, and
 * adjoint() applies the matching chain rule.  Pass NULL to clear.
 */
int purin_cp_plan_set_metric(purin_cp_plan* plan, const double* sqrt_diagonal);

/* First-kernel entry: out = K x (transpose = 0; x (B,n) -> out (B,m)) or
 * K^T x (transpose = 1; x (B,m) -> out (B,n)) over the kept rows, with the
 * row-scaled coefficients when scaled != 0.  Uses the plan's workspace
 * (calls on one plan ordered). */
int purin_cp_spmm(purin_cp_plan* plan, void* stream, int64_t batch, int32_t transpose,
                  int32_t scaled, const void* x, void* out);

/* Per-call options of solve/project. */
typedef struct {
  double tolerance;        /* ChambollePockConfig.tolerance (1e-9) */
  int64_t max_iterations;  /* ChambollePockConfig.max_iterations (10000) */
  int32_t early_stop;      /* 1: per-sample stop test each iteration (reference
                              semantics); 0: run exactly max_iterations */
  int32_t check_every;     /* iterations between reads of the all-done flag (0: 32) */
  int32_t shared_bounds;   /* 1: lower/upper (or the bound-row rhs) are the same
                              for every sample; only sample 0 is read */
  int32_t timing;          /* 1: bracket every iteration kernel with HIP events on
                              the call's stream (see purin_cp_last_timing) */
  int32_t streaming;       /* 1: force the streaming row/column passes even when the
                              resident on-chip kernel applies (fixed iterations) */
  int32_t reserved;
  void* workspace;         /* caller device workspace (256-byte aligned) or NULL for the
                              plan's own; see purin_cp_workspace_bytes */
  int64_t workspace_bytes; /* its size in bytes */
} purin_cp_solve_options;

void purin_cp_default_solve_options(purin_cp_solve_options* opts);

/*
 * Bytes of the state buffer that project()/solve() fill when ``saved`` is
 * not NULL and that adjoint() reads (the custom_vjp residuals,
 * bounds.py:74-78).  Layout is internal; the buffer must stay untouched
 * between the forward and the adjoint call.
 */
int64_t purin_cp_saved_bytes(const purin_cp_plan* plan, int64_t batch);

/*
 * The inner CP solve on the kept rows in the plan's scaled units
 * (CPOutput of kernels.py:178-305, called as bounds.py:42-66).
 *   rhs     (B, m) scaled kept right-hand sides
 *   target  (B, n) candidates yhat (q = 1, c = -yhat, y0 = yhat)
 *   dual0   (B, m) scaled initial duals, or NULL for zero
 *   lower, upper (B, n) bounds (±inf allowed), or (n) with shared_bounds
 *   tol     (B) per-sample tolerance, or NULL for opts->tolerance
 *   feasible (B) uint8 or NULL; converged is ANDed with it (bounds.py:66)
 * Outputs y (B,n), dual (B,m) scaled, iterations int32 (B), residual (B),
 * gap (B), converged uint8 (B).
 */
int purin_cp_solve(purin_cp_plan* plan, void* stream, int64_t batch, const void* rhs,
                   const void* target, const void* dual0, const void* lower,
                   const void* upper, const void* tol, const uint8_t* feasible,
                   const purin_cp_solve_options* opts, void* y, void* dual,
                   int32_t* iterations, void* residual, void* gap, uint8_t* converged,
                   void* saved);

/*
 * Full projection (BoundProjection.solve, bounds.py:170-317).
 *   target (B, n); rhs (B, me+mi) = -[h(theta,0); g(theta,0)];
 *   multipliers0 (B, me+mi) warm-start multipliers in original units or NULL.
 * Outputs: y (B,n); multipliers (B, me+mi) (equalities then inequalities,
 * bound rows included); slacks (B, mi); status int32 (B); iterations int32
 * (B); residual (B) original-unit residual; finite uint8 (B);
 * eligible uint8 (B) (gradient_eligible).  Any output except y may be NULL.
 */
int purin_cp_project(purin_cp_plan* plan, void* stream, int64_t batch, const void* target,
                     const void* rhs, const void* multipliers0,
                     const purin_cp_solve_options* opts, void* y, void* multipliers,
                     void* slacks, int32_t* status, int32_t* iterations, void* residual,
                     uint8_t* finite, uint8_t* eligible, void* saved);

/*
 * The same projection as purin_cp_project(), for callers that cannot allocate
 * device memory during the call (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  No counterpart in the reference:
 * it exists for those callers.  It runs the same kernels on the same inputs
 * and outputs, with the call's working buffers (and the saved state when
 * ``saved`` is NULL) in one static device array of
 * PURIN_CP_NOALLOC_SCRATCH_BYTES per GPU, which each GPU the library runs on
 * holds until the process ends.  It calls no hipMalloc / hipFree or other
 * allocating routine.
 * Limits (each a PURIN_CP_ERR_ARG with a message, nothing launched):
 *   - the call's buffers must fit the scratch array (at the config-2 shape,
 *     n = 4096 with 3072 kept rows in fp64, a batch of up to 128 samples);
 *   - opts->max_iterations must not exceed the step schedule the plan built
 *     at creation (65536 iterations) when the resident kernel runs;
 *   - opts->timing must be 0;
 *   - the current device must be the plan's.
 * Every call on one GPU shares that GPU's array, which keeps the last call's
 * contents (the kernels clear what must start at zero): calls that overlap on
 * one GPU -- on different streams, or from different threads or plans --
 * race, and must be ordered by the caller.  A saved state written into the
 * array (saved == NULL) is not kept for an adjoint call.
 */
#define PURIN_CP_NOALLOC_SCRATCH_BYTES (128LL << 20)

int purin_cp_project_noalloc(purin_cp_plan* plan, void* stream, int64_t batch,
                             const void* target, const void* rhs, const void* multipliers0,
                             const purin_cp_solve_options* opts, void* y, void* multipliers,
                             void* slacks, int32_t* status, int32_t* iterations, void* residual,
                             uint8_t* finite, uint8_t* eligible, void* saved);

/*
 * Full projection with per-sample coefficients: the same rows and sparsity as
 * the plan, with every sample's own coefficient values.  Replaces
 * BoundProjection.solve when the coefficients depend on the parameters
 * (src/purin/solvers/chambolle_pock/bounds.py:192-236: values (B, m_tot, w)
 * from jax.vmap(_numeric_one); per-sample bounds from the bound rows'
 * coefficients, per-sample row scales, norm bound, steps and tolerance,
 * kernels.py:209-227).
 *   values (B, nnz) in the plan's CSR entry order (indptr/indices given to
 *   plan_create; the plan's own values are not used by this call).
 * Other arguments and outputs as purin_cp_project(); opts->shared_bounds must
 * be 0.  The saved state is for purin_cp_adjoint_values() only.  The
 * iterations run on the resident kernel where the problem fits it (each
 * workgroup streams its samples' coefficients; opts->streaming = 1 forces the
 * streaming passes); the results agree to rounding.
 */
int purin_cp_project_values(purin_cp_plan* plan, void* stream, int64_t batch,
                            const void* values, const void* target, const void* rhs,
                            const void* multipliers0, const purin_cp_solve_options* opts,
                            void* y, void* multipliers, void* slacks, int32_t* status,
                            int32_t* iterations, void* residual, uint8_t* finite,
                            uint8_t* eligible, void* saved);

/*
 * General positive diagonal QP on the plan's rows (PreparedDiagonalQP.solve,
 * src/purin/solvers/diagonal_qp.py:222-319, through sparse_cp with general q,
 * kernels.py:178-305):
 *   min 0.5 y' diag(q) y + c'y  s.t.  K[:me] y == rhs[:me], K[me:] y <= rhs[me:],
 *                                     lower <= y <= upper,
 * every row kept (the plan must be created with bound_presolve = 0) and no
 * metric.  q, c, lower, upper (B, n); values (B, nnz) per-sample
 * coefficients in the plan's CSR entry order, or NULL for the plan's own;
 * rhs (B, me+mi); y0 (B, n) or NULL for zero; dual0 (B, me+mi) or NULL.
 * Outputs y (B, n), multipliers (B, me+mi), slacks (B, mi), status,
 * iterations, residual (original units), finite, converged (B); each but y
 * may be NULL.  opts->shared_bounds must be 0.  The iterations run on the
 * resident kernel where the problem fits it (opts->streaming = 1 forces the
 * streaming passes); the results agree to rounding.
 */
int purin_cp_qp_solve(purin_cp_plan* plan, void* stream, int64_t batch, const void* q,
                      const void* c, const void* values, const void* rhs, const void* lower,
                      const void* upper, const void* y0, const void* dual0,
                      const purin_cp_solve_options* opts, void* y, void* multipliers,
                      void* slacks, int32_t* status, int32_t* iterations, void* residual,
                      uint8_t* finite, uint8_t* converged, void* saved);

/*
 * The dense CP adapter's forward (solve_dense, chambolle_pock/dense.py:26-105,
 * as called by dense_layer.py:13-134 after any equilibration): the diagonal
 * QP of purin_cp_qp_solve with the adapter's policy -- the factored prox
 * a ((y - tau K^T d) - tau c) (kernels.py:140-142), no freezing of accepted
 * samples (all iterate until the last is accepted), no stationarity in the
 * stop test, power-iteration steps.  The plan keeps every row
 * (bound_presolve = 0) with row_scaling = 0, norm_bound = 0 and
 * diagonal_preconditioning = 0; dense matrices are rows over all n columns
 * (a packed inequality_support gives those rows its columns).
 * Inputs as purin_cp_qp_solve.  Outputs y (B, n), multipliers (B, me+mi)
 * (lambda then mu), iterations (B); each but y may be NULL.
 */
int purin_cp_dense_solve(purin_cp_plan* plan, void* stream, int64_t batch, const void* q,
                         const void* c, const void* values, const void* rhs, const void* lower,
                         const void* upper, const void* y0, const void* dual0,
                         const purin_cp_solve_options* opts, void* y, void* multipliers,
                         int32_t* iterations, void* saved);

/* Kernel times of the last solve()/project() call made with opts.timing = 1,
 * from HIP events recorded on that call's stream around each launch. */
typedef struct {
  int64_t iterations;   /* CP iterations timed */
  double row_ms;        /* summed row-pass time */
  double col_ms;        /* summed column-pass time */
  double diag_ms;       /* summed residual + decide time (stop test) */
  double loop_ms;       /* first iteration kernel start to last end */
  int32_t resident;     /* 1: the iterations ran in the resident kernel (one launch) */
  int32_t linear_kybar; /* 1: the streaming passes formed K ybar = (1 + theta) K y -
                           theta K y_prev instead of storing ybar (n > 2 m) */
  int32_t narrow_columns; /* 1: the fixed-iteration column pass took a quarter
                             wavefront per column (batch tiles of 16 lanes: the
                             gathered d+ slice of a tile fits an XCD's L2) */
} purin_cp_timing;

int purin_cp_last_timing(const purin_cp_plan* plan, purin_cp_timing* timing);

/* GMRES and gradient policy (LinearSolverConfig / ImplicitGradientConfig,
 * src/purin/solvers/config.py:13-16, 94). */
typedef struct {
  double tolerance;          /* 1e-9 */
  double atol;               /* 0 */
  int32_t restart;           /* 30 */
  int32_t max_iterations;    /* 100 */
  double adjoint_tolerance;  /* 1e-8 */
  int32_t force_eligible;    /* 1: treat every sample as converged (benchmark of
                                a fixed-iteration state); 0: reference rule */
  int32_t reserved;
  void* workspace;           /* caller device workspace (256-byte aligned) or NULL */
  int64_t workspace_bytes;   /* its size in bytes */
  int32_t* arnoldi_iterations; /* optional output, device int32 (B): per-sample Arnoldi
                                  steps of this call (as purin_cp_last_adjoint_iterations;
                                  the dense adjoint writes its BiCGSTAB iterations) */
} purin_cp_adjoint_options;

void purin_cp_default_adjoint_options(purin_cp_adjoint_options* opts);

/* Compute entry points, for purin_cp_workspace_bytes. */
enum purin_cp_entry {
  PURIN_CP_ENTRY_SPMM = 0,
  PURIN_CP_ENTRY_SOLVE = 1,
  PURIN_CP_ENTRY_PROJECT = 2,          /* also purin_cp_project_noalloc */
  PURIN_CP_ENTRY_PROJECT_VALUES = 3,
  PURIN_CP_ENTRY_QP_SOLVE = 4,
  PURIN_CP_ENTRY_DENSE_SOLVE = 5,
  PURIN_CP_ENTRY_ADJOINT = 6,
  PURIN_CP_ENTRY_ADJOINT_VALUES = 7,
  PURIN_CP_ENTRY_QP_ADJOINT = 8,
  PURIN_CP_ENTRY_DENSE_ADJOINT = 9
};

/*
 * Bytes of caller workspace an entry point needs for ``batch`` samples: the
 * largest over its optional arguments (a NULL ``saved``, whose state then
 * lives in the workspace; warm-start multipliers or duals; a dual cotangent).
 * For the adjoints ``adjoint_opts`` gives the GMRES restart length (NULL: the
 * defaults).  Returns -1 for an invalid plan, entry or batch (message in
 * purin_cp_last_error).  No reference counterpart (XLA sizes a custom call's
 * scratch from such a query); replaces the plan-owned workspace of the
 * jitted solve for callers that bring their own (bounds.py:33).
 */
int64_t purin_cp_workspace_bytes(const purin_cp_plan* plan, int32_t entry, int64_t batch,
                                 const purin_cp_adjoint_options* adjoint_opts);

/*
 * Implicit VJP at the state saved by project() (or solve()).
 *   target (B,n), rhs (B, me+mi) the same inputs as the forward call
 *   (for solve(): rhs (B, m) scaled); cot_y (B,n) cotangent of y.
 * Outputs g_target (B,n); g_rhs (B, me+mi) (for solve(): (B, m) scaled) or NULL;
 * g_lower, g_upper (B,n) or NULL (solve() only: gradients w.r.t. its bounds);
 * valid uint8 (B), info int32 (B) (0 converged, 1 not, 2 non-finite),
 * gmres_residual (B); each may be NULL.
 */
int purin_cp_adjoint(purin_cp_plan* plan, void* stream, int64_t batch, const void* saved,
                     const void* target, const void* rhs, const void* cot_y,
                     const purin_cp_adjoint_options* opts, void* g_target, void* g_rhs,
                     void* g_lower, void* g_upper, uint8_t* valid, int32_t* info,
                     void* gmres_residual);

/*
 * Implicit VJP at the state saved by purin_cp_project_values(), with the
 * same values (B, nnz).  The adjoint's steps are per sample, from each
 * sample's scaled matrix (bounds.py:83-101).  Outputs as purin_cp_adjoint()
 * plus g_values (B, nnz): the gradient w.r.t. values in the plan's CSR entry
 * order, through the VJP of cp_step w.r.t. the scaled coefficients
 * (bounds.py:109-141), the row scaling and the bound thresholds
 * (bounds.py:192-236).  Each output may be NULL.
 */
int purin_cp_adjoint_values(purin_cp_plan* plan, void* stream, int64_t batch, const void* saved,
                            const void* values, const void* cot_y,
                            const purin_cp_adjoint_options* opts, void* g_target, void* g_rhs,
                            void* g_values, uint8_t* valid, int32_t* info,
                            void* gmres_residual);

/*
 * Implicit VJP of purin_cp_qp_solve (the custom_vjp bwd of
 * diagonal_qp.py:131-219) at its saved state, with the same q, c and values
 * (NULL when the forward used the plan's).  cot_y (B, n); cot_dual (B, me+mi)
 * cotangent of the multipliers, or NULL.  Outputs (each may be NULL): g_q,
 * g_c (B, n); g_values (B, nnz); g_rhs (B, me+mi); g_lower, g_upper (B, n);
 * valid, info, gmres_residual (B).  The row scales are constants of the
 * derivative (stop_gradient, diagonal_qp.py:252-256).
 */
int purin_cp_qp_adjoint(purin_cp_plan* plan, void* stream, int64_t batch, const void* saved,
                        const void* q, const void* c, const void* values, const void* cot_y,
                        const void* cot_dual, const purin_cp_adjoint_options* opts, void* g_q,
                        void* g_c, void* g_values, void* g_rhs, void* g_lower, void* g_upper,
                        uint8_t* valid, int32_t* info, void* gmres_residual);

/*
 * The dense layer's backward (dense_implicit.py:160-210 with
 * autodiff/fixed_point.py:8-40) at the state saved by purin_cp_dense_solve:
 * BiCGSTAB (jax.scipy.sparse.linalg.bicgstab, jax 0.6.2) on
 * (I - J_z^T) v = [cot_y, cot_dual, 0] over the whole batch as one vector,
 * tolerance opts->tolerance (the reference uses 1e-6) and at most
 * opts->max_iterations iterations (adjoint_iters, 50 there), with the step
 * sizes and the prox inverse frozen -- so g_q is zero -- and no convergence
 * masking.  Outputs (each may be NULL): g_q, g_c (B, n); g_values (B, nnz);
 * g_rhs (B, me+mi); g_lower, g_upper (B, n).  purin_cp_last_adjoint_stats
 * reports the BiCGSTAB iterations (arnoldi_steps) and its final counter
 * (cycles: the iterations, or -10 / -11 at a breakdown).
 */
int purin_cp_dense_adjoint(purin_cp_plan* plan, void* stream, int64_t batch, const void* saved,
                           const void* q, const void* c, const void* values, const void* cot_y,
                           const void* cot_dual, const purin_cp_adjoint_options* opts, void* g_q,
                           void* g_c, void* g_values, void* g_rhs, void* g_lower,
                           void* g_upper);

/* Work done by the last adjoint() call on this plan.  No reference counterpart
 * (the reference's GMRES returns only per-sample info codes); it reports how
 * many batched Arnoldi steps ran, which sets the adjoint's algorithmic bytes. */
typedef struct {
  int64_t arnoldi_steps;  /* Arnoldi steps run over all restart cycles (the batch
                             steps together until its last active sample stops) */
  int32_t cycles;         /* restart cycles started */
  int32_t reserved;
} purin_cp_adjoint_stats;

int purin_cp_last_adjoint_stats(const purin_cp_plan* plan, purin_cp_adjoint_stats* stats);

/* Per-sample Arnoldi steps (summed over restart cycles) of the last GMRES
 * adjoint call (adjoint / adjoint_values / qp_adjoint) on this plan: the
 * reference's row_iterations, _batched_restarted_gmres(..., return_iterations=True)
 * (src/purin/solvers/primal_dual_interior_point/operators.py:1092-1097, 1121-1123).
 * Copies ``batch`` int32 values (batch must be that call's) into the device
 * array ``iterations``, stream-ordered on ``stream``.  The values live in the
 * plan's adjoint workspace until its next adjoint call. */
int purin_cp_last_adjoint_iterations(const purin_cp_plan* plan, void* stream, int64_t batch,
                                     int32_t* iterations);

/* Message of the calling thread's last error ("" if none). */
const char* purin_cp_last_error(void);

/* Build identification (ABI version, offload target). */
const char* purin_cp_build_info(void);

#ifdef __cplusplus
}
#endif

#endif /* PURIN_CP_H */
