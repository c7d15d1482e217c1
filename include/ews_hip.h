/* C ABI of the MI355X EWS Chen-scan library (libews_mi355x.so).
 *
 * The entry points replace the combine/leaf stage behind the reference layer `EWS._single_path`
 * (ews/layer.py:154-265): the leaf `local_signatures` (ews/core/leaf.py:50-198), the flows
 * `_chen_M_per_interval` (ews/core/chen_scan.py:155-168) and the Chen combine `combine_packed`
 * (ews/core/kernels/combine.py:193-269) / `chen_associative_scan_prefix_packed_with_M` (chen_scan.py:172-214),
 * together with the custom VJPs of the Pallas kernels (ews/core/kernels/pallas_combine.py:1673-1801).
 *
 * Conventions: every pointer is device memory owned by the caller; nothing here allocates; all work is
 * stream-ordered on `stream`; the calls are re-entrant (no global mutable state), except
 * `ews_diag_forward_noalloc`, whose scratch is one fixed device array per GPU: its calls that overlap on one GPU
 * race. Sign convention is the reference's: the flow over a clock step h is exp(-h A).
 */
#ifndef EWS_HIP_H
#define EWS_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* ews_stream_t; /* hipStream_t */

/* return codes */
#define EWS_OK 0
#define EWS_ERR_NULL (-1)      /* a required pointer is NULL */
#define EWS_ERR_SHAPE (-2)     /* batch/length/dim out of range */
#define EWS_ERR_DEPTH (-3)     /* depth not supported by this structure */
#define EWS_ERR_OPTION (-4)    /* unknown structure / flow mode / readout / dtype */
#define EWS_ERR_LAUNCH (-5)    /* a kernel launch failed */
#define EWS_ERR_SCRATCH (-6)   /* ews_diag_forward_noalloc: the call needs more than its fixed scratch (64 MiB) */

/* generator structure */
#define EWS_STRUCT_PLANES 1    /* rotation planes A_j = [[d_j, w_j], [-w_j, d_j]] on channels (2j, 2j+1) */
#define EWS_STRUCT_REAL_DIAG 2 /* A = diag(lambda) */

/* flows M_t = exp(-h A) (chen_scan.py:155-168): per interval, or one shared flow (cached) */
#define EWS_FLOW_PER_INTERVAL 0       /* reweighting_mode "displacement" */
#define EWS_FLOW_CACHED 1             /* "displacement_uniform": every interval uses dtheta[0] */
#define EWS_FLOW_CACHED_BASEPOINT 2   /* "displacement_uniform_basepoint": dtheta[1], interval 0 = I */

/* readouts (ews/layer.py:189-265) */
#define EWS_READOUT_PREFIX 0   /* (B, L-1, W) */
#define EWS_READOUT_TERMINAL 1 /* (B, W) */
#define EWS_READOUT_MEAN 2     /* (B, W) */
#define EWS_READOUT_MAX 3      /* (B, W) */
/* LogEWS prefix rows (ews/layer.py:488-517 with readout "prefix"): per prefix row the compressed log
 * signature, level 1 then S2[a,b] - S1_a S1_b / 2 at the Lyndon words a < b in lexicographic order (real
 * coordinates; a rotation plane j is coordinates 2j, 2j+1), (B, L-1, d + d(d-1)/2), no level-0 column (level0
 * is ignored). Depth 2, any structure and flow mode. The scan's output pass writes these rows; the flat rows never
 * reach memory. A real diagonal with d <= 32 and per-interval flows runs on the per-sample sequential kernels when
 * chunk 0 selects them (B >= 128 and L <= 1025, as for flat rows) or EWS_CHUNK_SEQUENTIAL asks for them; every other
 * case on the chunk kernels, whose residual then also keeps level 1 of every step and whose backward workspace
 * holds one flat-row cotangent per step. */
#define EWS_READOUT_LOGPREFIX 4

/* ews_diag_desc.chunk: 0 selects the kernels and chunk length; EWS_CHUNK_SEQUENTIAL asks for the per-sample
 * sequential kernels (one workgroup per sample, the whole sequence in one pass; real diagonal, depth 2, d <= 32,
 * prefix or log-prefix readout, per-interval flows), which chunk 0 also selects for B >= 128 and L <= 1025. */
#define EWS_CHUNK_SEQUENTIAL (-1)

#define EWS_DTYPE_F32 0
#define EWS_DTYPE_BF16 1

typedef struct ews_diag_desc {
  int32_t batch;      /* B >= 1 */
  int32_t length;     /* L >= 2 knots (L-1 intervals) */
  int32_t dim;        /* d: even for planes (d <= 64), real diagonal d <= 32 */
  int32_t depth;      /* N in {1, 2} (closed-form local terms exist for depths 1-2) */
  int32_t structure;  /* EWS_STRUCT_* */
  int32_t flow_mode;  /* EWS_FLOW_* */
  int32_t readout;    /* EWS_READOUT_* */
  int32_t level0;     /* 1: rows carry the leading level-0 constant (the "flat" format), 0: packed */
  int32_t path_dtype; /* EWS_DTYPE_F32 or EWS_DTYPE_BF16 */
  int32_t chunk;      /* intervals per chunk; 0 selects the default; EWS_CHUNK_SEQUENTIAL: one chunk per sample */
  int32_t leaf;       /* EWS_DIAG_LEAF_* (0: the exact closed forms) */
  int32_t series_q;   /* series order q in [1, 40] of the series leaves (letters b_0..b_q, total order |m| <= q) */
} ews_diag_desc;

/* local terms of the plane / diagonal path (ews/core/leaf.py:99-175). The flows exp(-h A) are exact in all three. */
#define EWS_DIAG_LEAF_CLOSED 0       /* "plane_closed" (ews/core/kernels/plane_engine.py:134-152): exact integrals */
#define EWS_DIAG_LEAF_BLOCK_SERIES 1 /* "block_series" (blockdiag_engine.py:88-155): exact level 1, order-q series at
                                        level 2 (series_q may be 0 at depth 1) */
#define EWS_DIAG_LEAF_SERIES 2       /* "series" (series_leaf.py:116-126): the order-q series at every level */

/* Scratch the forward/backward need between launches (chunk summaries, carries, partial reductions).
 * Replaces the XLA-side chunk scan of pallas_combine.py:1395-1422. */
size_t ews_diag_workspace_bytes(const ews_diag_desc* desc);

/* Residual the forward leaves for the backward: float64 chunk-start states (B, C+1, D) and, for the max
 * readout, int32 argmax (B, W). Replaces the custom-VJP residuals of pallas_combine.py:1684-1697. */
size_t ews_diag_residual_bytes(const ews_diag_desc* desc);

/* Forward: path (B, L, d) [f32 or bf16], clock (B, L) f32, params f32 [planes: (d/2, 2) rows (d_j, w_j);
 * real diagonal: (d,)], out f32 [(B, L-1, W) for prefix, (B, W) otherwise], W = level0 + sum_k d^k.
 * Replaces local_signatures + combine_packed + the readout of EWS._single_path (ews/layer.py:172-265). */
int ews_diag_forward(const ews_diag_desc* desc, const void* path, const float* clock, const float* params,
                     float* out, void* residual, void* workspace, ews_stream_t stream);

/* Backward: cotangent grad_out shaped like out; writes grad_path (B, L, d) f32, grad_clock (B, L) f32 and
 * grad_params (same shape as params). grad_clock may be NULL when the clock needs no gradient (a data clock, as
 * JAX prunes an undifferentiated input): its terms are then skipped. Replaces the custom VJP _cvjp_bwd
 * (pallas_combine.py:1698-1798) and JAX autodiff through the leaf (plane_engine.py:134-152). */
int ews_diag_backward(const ews_diag_desc* desc, const void* path, const float* clock, const float* params,
                      const void* residual, const float* grad_out, float* grad_path, float* grad_clock,
                      float* grad_params, void* workspace, ews_stream_t stream);

/* One pass of ews_diag_forward (pass 0 chunk summaries, 1 float64 carry scan over chunks, 2 chunk outputs,
 * 3 mean/max reduction); running passes 0..ews_diag_num_passes(0)-1 in order is ews_diag_forward. A pass that
 * does not apply to the readout launches nothing. For callers that place each kernel in its own custom call
 * or time kernels separately. Replaces pass 1 / the XLA chunk scan / pass 3 of pallas_combine.py:1395-1422. */
int ews_diag_forward_pass(const ews_diag_desc* desc, int pass, const void* path, const float* clock,
                          const float* params, float* out, void* residual, void* workspace, ews_stream_t stream);

/* One pass of ews_diag_backward (0 chunk-local adjoints, 1 float64 reverse adjoint scan, 2 full chunk adjoints,
 * 3 knot gradients, 4 parameter reduction). Replaces B1 / B2 / B3 of pallas_combine.py:1698-1798. */
int ews_diag_backward_pass(const ews_diag_desc* desc, int pass, const void* path, const float* clock,
                           const float* params, const void* residual, const float* grad_out, float* grad_path,
                           float* grad_clock, float* grad_params, void* workspace, ews_stream_t stream);

/* Number of passes: direction 0 = forward, 1 = backward. */
int ews_diag_num_passes(int direction);

/* The forward's status word, after ews_diag_forward on `stream` (this call waits for the stream): *status is 0,
 * or 1 when a chunk carry of the one-launch look-back forward waited on an earlier quad's aggregate past its spin
 * limit and was set to NaN (the prefix rows of that sample from there on are NaN). Always 0 for configurations
 * without the look-back forward. No counterpart in the reference (XLA reports no such condition); it lets a
 * caller or a test tell a look-back timeout from a numerical NaN. */
int ews_diag_forward_status(const ews_diag_desc* desc, const void* residual, int* status, ews_stream_t stream);

/* ews_diag_forward without a residual or workspace argument and without any allocation: no counterpart in the
 * reference. For callers that cannot allocate device memory: code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc. Its scratch (the forward's float64 carries, chunk summaries and group carries)
 * is a fixed 64 MiB device array that every GPU the library runs on holds until the process ends; calls whose
 * scratch exceeds it return EWS_ERR_SCRATCH (c2 and c5 fit; the c4 shape at B = 256 does not). The stream must
 * belong to the current device. Every call on one GPU shares that GPU's array: calls that overlap in time on one
 * GPU (several streams, several host threads) race and must be serialised by the caller. The output equals
 * ews_diag_forward's bit for bit; the residual it would leave is not kept for a backward. */
int ews_diag_forward_noalloc(const ews_diag_desc* desc, const void* path, const float* clock, const float* params,
                             float* out, ews_stream_t stream);

/* ---------------------------------------------------------------------------------------------------------
 * Dense generators: any d x d matrix A (d <= 16), depths 1-3, the series leaf (ews/core/series_leaf.py).
 * Flows M_t = exp(-h_t A) are evaluated in the kernels (Taylor polynomial on a scaled argument, then
 * squarings), replacing _chen_M_per_interval (ews/core/chen_scan.py:155-168) with chen_expm="exact".
 * --------------------------------------------------------------------------------------------------------- */
/* leaves of the dense path (ews/core/leaf.py:50-198) */
#define EWS_LEAF_SERIES 0   /* series_local_signatures (ews/core/series_leaf.py:116-126) */
#define EWS_LEAF_VAN_LOAN 1 /* reweighted_segments_van_loan + compute_reweighted_signatures (van_loan.py:163-184) */
/* block_series (ews/core/leaf.py:138-175, ews/core/kernels/blockdiag_engine.py:88-155): the exact level 1
 * G v, G = int_0^1 exp(-s h A) ds at any step, and the series leaf's order-series_q level 2 (depths 1 and 2; on a
 * block-diagonal A the blockwise letters are the letters of A) */
#define EWS_LEAF_BLOCK_SERIES 2

/* matrix exponential schemes (ews/core/expm_approx.py:13-41) */
#define EWS_EXPM_EXACT 0
#define EWS_EXPM_EULER 1
#define EWS_EXPM_CAYLEY 2
#define EWS_EXPM_PADE 3 /* the [2/2] Pade approximant ("pade", "pade_lite") */

typedef struct ews_dense_desc {
  int32_t batch;     /* B >= 1 */
  int32_t length;    /* L >= 2 knots */
  int32_t dim;       /* 1 <= d <= 16; or 16 < d <= 32 at depths 1-2 with the series or Van Loan leaf (ews_dense_forward,
                      * ews_dense_backward and their _keep / _kept forms; the other dense entry points take d <= 16) */
  int32_t depth;     /* N in {1, 2, 3} */
  int32_t series_q;  /* series order q in [0, 40] (letters b_0..b_q, total order |m| <= q); series leaf only */
  int32_t flow_mode; /* EWS_FLOW_* of the Chen flows */
  int32_t readout;   /* EWS_READOUT_* (mean / max need level0 = 1) */
  int32_t level0;    /* 1: rows carry the leading level-0 constant */
  int32_t chunk;     /* intervals per chunk; 0 selects the default (64) */
  int32_t leaf;      /* EWS_LEAF_* (0: series) */
  int32_t vl_steps;  /* Van Loan leaf: knots per interval M, 1 <= M <= 64 (the layer's M) */
  int32_t vl_expm;   /* Van Loan leaf: EWS_EXPM_* of the augmented exponential (the layer's van_loan_expm) */
  int32_t vl_mode;   /* Van Loan leaf: reweighting as EWS_FLOW_* (displacement / uniform / uniform_basepoint) */
  int32_t chen_expm; /* EWS_EXPM_* of the flows M_t (the layer's chen_expm; 0: exact) */
} ews_dense_desc;

/* Scratch of the dense forward: powers table, padded local terms and flows (B, L-1, 16+256+4096 | 256),
 * chunk summaries and carries, and the per-sample step matrices of the uniform modes (B, 3, 256). For d > 16:
 * the step matrices padded to 32 x 32 (per interval or per sample), local terms (B, L-1, 32 + 1024), chunk
 * summaries, flow products and carries. */
size_t ews_dense_workspace_bytes(const ews_dense_desc* desc);

/* Forward: path (B, L, d) f32, clock (B, L) f32, A (d, d) f32 row-major (reference sign), out f32
 * [(B, L-1, W) for prefix, (B, W) otherwise], W = level0 + sum_k d^k. Replaces EWS._single_path for a dense A
 * with leaf="series" (series_local_signatures, ews/core/series_leaf.py:116-126) or leaf="van_loan"
 * (reweighted_segments_van_loan, ews/core/van_loan.py:163-184, and the knot signatures of
 * ews/core/signature.py:20-35), the flows and the combine (ews/core/chen_scan.py:155-241;
 * ews/core/kernels/pallas_combine.py:803-858 dense_kernel) and the readout (ews/layer.py:189-265). */
int ews_dense_forward(const ews_dense_desc* desc, const float* path, const float* clock, const float* A,
                      float* out, void* workspace, ews_stream_t stream);

/* One pass of ews_dense_forward: 0 local terms + flows, 1 chunk summaries, 2 carry scan, 3 outputs. */
int ews_dense_forward_pass(const ews_dense_desc* desc, int pass, const float* path, const float* clock,
                           const float* A, float* out, void* workspace, ews_stream_t stream);
int ews_dense_num_passes(void);

/* The leaf alone: levels (B, L-1, sum_k d^k) packed as ews/core/chen_scan.py:33-46 and flows (B, L-1, d, d).
 * Replaces local_signatures(kind="series" | "van_loan") (ews/core/leaf.py:86-114) plus _chen_M_per_interval. */
int ews_dense_local_terms(const ews_dense_desc* desc, const float* path, const float* clock, const float* A,
                          float* levels, float* flows, void* workspace, ews_stream_t stream);

/* The combine alone on given levels (B, L-1, sum_k d^k) and flows (B, L-1, d, d), with the readout of desc.
 * Replaces combine_packed(kind="dense_kernel") (ews/core/kernels/combine.py:259-269 ->
 * pallas_combine.py:2628 dense_general_prefix_vjp forward). */
int ews_dense_combine(const ews_dense_desc* desc, const float* levels, const float* flows, float* out,
                      void* workspace, ews_stream_t stream);

/* Scratch of the dense backward entry points: the forward's buffers (with the prefix rows) and the adjoint
 * scan's per-chunk cotangents and carries. */
size_t ews_dense_backward_workspace_bytes(const ews_dense_desc* desc);

/* Backward of ews_dense_forward: given the cotangent grad_out of out, writes grad_path (B, L, d), grad_clock (B, L)
 * (may be NULL) and grad_A (d, d). Recomputes the forward up to the chunk carries, runs the combine's adjoint (as
 * ews_dense_combine_backward), then the leaf's and the flows' adjoints per interval and one reduction for grad_A.
 * Replaces JAX autodiff through the leaf (series_local_signatures, ews/core/series_leaf.py:72-126, or
 * reweighted_segments_van_loan + the knot signatures, ews/core/van_loan.py:31-160 and ews/core/signature.py:20-35)
 * and _chen_M_per_interval (ews/core/chen_scan.py:155-168, every chen_expm scheme) around the dense kernel's custom
 * VJP (ews/core/kernels/pallas_combine.py:2360-2565). */
int ews_dense_backward(const ews_dense_desc* desc, const float* path, const float* clock, const float* A,
                       const float* grad_out, float* grad_path, float* grad_clock, float* grad_A, void* workspace,
                       ews_stream_t stream);

/* The same forward and backward with the forward's intermediates kept for the backward instead of recomputed;
 * the residuals a custom VJP keeps between its two halves (pallas_combine.py:2360-2565) are here the leaf, the
 * flows, the chunk summaries and carries: about B (L-1) (sum_k d^k + 256) floats, 1.2 GB at c3's shape (for
 * 16 < d <= 32 also the padded prefix states, 32 x 33 floats per interval, and the per-interval step matrices).
 * ews_dense_forward_keep is ews_dense_forward on a workspace of ews_dense_backward_workspace_bytes(desc) bytes;
 * ews_dense_backward_kept is ews_dense_backward on that workspace, unchanged since, with the same desc and inputs:
 * it skips the recompute (at c3, 1.3 ms of the backward) and overwrites the kept data (one backward per forward).
 * out is the forward's output, unchanged since, or NULL: with the prefix readout at d = 16 its rows are the states
 * the adjoint needs, which it then reads instead of recomputing them (0.36 ms at c3). */
int ews_dense_forward_keep(const ews_dense_desc* desc, const float* path, const float* clock, const float* A,
                           float* out, void* workspace, ews_stream_t stream);
int ews_dense_backward_kept(const ews_dense_desc* desc, const float* path, const float* clock, const float* A,
                            const float* out, const float* grad_out, float* grad_path, float* grad_clock,
                            float* grad_A, void* workspace, ews_stream_t stream);

/* Backward of ews_dense_combine: given the cotangent grad_out of out, writes grad_levels (B, L-1, sum_k d^k) and
 * grad_flows (B, L-1, d, d). Replaces the custom VJP of dense_general_prefix_vjp (the dense kernel's
 * _dense_kernel_general_bwd, ews/core/kernels/pallas_combine.py:2360-2565, and _cvjp_bwd :1698-1798): a local
 * reverse scan per chunk, a reverse scan of the chunk carries over the chunk summaries, and a reverse scan per
 * chunk from its carry that emits the cotangents (the max readout's cotangent goes to the first row attaining
 * the maximum). */
int ews_dense_combine_backward(const ews_dense_desc* desc, const float* levels, const float* flows,
                               const float* grad_out, float* grad_levels, float* grad_flows, void* workspace,
                               ews_stream_t stream);

/* Backward of ews_dense_local_terms: the cotangents grad_levels (B, L-1, sum_k d^k) and grad_flows (B, L-1, d, d)
 * -> grad_path (B, L, d), grad_clock (B, L) (may be NULL) and grad_A (d, d). Workspace:
 * ews_dense_backward_workspace_bytes. Replaces JAX autodiff through local_signatures + _chen_M_per_interval
 * (ews/core/leaf.py:86-114, ews/core/chen_scan.py:155-168), as build_token_cache (ews/core/token_scan.py:44-88)
 * needs it for the per-token segments. */
int ews_dense_local_terms_backward(const ews_dense_desc* desc, const float* path, const float* clock, const float* A,
                                   const float* grad_levels, const float* grad_flows, float* grad_path,
                                   float* grad_clock, float* grad_A, void* workspace, ews_stream_t stream);

/* Token-cached scan (ews/core/token_scan.py:91-118): desc as for ews_dense_combine with length = steps + 1; step t
 * of sample b uses P_cache[g] (vocab, sum_k d^k) and D_cache[g] (vocab, d, d) for g = token_ids[b, t] (clamped to
 * [0, vocab)); a step with mask[b, t] == 0 is the unit signature with the identity flow (mask may be NULL). */
size_t ews_token_scan_workspace_bytes(const ews_dense_desc* desc, int vocab);
int ews_token_scan(const ews_dense_desc* desc, const int32_t* token_ids, const uint8_t* mask, const float* P_cache,
                   const float* D_cache, int vocab, float* out, void* workspace, ews_stream_t stream);
/* Backward: grad_out -> grad_P_cache (vocab, sum_k d^k) and grad_D_cache (vocab, d, d), the per-step cotangents
 * summed by token in a fixed order (deterministic). Replaces JAX autodiff through token_cached_prefix_scan.
 * The workspace holds per-512-step partial sums for every token: about ceil(B (L-1) / 512) x vocab x
 * (sum_k d^k + 256) floats beside the scan's own (70 MB at B = 256, L = 512, d = 16, depth 2, vocab 128; 0.6 GB at
 * depth 3), and the cotangent stream is read once per group of 16 tokens. */
int ews_token_scan_backward(const ews_dense_desc* desc, const int32_t* token_ids, const uint8_t* mask,
                            const float* P_cache, const float* D_cache, int vocab, const float* grad_out,
                            float* grad_P_cache, float* grad_D_cache, void* workspace, ews_stream_t stream);

/* ---------------------------------------------------------------------------------------------------------
 * Jordan chains: the closed-form local terms of the leaves jordan_closed / jordan_closed_tables
 * (ews/core/kernels/jordan_engine.py:324-353) for a block-diagonal A of uniform Jordan chains, exact at any clock
 * step: a real chain of size n is lambda I + eps Nil (lambda = A[f][f], eps = A[f][f+1]); a complex chain of size 2k
 * is c = a + ib (a = A[f][f], b = A[f+1][f]) on the coordinates v_2i + i v_2i+1 with eps = A[f][f+2] coupling them.
 * Level 1 is sum_p (-h)^p phi^(p)(-h c) / p! (eps Nil)^p v and level 2 the pair integrals' derivatives
 * D^(p,q) (jordan_engine.py:175-321), evaluated in float64 on the device. The flows and the combine are those of
 * the dense family (ews_dense_local_terms / ews_dense_combine and their backward).
 * --------------------------------------------------------------------------------------------------------- */
#define EWS_JORDAN_REAL 0    /* chain sizes 2, 3, 4 (size 1: a real diagonal) */
#define EWS_JORDAN_COMPLEX 1 /* chain sizes 4, 6, 8: 2, 3, 4 complex coordinates (size 2: rotation planes, the
                                closed forms of ews/core/kernels/plane_engine.py:134-152) */

typedef struct ews_jordan_desc {
  int32_t batch;  /* B >= 1 */
  int32_t length; /* L >= 2 knots */
  int32_t dim;    /* d = chains x size, d <= 16, at most 8 chains */
  int32_t depth;  /* N in {1, 2} */
  int32_t kind;   /* EWS_JORDAN_REAL or EWS_JORDAN_COMPLEX */
  int32_t size;   /* chain size in real coordinates */
} ews_jordan_desc;

/* Local terms: path (B, L, d) f32, clock (B, L) f32, A (d, d) f32 row-major (reference sign) -> levels
 * (B, L-1, d [+ d*d]) f32 packed (level 1, then level 2 row-major; ews/core/chen_scan.py:33-46). Replaces
 * jordan_engine.local_terms (ews/core/kernels/jordan_engine.py:324-353) behind ews/core/leaf.py:177-198. */
int ews_jordan_local_terms(const ews_jordan_desc* desc, const float* path, const float* clock, const float* A,
                           float* levels, ews_stream_t stream);

/* Scratch of ews_jordan_local_terms_backward: per-interval dv, dh and chain-parameter partials. */
size_t ews_jordan_workspace_bytes(const ews_jordan_desc* desc);

/* Backward: grad_levels (B, L-1, d [+ d*d]) -> grad_path (B, L, d), grad_clock (B, L) (may be NULL) and grad_A
 * (d, d), all written (not accumulated); grad_A is nonzero only at the entries the chains are read from. The
 * per-interval parameter partials are summed in a fixed order (deterministic). Replaces JAX autodiff through
 * jordan_engine.local_terms. */
int ews_jordan_local_terms_backward(const ews_jordan_desc* desc, const float* path, const float* clock,
                                    const float* A, const float* grad_levels, float* grad_path, float* grad_clock,
                                    float* grad_A, void* workspace, ews_stream_t stream);

/* ---------------------------------------------------------------------------------------------------------
 * Depth-1 scan of a block-diagonal A of uniform chains, any number of chains (chain d/size <= 64): the EWS at
 * N = 1 (ews/layer.py:154-265 with leaf jordan_closed, series, van_loan or block_series, whose level 1 is the
 * exact phi(-hA) v or its order-q truncation) under exact flows, which for a chain are the closed form of
 * jordan_block_operators (ews/core/kernels/combine.py:143-190; with jordan_flows or chen_expm "exact"). Chains as
 * in ews_jordan_desc: real chains of 1-4 coordinates (size 1: a real diagonal), complex chains of 1-4 complex
 * coordinates (size 2: rotation planes). Everything per chain in float64; chunk carries in float64.
 * --------------------------------------------------------------------------------------------------------- */
typedef struct ews_chain_desc {
  int32_t batch;     /* B >= 1 */
  int32_t length;    /* L >= 2 knots */
  int32_t dim;       /* d = chains x size */
  int32_t kind;      /* EWS_JORDAN_REAL or EWS_JORDAN_COMPLEX */
  int32_t size;      /* chain size in real coordinates: real 1-4; complex 2, 4, 6, 8 */
  int32_t flow_mode; /* EWS_FLOW_* of the flows (chen_scan.py:155-168) */
  int32_t leaf_mode; /* EWS_FLOW_* of the leaf's clock step: per interval, or van_loan's uniform modes
                        (van_loan.py:147-160: one shared step; basepoint: interval 0 has none) */
  int32_t readout;   /* EWS_READOUT_PREFIX (B, L-1, W) or EWS_READOUT_TERMINAL (B, W), W = level0 + d */
  int32_t level0;    /* 1: the leading level-0 column of the flat format */
  int32_t series_q;  /* 0: the exact level 1 phi(-hA) v; 1..48: the series leaf's order-q truncation */
  int32_t chunk;     /* intervals per chunk, 0: 32; at most 64 */
} ews_chain_desc;

/* Residual the forward leaves for the backward: the float64 chunk carries (B, C+1, chains, coordinates). */
size_t ews_chain_residual_bytes(const ews_chain_desc* desc);
/* Scratch of both directions: chunk summaries, adjoint carries, per-interval dv and dh, parameter partials. */
size_t ews_chain_workspace_bytes(const ews_chain_desc* desc);

/* Forward: path (B, L, d) f32, clock (B, L) f32, A (d, d) f32 row-major (reference sign; the chains' parameters
 * are read from A[f][f], A[f+1][f] and A[f][f+1] / A[f][f+2], f each chain's first row, as
 * jordan_engine.local_terms reads them) -> out. Replaces local_signatures + combine_packed at N = 1 for these
 * generators (ews/core/leaf.py:50-198, ews/core/kernels/combine.py:193-269). */
int ews_chain_forward(const ews_chain_desc* desc, const void* path, const float* clock, const float* A, float* out,
                      void* residual, void* workspace, ews_stream_t stream);

/* Backward: grad_out shaped like out -> grad_path (B, L, d), grad_clock (B, L) (may be NULL) and grad_A (d, d),
 * written; grad_A is nonzero only at the entries each chain is read from (the chain parameters' gradients, summed
 * in a fixed order). Replaces JAX autodiff through the leaf and jordan_block_operators and the custom VJP of the
 * block kernel (pallas_combine.py:1673-1801). */
int ews_chain_backward(const ews_chain_desc* desc, const void* path, const float* clock, const float* A,
                       const void* residual, const float* grad_out, float* grad_path, float* grad_clock,
                       float* grad_A, void* workspace, ews_stream_t stream);

/* ---------------------------------------------------------------------------------------------------------
 * Token-cached scan at depth 1 for any width up to 64 (ews/core/token_scan.py:91-118 with trunc 1): from dense
 * per-token caches, P_cache (V, d) the level 1 of each token's segment and D_cache (V, d, d) its flow,
 * S_t = D_{g_t} S_{t-1} + P_{g_t} from S = 0; a padded step (mask 0) keeps the state (D = I, unit signature).
 * --------------------------------------------------------------------------------------------------------- */
typedef struct ews_token1_desc {
  int32_t batch; /* B >= 1 */
  int32_t steps; /* n >= 1 scan steps (tokens) per sample */
  int32_t dim;   /* d: 1..64 */
  int32_t vocab; /* V >= 1; ids are clamped to [0, V) */
  int32_t block; /* 0: dense flows; BS in {1, 2, 3, 4, 6, 8} (d % BS == 0, V (BS + 1) <= 64): every flow is
                    block-diagonal with blocks of BS consecutive coordinates (the chain-structured caches); entries
                    outside the blocks are taken as zero and their gradients written as zero */
} ews_token1_desc;

/* Scratch of both directions: dense flows, a transposed flow cache, every step's cotangent and per-chunk token
 * partials; block-diagonal flows, the per-sample token partials. */
size_t ews_token1_workspace_bytes(const ews_token1_desc* desc);

/* tokens (B, n) int32, mask (B, n) uint8 or NULL, caches f32 -> out (B, n, d) f32, the packed prefix states
 * (no level-0 column). Replaces token_cached_prefix_scan (ews/core/token_scan.py:91-118) at trunc 1. */
int ews_token1_scan(const ews_token1_desc* desc, const int32_t* tokens, const uint8_t* mask, const float* P_cache,
                    const float* D_cache, float* out, void* workspace, ews_stream_t stream);

/* Backward: the forward's out (its states) and grad_out (B, n, d) -> grad_P (V, d), grad_D (V, d, d), written,
 * summed over every step carrying the token in a fixed order (deterministic). Replaces JAX autodiff through the
 * scan's gather (token_scan.py:104-118). */
int ews_token1_scan_backward(const ews_token1_desc* desc, const int32_t* tokens, const uint8_t* mask,
                             const float* P_cache, const float* D_cache, const float* out, const float* grad_out,
                             float* grad_P, float* grad_D, void* workspace, ews_stream_t stream);

/* ---------------------------------------------------------------------------------------------------------
 * Log-signature readout of LogEWS (ews/layer.py:440-556): per state row the truncated tensor log and its
 * coefficients at the Lyndon words (signax.signature_to_logsignature), then the readout (log-then-pool).
 * --------------------------------------------------------------------------------------------------------- */
typedef struct ews_log_desc {
  int32_t batch;   /* B >= 1 */
  int32_t rows;    /* R state rows per sample (L-1 prefix rows, or 1 for the terminal readout) */
  int32_t dim;     /* d: 1..64 (1..16 at depth 3) */
  int32_t depth;   /* N in {1, 2, 3} */
  int32_t level0;  /* 1: the rows carry the leading level-0 column */
  int32_t readout; /* EWS_READOUT_*: prefix (B, R, Dlog), terminal / mean / max (B, Dlog) */
} ews_log_desc;

/* Dlog = sum_k W_d(k), the Witt numbers (ews/layer.py:417-425). */
int ews_log_dim(int dim, int depth);
size_t ews_log_workspace_bytes(const ews_log_desc* desc);

/* rows (B, R, level0 + sum_k d^k) of EWS states -> out. Replaces the vmapped
 * signax.signature_to_logsignature and the pooling of LogEWS._single_path (ews/layer.py:488-517). */
int ews_log_forward(const ews_log_desc* desc, const float* sig_rows, float* out, void* workspace,
                    ews_stream_t stream);

/* Cotangent of the rows (level-0 column zero) for the cotangent grad_out of out. */
int ews_log_backward(const ews_log_desc* desc, const float* sig_rows, const float* grad_out, float* grad_rows,
                     void* workspace, ews_stream_t stream);

/* ---------------------------------------------------------------------------------------------------------
 * Mixer epilogue of an EWS block (ews/block.py:282-306, 336-357, 405-408; ews/norms.py:47-134): the prefix
 * rows' levels without the level-0 column, an optional leading zero row, the optional binomial prescale, the
 * per-level GradedRMSNorm and the c_down linear map, fused in one pass over the rows.
 * --------------------------------------------------------------------------------------------------------- */
#define EWS_GRADED_LIVE_RMS 0    /* g_k x_k / (RMS_k + eps_k) */
#define EWS_GRADED_STATIC_GAIN 1 /* g_k x_k */
#define EWS_GRADED_DILATION 2    /* lam^k x_k */

typedef struct ews_mixer_desc {
  int32_t batch;    /* B >= 1 */
  int32_t rows;     /* R scan rows per sample (>= 1) */
  int32_t dim;      /* d: 1..64 (1..16 at depth 3) */
  int32_t depth;    /* N in {1, 2, 3} */
  int32_t level0;   /* 1: the rows carry the leading level-0 column (the flat EWS output) */
  int32_t hidden;   /* output width of c_down (>= 1) */
  int32_t variant;  /* EWS_GRADED_* */
  int32_t prepend;  /* 1: the levels start with a zero row (ews/block.py:304-305): out has R + 1 rows */
  int32_t prescale; /* 1: level k of levels row t scaled by 1 / C(max(t + 1, k), k) (graded_prescale="binomial") */
  float eps[3];     /* live_rms floors per level */
} ews_mixer_desc;

/* Residual saved by the forward for the backward: per scan row, each level's products with its c_down block,
 * its total scale and the two derivative factors. */
size_t ews_mixer_residual_bytes(const ews_mixer_desc* desc);

/* rows (B, R, level0 + D) -> out (B, R + prepend, hidden) = c_down(graded(prescale(levels))). weight
 * (hidden, D) row-major and bias (hidden,) are c_down's (eqx.nn.Linear); gains are GradedRMSNorm.gains (N,) or,
 * for the dilation variant, lam (1,). Replaces jax.vmap(self.c_down)(self.graded(levels)) of
 * EWSBlock.mixer_levels / _forward (ews/block.py:405-406) after _mixer_levels / _prescale. */
int ews_mixer_forward(const ews_mixer_desc* desc, const float* rows, const float* weight, const float* bias,
                      const float* gains, float* out, void* residual, ews_stream_t stream);

/* Backward: the cotangent grad_out of out -> grad_rows (B, R, level0 + D) (level-0 column zero; the input of the
 * scan's backward) and row_dots (B, R, N), the dot product of each level's c_down products with the row's
 * cotangent. The parameter gradients follow from these on the host: grad_bias = sum of grad_out, grad_gains =
 * sum over rows of row_dots times the residual's gain factor, grad_weight[:, level k] = sum over rows of
 * (scale_k grad_out) (x) level k (a plain GEMM). */
int ews_mixer_backward(const ews_mixer_desc* desc, const float* rows, const float* weight, const void* residual,
                       const float* grad_out, float* grad_rows, float* row_dots, ews_stream_t stream);

/* ews_mixer_backward that also forms c_down's weight gradient in the same pass over the rows: grad_weight (hidden,
 * D) = sum over rows of (scale_k grad_out) (x) level k, accumulated per chunk of 512 rows on MFMA into the
 * workspace and summed in chunk order (float64, deterministic). hidden <= 128 (EWS_ERR_SHAPE above);
 * workspace of ews_mixer_backward_workspace_bytes (0 for an invalid descriptor or hidden > 128). grad_bias and
 * grad_gains follow from grad_out and row_dots on the host as above. Replaces the same backward as
 * ews_mixer_backward together with c_down's weight cotangent (eqx.nn.Linear's, ews/block.py:405-406). */
size_t ews_mixer_backward_workspace_bytes(const ews_mixer_desc* desc);
int ews_mixer_backward_weight(const ews_mixer_desc* desc, const float* rows, const float* weight,
                              const void* residual, const float* grad_out, float* grad_rows, float* row_dots,
                              float* grad_weight, void* workspace, ews_stream_t stream);

/* 1 when ews_diag_forward runs this configuration on the chunk kernels (where ews_diag_mixer_forward applies), 0
 * otherwise (the pair-group planes, the per-sample sequential kernels, an invalid descriptor). No counterpart in
 * the reference: it tells a caller which route of the block's epilogue to take. */
int ews_diag_uses_chunk_kernels(const ews_diag_desc* desc);

/* The scan of ews_diag_forward (prefix readout) with the mixer epilogue in its output pass: the levels of each
 * prefix row go straight from the scan into GradedRMSNorm and c_down, so that out (B, L-1 + prepend, hidden) and the
 * mixer's residual (as ews_mixer_forward's, ews_mixer_residual_bytes of mdesc) are written and the D-wide prefix
 * rows never are. mdesc describes the same rows (batch B, rows L-1, dim, depth). The scan's residual and workspace
 * are ews_diag_forward's. Runs where the scan runs on the chunk kernels (the configurations that are neither the
 * d = 16 pair-group planes nor the per-sample sequential kernels); elsewhere it returns EWS_ERR_OPTION and the
 * caller composes ews_diag_forward and ews_mixer_forward. hidden <= 64. The backward: the prefix rows regenerated
 * by ews_diag_forward_pass (pass 2) from the same residual, then ews_mixer_backward_weight and ews_diag_backward.
 * Replaces EWSBlock._mixer_levels followed by c_down(graded(...)) (ews/block.py:282-306, 405-408). */
int ews_diag_mixer_forward(const ews_diag_desc* desc, const ews_mixer_desc* mdesc, const void* path,
                           const float* clock, const float* params, const float* weight, const float* bias,
                           const float* gains, float* out, void* mixer_residual, void* residual, void* workspace,
                           ews_stream_t stream);

/* ---------------------------------------------------------------------------------------------------------
 * Front of an EWS block: the clock theta (ews/clocks.py) and the lifted path p (ews/params.py:1165-1191,
 * ews/block.py:284-301, ews/paths.py:126-131), computed from the block's raw inputs on the device.
 * --------------------------------------------------------------------------------------------------------- */
#define EWS_CLOCK_TIME 0           /* "time" */
#define EWS_CLOCK_VARIATION 1      /* "blended_variation", "blended_learn" */
#define EWS_CLOCK_QUAD_VARIATION 2 /* "blended_quad_variation" */
#define EWS_CLOCK_TOKEN_GATED 3    /* "token_gated": relu(w . dx - b) */
#define EWS_CLOCK_CLAMPED_GATE 4   /* "clamped_gate": sum_k clip(w_k . dx - b_k, 0, 1) */

#define EWS_SCALING_NONE 0  /* "none" */
#define EWS_SCALING_UNIT 1  /* "[0,1]" */
#define EWS_SCALING_SYM 2   /* "[-1,1]" */
#define EWS_SCALING_STEPS 3 /* "steps" (time mode only) */

typedef struct ews_clock_desc {
  int32_t batch;            /* B >= 1 */
  int32_t length;           /* L >= 1 rows per sample */
  int32_t channels;         /* c: driver channels, 1..64 (unused by EWS_CLOCK_TIME) */
  int32_t mode;             /* EWS_CLOCK_* */
  int32_t scaling;          /* EWS_SCALING_* */
  int32_t normalize;        /* 0 "per_sample", 1 "constant" */
  int32_t gates;            /* rows K of the gate weight: 1 (token_gated) or 1..8 (clamped_gate) */
  int32_t has_mask;         /* 1: mask (B, L) of prefix-structured validity bytes */
  int32_t increment_driver; /* 1: driver rows are increments; the clock's driver is their masked cumulative sum */
  int32_t has_time_denominator;
  int32_t basepoint;        /* 1: theta gets a leading copy of its first row (ews/block.py:298): (B, L + 1) */
  int32_t learned_alpha;    /* 1: alpha is params[0] (blended_learn, after its clip or sigmoid) */
  float alpha;              /* blended modes: the weight of the time component when learned_alpha == 0 */
  float norm_constant;      /* "constant" normalisation (and the gated modes' divisor) */
  float time_denominator;
  float variation_eps;      /* sqrt(|dx|^2 + eps) of blended_variation */
  float in_scale;           /* gated modes: the driver's fixed factor before the difference */
} ews_clock_desc;

/* Residual of the forward kept for the backward (per-chunk increment sums, row counts). */
size_t ews_clock_residual_bytes(const ews_clock_desc* desc);
/* Scratch of the backward. */
size_t ews_clock_workspace_bytes(const ews_clock_desc* desc);
/* Number of floats in params / grad_params: 1 (learned alpha), K c + K (gated: w row-major, then b), else 0. */
int ews_clock_num_params(const ews_clock_desc* desc);

/* times (L,) shared by the batch, driver (B, L, c), mask (B, L) -> theta (B, L + basepoint). Replaces
 * Clock.__call__ (FixedClock / GatedClock / LearnableBlendedClock, ews/clocks.py:393-533) on every sample, i.e.
 * build_clock_jnp (ews/clocks.py:164-267) and GatedClock.__call__ (:443-466). */
int ews_clock_forward(const ews_clock_desc* desc, const float* times, const float* driver, const uint8_t* mask,
                      const float* params, float* theta, void* residual, ews_stream_t stream);

/* Backward: grad_theta (B, L + basepoint) -> grad_driver (B, L, c) (may be NULL) and grad_params (the layout of
 * params; d theta / d alpha for a learned alpha). stop_gradient is the caller's: it skips this call. */
int ews_clock_backward(const ews_clock_desc* desc, const float* times, const float* driver, const uint8_t* mask,
                       const float* params, const void* residual, const float* grad_theta, float* grad_driver,
                       float* grad_params, void* workspace, ews_stream_t stream);

#define EWS_LIFT_NONE 0     /* no B: p = u */
#define EWS_LIFT_FULL 1     /* p = u B^T, B (out_dim, in) */
#define EWS_LIFT_PRESERVE 2 /* preserve_first_channel: p = [u_0, u_{1:} B^T], B (out_dim - 1, in - 1) */

typedef struct ews_lift_desc {
  int32_t batch;      /* B >= 1 */
  int32_t length;     /* L >= 1 */
  int32_t branch_dim; /* H: branch channels, 1..64 */
  int32_t append;     /* 1: u = [theta_app | branch] (the appended clock channel) */
  int32_t out_dim;    /* w: path channels, 1..64 (H + append without a lift) */
  int32_t lift;       /* EWS_LIFT_* */
  int32_t increment;  /* 1: path_mode "increment": the branch becomes its masked cumulative sum */
  int32_t has_mask;   /* 1: forward fill of p past the last real row */
  int32_t basepoint;  /* 1: a zero row in front: p (B, L + 1, w) */
} ews_lift_desc;

size_t ews_lift_residual_bytes(const ews_lift_desc* desc);
size_t ews_lift_workspace_bytes(const ews_lift_desc* desc);

/* branch (B, L, H), theta_app (B, L) (append only), mask (B, L), matrix (B's weight) -> path (B, L + basepoint, w).
 * Replaces the path half of EWSBlock._mixer_levels (ews/block.py:284-301) with B.__call__ (ews/params.py:1181-1191)
 * and, for path_mode "increment", to_increment_path_jnp (ews/paths.py:126-131) on the branch. */
int ews_lift_forward(const ews_lift_desc* desc, const float* branch, const float* theta_app, const uint8_t* mask,
                     const float* matrix, float* path, void* residual, ews_stream_t stream);

/* Backward: grad_path -> grad_branch (B, L, H), grad_theta_app (B, L) (append only) and grad_matrix (the shape of
 * matrix; lift != NONE). */
int ews_lift_backward(const ews_lift_desc* desc, const float* branch, const float* theta_app, const uint8_t* mask,
                      const float* matrix, const void* residual, const float* grad_path, float* grad_branch,
                      float* grad_theta_app, float* grad_matrix, void* workspace, ews_stream_t stream);

/* Human-readable text of a return code. */
const char* ews_error_string(int code);

/* Library version, "major.minor.patch". */
const char* ews_version(void);

#ifdef __cplusplus
}
#endif

#endif /* EWS_HIP_H */
