// Argument block shared by the generic chunk kernels (ews_diag.hip) and the plane pair-group kernels
// (ews_pairs.hip): shapes, the chunk plan and every device pointer of one forward or backward call.
#pragma once

#include <stddef.h>

namespace ews {

// ------------------------------------------------------------------------------------------- arguments
struct DiagArgs {
  int B, L, n_int, d, K;  // K: planes (complex) or channels (real)
  int N, flow_mode, readout;
  int T, C;               // chunk length, chunk count
  int scan_cb;            // chunks per LDS-staged block in the float64 scans
  int kb;                 // checkpoint block (steps) of the recomputing adjoint, <= kBLK
  int W, off1, off2, lvl0, D, npar;
  int path_bf16;
  int sq1, sq2;           // series order of the level-1 / level-2 local terms (0: exact closed forms)
  const void* path;
  const float* clock;
  const float* params;
  float* out;
  const float* gout;
  // residual
  double* carries;  // (B, C+1, D)
  int* argmax;      // (B, W)
  // workspace
  float* summ;      // (B, C, D)
  float* mu;        // (B, C, D)
  float* mt;        // (B, C, D)
  float* red;       // (B, C, W)
  int* red_idx;     // (B, C, W)
  float* dv;        // (B, n_int, d)
  float* dh;        // (B, n_int)
  float* gp;        // (B, C, npar)
  float* gph;       // (B, C)
  double* gpart;    // (kParamBlocks, npar) partial parameter sums
  double* gagg;     // (B, NG, D) group aggregates (forward) / group cotangent aggregates (backward)
  double* gcar;     // (B, NG, D) state before each group (forward) / cotangent after each group (backward)
  int NG;           // chunk groups of scan_cb chunks
  // per-chunk clock classification (residual): bit 0 = uniform (the pair-group kernels own the chunk),
  // bit 1 = the steps may be inverted backwards; and the chunk's mean clock step
  int* cflag;       // (B, C)
  float* chbar;     // (B, C)
  float* ctab;      // pair-group coefficient table at one reference step (residual)
  int fast_ok;      // 1 if this configuration has pair-group kernels (flags are valid), else 0
  // quad carry scan of the pair-group path (quads of four chunks)
  int NQ;           // quads per sample
  float* qagg;      // (B, NQ, D) quad summaries (forward) / quad adjoint aggregates (backward)
  double* qflow;    // (B, NQ, K, 2) quad flows exp(u tau_quad)
  double* ql1;      // (B, NQ, K, 2) level-1 increments of the quads (backward)
  double* cflow;    // (B, C, K, 2) chunk flows exp(u tau_chunk)
  // look-back of the pair-group forward (one workgroup per quad, a sample's quads in ticket order): status words
  // (0 nothing, 1 published) of every (sample, quad), then of every (sample, group of 8 quads), then one ticket
  // counter per sample (32 words apart); the quad aggregates, then the group aggregates (state D, then the K plane
  // flows), float64
  int* lbflag;      // (B NQ + B NG + 32 B)
  double* lbagg;    // (B NQ + B NG, D + 2K)
  // LogEWS rows written by the chunk kernels' output pass (log-prefix readout off the sequential kernels): the
  // forward writes rows of Wlog = d + d (d - 1) / 2 floats (level 1, then the level-2 Lyndon coefficients) to out
  // and level 1 of every step to s1rows; the backward turns the log cotangent into the flat-row cotangent gcot
  // (layout W = D, no level 0) and runs on that
  int log, Wlog;
  float* s1rows;    // (B, n_int, d) level 1 of every step (residual)
  float* gcot;      // (B, n_int, D) flat-row cotangent (backward workspace)
  // per-sample sequential kernels (real diagonal, ews_seq.hip)
  float* seqck;     // (B, blocks, lanes + K) state checkpoints (residual; null: the forward keeps none)
  float* seqgp;     // (B, K) per-sample parameter partials (backward)
  // backward outputs
  float* dpath;
  float* dclock;
  float* dparams;
};

}  // namespace ews
