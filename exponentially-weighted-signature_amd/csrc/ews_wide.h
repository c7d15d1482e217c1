// Dense generators with 16 < d <= 32 at depths 1-2 (csrc/ews_wide.hip): arguments of the kernels and the host
// entry points that ews_dense_* calls for such a descriptor.
#pragma once

#include <stddef.h>
#include <stdint.h>

#include "ews_hip.h"

namespace ews {
namespace wide {

struct WArgs {
  int B, L, n, d, N, T, C, W, lvl0, readout;
  int TL, NSL, CP;  // leaf adjoint: intervals per slice, slices per sample; CP = max(C, NSL)
  int flow_mode, chen, leaf, q, vm, vl_expm, vl_mode;
  const float* path;
  const float* clock;
  const float* A;
  float* out;
  // forward workspace (padded 32 x 32 matrices, rows of 32 + 32 x 32 floats)
  float* fl;    // flows: per interval (B, n) or per sample (B)
  float* vlm;   // Van Loan (P, V): per interval or per sample
  float* loc;   // local terms (B, n)
  float* summ;  // chunk summaries (B, C)
  float* sfl;   // chunk flow products (B, C)
  float* car;   // carries (B, C + 1): the state before each chunk, then the final state
  float* rows;  // padded prefix states (B, n), for the backward
  float* rpart;  // mean / max readout: each chunk's sum or maximum of its padded rows (B, C)
  int* ridx;     // max readout: the first row attaining each chunk's maximum (B, C)
  int* amax;    // max readout: row of the maximum per (sample, column)
  // backward workspace
  const float* gout;  // the readout's cotangent (packed rows of W)
  float* mu;     // each chunk's own cotangent on its carry-in state (B, C)
  float* lend;   // cotangent on each chunk's end state from the later chunks (B, C)
  float* dloc;   // local-term cotangents (B, n)
  float* dfl;    // per-interval flow cotangents (B, n)
  float* cpart;  // per-chunk sums of the shared flow's cotangent and per-slice sums of the Van Loan pair's (B, CP, 3)
  float* dvlm;   // per-interval Van Loan pair cotangents (B, n, 2)
  float* apart;  // dA partials of the workgroups
  float* dv;     // increment cotangents (B, n, 32)
  float* dhl;    // series leaf's clock-step cotangents (B, n)
  float* dhm;    // per-interval matrix functions' clock-step cotangents (B, n, 2): flow, Van Loan
  float* dsh;    // shared steps' cotangents (B, 2): flow, Van Loan
  // power series of the per-interval matrix functions
  float* apow;   // A^0 .. A^PW (padded, float), ||A||_1 and the Van Loan knots' coefficients phi[m][k]
  int* mflag;    // per interval: bit 0 the flow, bit 1 the Van Loan pair outside the series radius, bit 2 the
                 // Van Loan knots by the M-step chain (M |c| ||A||_1 outside the radius)
  int* sflag;    // per sample (uniform modes): bit 0 the shared flow, bit 1 the shared pair outside the series radius
  float* hpart;  // the adjoint's sums H_k = sum gamma_k c^k dOut per workgroup
  double* hsum;  // H_k summed over the workgroups
  float* ubuf;   // series-path knots: u_k = A^k w per interval (B, n, PW + 1, 32)
  float* ebuf;   // their cotangents e_k = sum_m phi[m][k] dDelta_m (B, n, PW + 1, 32)
};

// The descriptor takes this path: 16 < d <= 32, depth 1 or 2, leaf series or van_loan.
bool eligible(const ews_dense_desc* s);
size_t workspace_bytes(const ews_dense_desc* s, bool backward);
int forward(const ews_dense_desc* s, const float* path, const float* clock, const float* A, float* out,
            void* workspace, bool backward_layout, hipStream_t st);
// kept: the workspace holds what forward(.., backward_layout = true, ..) wrote for the same inputs (the step
// matrices, local terms, chunk summaries and carries, padded prefix states and the maxima's rows); else the backward
// runs that forward first
int backward(const ews_dense_desc* s, const float* path, const float* clock, const float* A, const float* grad_out,
             float* grad_path, float* grad_clock, float* grad_A, void* workspace, bool kept, hipStream_t st);

}  // namespace wide
}  // namespace ews
