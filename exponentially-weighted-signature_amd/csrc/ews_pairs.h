// Host entry points of the plane pair-group kernels (ews_pairs.hip), called by the C ABI in ews_diag.hip.
#pragma once

#include <hip/hip_runtime.h>

#include "ews_args.h"

namespace ews {

constexpr int kMaxT = 64;  // longest chunk the pair-group kernels stage
// coefficient table of the pair-group kernels: header (16 floats), 9 complex per plane, 16 complex per pair
constexpr int kCoefTabFloats = 16 + 2 * 9 * 8 + 2 * 16 * 64;
// header word (an int) set to 1 by the look-back forward when a wait gave up (its rows are NaN), else 0
constexpr int kCtabStatus = 3;

// True if the configuration has pair-group kernels (rotation planes, d = 16, depth 2, prefix readout,
// per-interval flows, chunk length <= kMaxT).
bool pairs_eligible(int structure, int depth, int dim, int readout, int flow_mode, int T);
// The forward: the coefficient table a.ctab and the look-back words zeroed (out = false; runs before any other
// kernel of the call), or the look-back forward (out = true): every chunk's classification (a.cflag / a.chbar),
// the float64 carries (a.carries) and the prefix rows, in one launch.
int pairs_forward(const DiagArgs& a, hipStream_t st, bool out);
// Float64 adjoint carry scan over quads of four chunks; the full-adjoint kernels rebuild the carries inside each
// quad.
int pairs_carry_scan(const DiagArgs& a, hipStream_t st);
// Uniform chunks of the backward: chunk-local adjoints (full = false) or the full adjoint (full = true).
int pairs_backward(const DiagArgs& a, hipStream_t st, bool full);

}  // namespace ews
