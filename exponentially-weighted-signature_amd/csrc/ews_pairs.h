// Host entry points of the plane pair-group kernels (ews_pairs.hip), called by the C ABI in ews_diag.hip.
#pragma once

#include <hip/hip_runtime.h>

#include "ews_args.h"

namespace ews {

constexpr int kMaxT = 64;  // longest chunk the pair-group kernels stage

// True if the configuration has pair-group kernels (rotation planes, d = 16, depth 2, prefix readout,
// per-interval flows, chunk length <= kMaxT).
bool pairs_eligible(int structure, int depth, int dim, int readout, int flow_mode, int T);
// Uniform chunks of the forward: summaries (out = false; this launch also writes every chunk's classification
// a.cflag / a.chbar, so it runs before any other kernel of the call) or prefix rows (out = true).
int pairs_forward(const DiagArgs& a, hipStream_t st, bool out);
// Uniform chunks of the backward: chunk-local adjoints (full = false) or the full adjoint (full = true).
int pairs_backward(const DiagArgs& a, hipStream_t st, bool full);

}  // namespace ews
