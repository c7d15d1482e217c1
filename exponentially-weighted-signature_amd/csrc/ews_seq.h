// Host entry points of the per-sample sequential kernels (ews_seq.hip), called by the C ABI in ews_diag.hip.
#pragma once

#include <hip/hip_runtime.h>

#include "ews_args.h"

namespace ews {

constexpr int kSeqCB = 16;    // steps per staged block and between checkpoints
constexpr int kSeqMaxK = 32;  // widest real diagonal

// lanes per workgroup (one per level-2 pair, rows of 32 lanes) and checkpoint blocks per sample
__host__ __device__ inline int seq_threads(int K) { return ((K * 32 + 63) / 64) * 64; }
__host__ __device__ inline int seq_blocks(int n_int) { return (n_int + kSeqCB - 1) / kSeqCB; }
// floats of one sample's checkpoints: per block the level-2 state of every lane and the level-1 state
__host__ __device__ inline size_t seq_ckpt_floats(int K, int n_int) { return (size_t)seq_blocks(n_int) * (seq_threads(K) + K); }

// dynamic LDS of the backward: two staging buffers of 8 cotangent rows of W floats
inline size_t seq_bwd_lds_bytes(int W) { return (size_t)2 * 8 * W * 4; }

// Forward: prefix rows (a.readout EWS_READOUT_PREFIX) or LogEWS rows (EWS_READOUT_LOGPREFIX); writes the
// checkpoints a.seqck when it is not null.
int seq_forward(const DiagArgs& a, hipStream_t st);
// Backward from the forward's checkpoints: a.dpath, a.dclock (if not null), per-sample parameter partials a.seqgp,
// then a.dparams.
int seq_backward(const DiagArgs& a, hipStream_t st);

}  // namespace ews
