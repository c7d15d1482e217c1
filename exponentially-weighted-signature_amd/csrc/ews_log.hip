// The log-signature readout of LogEWS on MI355X: per state row the truncated tensor log and its coefficients at
// the Lyndon words, then the readout, and the backward of both.
//
// Reference: LogEWS._single_path (ews/layer.py:488-517) applies signax.signature_to_logsignature (signax 0.2.1, not
// vendored) to the terminal row or to every prefix row, then pools (log-then-pool). With X = S - 1 (levels 1..N):
//   log S = X - X (x) X / 2 + X (x) X (x) X / 3 - ...,  level by level (truncated at N):
//   L1 = S1,  L2 = S2 - S1 (x) S1 / 2,  L3 = S3 - (S1 (x) S2 + S2 (x) S1) / 2 + S1 (x) S1 (x) S1 / 3,
// and the compressed log keeps each level's coefficients at its Lyndon words (each length in lexicographic order,
// as Duval's algorithm generates them; ews/layer.py:417-425 sizes the levels by them).
#include <hip/hip_runtime.h>

#include "ews_hip.h"

namespace ews {
namespace logsig {

struct LArgs {
  int B, R, d, N, lvl0, W, Dlog, readout;
  const float* rows;  // (B, R, W) state rows: optional level-0 column, then levels 1..N
  float* out;         // (B, R, Dlog) for prefix, (B, Dlog) otherwise
  int* words;         // (Dlog, 4): length, letters
  float* logs;        // (B, R, Dlog) per-row logs of the mean / max readouts
  int* amax;          // (B, Dlog) first row of the maximum (max readout)
};

// Lyndon words of lengths 1..N over {0..d-1}, Duval's algorithm (one thread); off[k]: first word of length k + 1.
__global__ void k_lyndon(int* words, int d, int N, int off1, int off2) {
  if (threadIdx.x != 0 || blockIdx.x != 0) return;
  int w[3] = {-1, 0, 0};
  int len = 1;
  int cnt[3] = {0, off1, off2};
  while (len > 0) {
    w[len - 1] += 1;
    int* o = words + 4 * cnt[len - 1]++;
    o[0] = len;
    o[1] = w[0];
    o[2] = len > 1 ? w[1] : 0;
    o[3] = len > 2 ? w[2] : 0;
    const int m = len;
    while (len < N) {
      w[len] = w[len - m];
      ++len;
    }
    while (len > 0 && w[len - 1] == d - 1) --len;
  }
}

// log coefficient of word wd on the row (levels 1..N, no level-0 column)
__device__ __forceinline__ float log_coef(const float* s, const int* wd, int d) {
  const int len = wd[0], i = wd[1], j = wd[2], k = wd[3];
  const float* S2 = s + d;
  const float* S3 = S2 + d * d;
  if (len == 1) return s[i];
  if (len == 2) return fmaf(-0.5f * s[i], s[j], S2[i * d + j]);
  const float half = 0.5f * (s[i] * S2[j * d + k] + S2[i * d + j] * s[k]);
  return fmaf((1.0f / 3.0f) * s[i] * s[j], s[k], S3[(i * d + j) * d + k] - half);
}

// per-row logs: one workgroup per (row, sample); the prefix / terminal readouts write out, mean / max write logs
__global__ __launch_bounds__(256) void k_logrows(LArgs a) {
  const int r = blockIdx.x, b = blockIdx.y;
  const float* s = a.rows + ((size_t)b * a.R + r) * a.W + a.lvl0;
  const bool pool = a.readout == EWS_READOUT_MEAN || a.readout == EWS_READOUT_MAX;
  float* o = (pool ? a.logs : a.out) + ((size_t)b * a.R + r) * a.Dlog;
  for (int w = threadIdx.x; w < a.Dlog; w += blockDim.x) o[w] = log_coef(s, a.words + 4 * w, a.d);
}

// mean / max over the rows, per coefficient (first row of the maximum kept for the backward)
__global__ void k_logpool(LArgs a) {
  const int b = blockIdx.y;
  const int w = blockIdx.x * blockDim.x + threadIdx.x;
  if (w >= a.Dlog) return;
  const float* p = a.logs + (size_t)b * a.R * a.Dlog + w;
  if (a.readout == EWS_READOUT_MEAN) {
    float acc = 0.0f;
    for (int r = 0; r < a.R; ++r) acc += p[(size_t)r * a.Dlog];
    a.out[(size_t)b * a.Dlog + w] = acc / (float)a.R;
  } else {
    float best = p[0];
    int arg = 0;
    for (int r = 1; r < a.R; ++r) {
      const float v = p[(size_t)r * a.Dlog];
      if (v > best) {
        best = v;
        arg = r;
      }
    }
    a.out[(size_t)b * a.Dlog + w] = best;
    a.amax[(size_t)b * a.Dlog + w] = arg;
  }
}

// Backward, one workgroup per (row, sample): the row's cotangent gw of its log coefficients (by readout), then
//   level 3 words (i,j,k): dS3[ijk] = g, dS1[i] -= g S2[jk]/2 - g S1[j] S1[k]/3, dS2[jk] -= g S1[i]/2,
//                          dS2[ij] -= g S1[k]/2, dS1[k] -= g S2[ij]/2 - g S1[i] S1[j]/3, dS1[j] += g S1[i] S1[k]/3
//   level 2 words (i,j):   dS2[ij] += g, dS1[i] -= g S1[j]/2, dS1[j] -= g S1[i]/2
//   level 1 words (i):     dS1[i] += g
// (LDS atomics for levels 1-2; the level-3 entries outside the words and the level-0 column are zero).
__global__ __launch_bounds__(256) void k_logrows_bwd(LArgs a, const float* gout, float* grows) {
  extern __shared__ float acc[];  // d + d*d
  const int r = blockIdx.x, b = blockIdx.y, d = a.d;
  const float* s = a.rows + ((size_t)b * a.R + r) * a.W + a.lvl0;
  float* gr = grows + ((size_t)b * a.R + r) * a.W;
  const int D12 = d + (a.N >= 2 ? d * d : 0);
  for (int e = threadIdx.x; e < D12; e += blockDim.x) acc[e] = 0.0f;
  if (a.N >= 3) {
    for (int e = threadIdx.x; e < d * d * d; e += blockDim.x) gr[a.lvl0 + D12 + e] = 0.0f;
  }
  if (a.lvl0 && threadIdx.x == 0) gr[0] = 0.0f;
  __syncthreads();
  const float* S2 = s + d;
  for (int w = threadIdx.x; w < a.Dlog; w += blockDim.x) {
    float g;
    if (a.readout == EWS_READOUT_PREFIX) g = gout[((size_t)b * a.R + r) * a.Dlog + w];
    else if (a.readout == EWS_READOUT_TERMINAL) g = gout[(size_t)b * a.Dlog + w];
    else if (a.readout == EWS_READOUT_MEAN) g = gout[(size_t)b * a.Dlog + w] / (float)a.R;
    else g = a.amax[(size_t)b * a.Dlog + w] == r ? gout[(size_t)b * a.Dlog + w] : 0.0f;
    const int* wd = a.words + 4 * w;
    const int len = wd[0], i = wd[1], j = wd[2], k = wd[3];
    if (len == 1) {
      atomicAdd(&acc[i], g);
    } else if (len == 2) {
      atomicAdd(&acc[d + i * d + j], g);
      atomicAdd(&acc[i], -0.5f * g * s[j]);
      atomicAdd(&acc[j], -0.5f * g * s[i]);
    } else {
      gr[a.lvl0 + D12 + (i * d + j) * d + k] = g;
      const float t3 = g * (1.0f / 3.0f);
      atomicAdd(&acc[i], fmaf(t3, s[j] * s[k], -0.5f * g * S2[j * d + k]));
      atomicAdd(&acc[j], t3 * s[i] * s[k]);
      atomicAdd(&acc[k], fmaf(t3, s[i] * s[j], -0.5f * g * S2[i * d + j]));
      atomicAdd(&acc[d + j * d + k], -0.5f * g * s[i]);
      atomicAdd(&acc[d + i * d + j], -0.5f * g * s[k]);
    }
  }
  __syncthreads();
  for (int e = threadIdx.x; e < D12; e += blockDim.x) gr[a.lvl0 + e] = acc[e];
}

}  // namespace logsig
}  // namespace ews

// ================================================================================================= C ABI
namespace {

using namespace ews::logsig;

size_t al256l(size_t x) { return (x + 255) & ~(size_t)255; }

// Witt numbers by level (number of Lyndon words of each length), host Duval
void witt(int d, int N, int* sz) {
  sz[0] = sz[1] = sz[2] = 0;
  int w[3] = {-1, 0, 0}, len = 1;
  while (len > 0) {
    w[len - 1] += 1;
    ++sz[len - 1];
    const int m = len;
    while (len < N) {
      w[len] = w[len - m];
      ++len;
    }
    while (len > 0 && w[len - 1] == d - 1) --len;
  }
}

struct LPlan {
  int B, R, d, N, lvl0, W, Dlog, readout, sz[3];
  size_t words, logs, amax, total;
};

int log_plan(const ews_log_desc* s, LPlan& p) {
  if (!s) return EWS_ERR_NULL;
  if (s->depth < 1 || s->depth > 3) return EWS_ERR_DEPTH;
  if (s->readout < 0 || s->readout > 3) return EWS_ERR_OPTION;
  if (s->batch < 1 || s->rows < 1 || s->dim < 1 || s->dim > 64) return EWS_ERR_SHAPE;
  if (s->depth == 3 && s->dim > 16) return EWS_ERR_SHAPE;
  if (s->readout == EWS_READOUT_TERMINAL && s->rows != 1) return EWS_ERR_SHAPE;
  p.B = s->batch; p.R = s->rows; p.d = s->dim; p.N = s->depth; p.lvl0 = s->level0 ? 1 : 0;
  p.readout = s->readout;
  int D = 0;
  for (int k = 1, m = 1; k <= p.N; ++k) {
    m *= p.d;
    D += m;
  }
  p.W = D + p.lvl0;
  witt(p.d, p.N, p.sz);
  p.Dlog = p.sz[0] + p.sz[1] + p.sz[2];
  const bool pool = p.readout == EWS_READOUT_MEAN || p.readout == EWS_READOUT_MAX;
  size_t off = 0;
  p.words = off; off += al256l((size_t)p.Dlog * 4 * 4);
  p.logs = off; off += pool ? al256l((size_t)p.B * p.R * p.Dlog * 4) : 0;
  p.amax = off; off += al256l((size_t)p.B * p.Dlog * 4);
  p.total = off;
  return EWS_OK;
}

LArgs log_args(const LPlan& p, const float* rows, float* out, void* ws) {
  LArgs a{};
  a.B = p.B; a.R = p.R; a.d = p.d; a.N = p.N; a.lvl0 = p.lvl0; a.W = p.W; a.Dlog = p.Dlog; a.readout = p.readout;
  a.rows = rows; a.out = out;
  char* w = (char*)ws;
  a.words = (int*)(w + p.words); a.logs = (float*)(w + p.logs); a.amax = (int*)(w + p.amax);
  return a;
}

#define LOG_CHECK()                                            \
  do {                                                         \
    if (hipGetLastError() != hipSuccess) return EWS_ERR_LAUNCH; \
  } while (0)

}  // namespace

extern "C" {

int ews_log_dim(int dim, int depth) {
  if (dim < 1 || depth < 1 || depth > 3) return 0;
  int sz[3];
  witt(dim, depth, sz);
  return sz[0] + sz[1] + sz[2];
}

size_t ews_log_workspace_bytes(const ews_log_desc* desc) {
  LPlan p;
  if (log_plan(desc, p) != EWS_OK) return 0;
  return p.total;
}

int ews_log_forward(const ews_log_desc* desc, const float* sig_rows, float* out, void* workspace,
                    ews_stream_t stream) {
  LPlan p;
  const int rc = log_plan(desc, p);
  if (rc != EWS_OK) return rc;
  if (!sig_rows || !out || !workspace) return EWS_ERR_NULL;
  const LArgs a = log_args(p, sig_rows, out, workspace);
  hipStream_t st = (hipStream_t)stream;
  hipLaunchKernelGGL(k_lyndon, dim3(1), dim3(1), 0, st, a.words, p.d, p.N, p.sz[0], p.sz[0] + p.sz[1]);
  LOG_CHECK();
  hipLaunchKernelGGL(k_logrows, dim3(p.R, p.B), dim3(256), 0, st, a);
  LOG_CHECK();
  if (p.readout == EWS_READOUT_MEAN || p.readout == EWS_READOUT_MAX) {
    hipLaunchKernelGGL(k_logpool, dim3((p.Dlog + 255) / 256, p.B), dim3(256), 0, st, a);
    LOG_CHECK();
  }
  return EWS_OK;
}

int ews_log_backward(const ews_log_desc* desc, const float* sig_rows, const float* grad_out, float* grad_rows,
                     void* workspace, ews_stream_t stream) {
  LPlan p;
  const int rc = log_plan(desc, p);
  if (rc != EWS_OK) return rc;
  if (!sig_rows || !grad_out || !grad_rows || !workspace) return EWS_ERR_NULL;
  const LArgs a = log_args(p, sig_rows, nullptr, workspace);
  hipStream_t st = (hipStream_t)stream;
  // the word table (and, for max, the argmax) are the forward's, recomputed here so the call stands alone
  hipLaunchKernelGGL(k_lyndon, dim3(1), dim3(1), 0, st, a.words, p.d, p.N, p.sz[0], p.sz[0] + p.sz[1]);
  LOG_CHECK();
  if (p.readout == EWS_READOUT_MAX) {
    LArgs f = a;
    f.out = grad_rows;  // scratch for the pooled values: overwritten below
    hipLaunchKernelGGL(k_logrows, dim3(p.R, p.B), dim3(256), 0, st, f);
    LOG_CHECK();
    hipLaunchKernelGGL(k_logpool, dim3((p.Dlog + 255) / 256, p.B), dim3(256), 0, st, f);
    LOG_CHECK();
  }
  const size_t shm = (size_t)(p.d + (p.N >= 2 ? p.d * p.d : 0)) * 4;
  hipLaunchKernelGGL(k_logrows_bwd, dim3(p.R, p.B), dim3(256), shm, st, a, grad_out, grad_rows);
  LOG_CHECK();
  return EWS_OK;
}

}  // extern "C"
