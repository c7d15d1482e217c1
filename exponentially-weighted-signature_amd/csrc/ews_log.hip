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

// Lyndon words of lengths 1..3 over {0..d-1}, each length in lexicographic order, one thread per word. A word of
// length 2 is Lyndon iff i < j; of length 3 iff a <= b and a < c (a rotation starting with a smaller letter, or the
// rotation aab of aba, would be smaller otherwise). So the lexicographic rank of a word has a closed form:
//   (i, j):    i (2d - i - 1) / 2 + (j - i - 1)
//   (a, b, c): sum_{x < a} (d - x)(d - x - 1) + (b - a)(d - a - 1) + (c - a - 1),
// the same table Duval's algorithm generates (sorted by length).
__device__ __forceinline__ int widx2(int i, int j, int d) { return i * (2 * d - i - 1) / 2 + (j - i - 1); }
__device__ __forceinline__ int widx3(int a, int b, int c, int d) {
  const int m = d - a;  // sum_{x < a} (d - x)(d - x - 1) = ((d^3 - d) - (m^3 - m)) / 3
  return ((d * d * d - d) - (m * m * m - m)) / 3 + (b - a) * (m - 1) + (c - a - 1);
}
__global__ void k_words(int* words, int d, int n1, int n2, int Dlog) {
  const int w = blockIdx.x * blockDim.x + threadIdx.x;
  if (w >= Dlog) return;
  int len, i = 0, j = 0, k = 0;
  if (w < n1) {
    len = 1;
    i = w;
  } else if (w < n1 + n2) {
    len = 2;
    int q = w - n1;
    while (q >= d - 1 - i) q -= d - 1 - i++;
    j = i + 1 + q;
  } else {
    len = 3;
    int q = w - n1 - n2;
    while (q >= (d - i) * (d - i - 1)) {
      q -= (d - i) * (d - i - 1);
      ++i;
    }
    j = i + q / (d - i - 1);
    k = i + 1 + q % (d - i - 1);
  }
  int* o = words + 4 * w;
  o[0] = len;
  o[1] = i;
  o[2] = j;
  o[3] = k;
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

// per-row logs: one wavefront per (row, sample), four rows per workgroup (a workgroup per row left the chip
// scheduling tiny workgroups); the prefix / terminal readouts write out, mean / max write logs
__global__ __launch_bounds__(256) void k_logrows(LArgs a) {
  const int r = blockIdx.x * 4 + (threadIdx.x >> 6), b = blockIdx.y, lane = threadIdx.x & 63;
  if (r >= a.R) return;
  const float* s = a.rows + ((size_t)b * a.R + r) * a.W + a.lvl0;
  const bool pool = a.readout == EWS_READOUT_MEAN || a.readout == EWS_READOUT_MAX;
  float* o = (pool ? a.logs : a.out) + ((size_t)b * a.R + r) * a.Dlog;
  for (int w = lane; w < a.Dlog; w += 64) o[w] = log_coef(s, a.words + 4 * w, a.d);
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

// Backward, one wavefront per (row, sample). The row's word cotangents g (by readout) and its level 1 (and level 2
// at depth 3) are staged in LDS, then every entry of the row cotangent is gathered from the words that contain it:
//   dS1[x] = g(x) - 1/2 sum_{y != x} g(min(x,y), max(x,y)) S1[y]
//            + sum over words (x,b,c): g (S1[b] S1[c] / 3 - S2[bc] / 2)       (x first)
//            + sum over words (a,x,c): g S1[a] S1[c] / 3                       (x second)
//            + sum over words (a,b,x): g (S1[a] S1[b] / 3 - S2[ab] / 2)       (x last)
//   dS2[xy] = g(x,y) [x < y] - 1/2 sum over words (a,x,y) of g S1[a] - 1/2 sum over words (x,y,c) of g S1[c]
//   dS3[abc] = g(a,b,c) on the Lyndon words, 0 elsewhere; the level-0 column is 0.
// No atomics: each entry is written once, rows stream through with coalesced stores.
__global__ __launch_bounds__(256) void k_logrows_bwd(LArgs a, const float* gout, float* grows, int per) {
  // one wavefront per row, four rows per workgroup; per wavefront: g (Dlog) | S1 (d) | S2 (d*d, depth 3)
  extern __shared__ float sh[];
  const int wv = threadIdx.x >> 6;
  const int rw = blockIdx.x * 4 + wv, b = blockIdx.y, d = a.d, N = a.N, l = threadIdx.x & 63;
  const bool ok = rw < a.R;
  const int r = ok ? rw : 0;  // rows past the end read row 0, write nothing and leave after the barrier
  float* g = sh + wv * per;
  float* s1 = g + a.Dlog;
  float* s2 = s1 + d;
  const float* s = a.rows + ((size_t)b * a.R + r) * a.W + a.lvl0;
  for (int w = l; w < a.Dlog; w += 64) {
    float v;
    if (a.readout == EWS_READOUT_PREFIX) v = gout[((size_t)b * a.R + r) * a.Dlog + w];
    else if (a.readout == EWS_READOUT_TERMINAL) v = gout[(size_t)b * a.Dlog + w];
    else if (a.readout == EWS_READOUT_MEAN) v = gout[(size_t)b * a.Dlog + w] / (float)a.R;
    else v = a.amax[(size_t)b * a.Dlog + w] == r ? gout[(size_t)b * a.Dlog + w] : 0.0f;
    g[w] = v;
  }
  for (int e = l; e < d; e += 64) s1[e] = s[e];
  if (N >= 3)
    for (int e = l; e < d * d; e += 64) s2[e] = s[d + e];
  __syncthreads();
  if (!ok) return;
  const int n1 = d, n12 = d + (N >= 2 ? d * (d - 1) / 2 : 0);
  float* gr = grows + ((size_t)b * a.R + r) * a.W;
  if (a.lvl0 && l == 0) gr[0] = 0.0f;
  gr += a.lvl0;
  for (int x = l; x < d; x += 64) {
    float v = g[x];
    if (N >= 2) {
      float t = 0.0f;
      for (int y = 0; y < d; ++y)
        if (y != x) t = fmaf(g[n1 + (x < y ? widx2(x, y, d) : widx2(y, x, d))], s1[y], t);
      v = fmaf(-0.5f, t, v);
    }
    if (N >= 3) {
      for (int p = 0; p < d; ++p) {
        for (int q = 0; q < d; ++q) {
          if (p >= x && q > x)  // (x, p, q)
            v += g[n12 + widx3(x, p, q, d)] * fmaf((1.0f / 3.0f) * s1[p], s1[q], -0.5f * s2[p * d + q]);
          if (p <= x && q > p)  // (p, x, q)
            v += g[n12 + widx3(p, x, q, d)] * ((1.0f / 3.0f) * s1[p] * s1[q]);
          if (p < x && q >= p)  // (p, q, x)
            v += g[n12 + widx3(p, q, x, d)] * fmaf((1.0f / 3.0f) * s1[p], s1[q], -0.5f * s2[p * d + q]);
        }
      }
    }
    gr[x] = v;
  }
  if (N >= 2) {
    for (int e = l; e < d * d; e += 64) {
      const int x = e / d, y = e - x * d;
      float v = x < y ? g[n1 + widx2(x, y, d)] : 0.0f;
      if (N >= 3) {
        float t = 0.0f;
        for (int c = 0; c < d; ++c) {
          if (c <= x && c < y) t = fmaf(g[n12 + widx3(c, x, y, d)], s1[c], t);  // (c, x, y)
          if (x <= y && x < c) t = fmaf(g[n12 + widx3(x, y, c, d)], s1[c], t);  // (x, y, c)
        }
        v = fmaf(-0.5f, t, v);
      }
      gr[d + e] = v;
    }
  }
  if (N >= 3) {
    for (int e = l; e < d * d * d; e += 64) {
      const int x = e / (d * d), y = (e / d) % d, z = e % d;
      gr[d + d * d + e] = (x <= y && x < z) ? g[n12 + widx3(x, y, z, d)] : 0.0f;
    }
  }
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
  hipLaunchKernelGGL(k_words, dim3((p.Dlog + 255) / 256), dim3(256), 0, st, a.words, p.d, p.sz[0], p.sz[1], p.Dlog);
  LOG_CHECK();
  hipLaunchKernelGGL(k_logrows, dim3((p.R + 3) / 4, p.B), dim3(256), 0, st, a);
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
  hipLaunchKernelGGL(k_words, dim3((p.Dlog + 255) / 256), dim3(256), 0, st, a.words, p.d, p.sz[0], p.sz[1], p.Dlog);
  LOG_CHECK();
  if (p.readout == EWS_READOUT_MAX) {
    LArgs f = a;
    f.out = grad_rows;  // scratch for the pooled values: overwritten below
    hipLaunchKernelGGL(k_logrows, dim3((p.R + 3) / 4, p.B), dim3(256), 0, st, f);
    LOG_CHECK();
    hipLaunchKernelGGL(k_logpool, dim3((p.Dlog + 255) / 256, p.B), dim3(256), 0, st, f);
    LOG_CHECK();
  }
  const int per = p.Dlog + p.d + (p.N >= 3 ? p.d * p.d : 0);
  const size_t shm = (size_t)4 * per * 4;
  (void)hipFuncSetAttribute(reinterpret_cast<const void*>(k_logrows_bwd), hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)shm);
  hipLaunchKernelGGL(k_logrows_bwd, dim3((p.R + 3) / 4, p.B), dim3(256), shm, st, a, grad_out, grad_rows, per);
  LOG_CHECK();
  return EWS_OK;
}

}  // extern "C"
