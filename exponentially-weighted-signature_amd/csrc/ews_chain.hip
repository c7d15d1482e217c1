// Depth-1 EWS scan of a block-diagonal generator made of uniform chains, any number of chains: Jordan chains
// (AParamJordanRepeated: real chains of 2-4 coordinates, complex chains of 2-4 complex coordinates), and, as chains of
// one coordinate, rotation planes and real diagonals. Forward and adjoint, float64 state per chain in registers,
// chunked in time with float64 carries between chunks.
//
// At depth 1 the EWS prefix row is the state S_t = M_t S_{t-1} + s_t (ews/core/chen_scan.py:125-152 at N = 1),
// and a block-diagonal A makes every chain an independent linear recurrence. A chain is J = c I + eps Nil with
// (Nil P)_i = P_{i+1}: a real chain of n coordinates (c = lambda), or a complex chain of k coordinates
// P_i = v_{2i} + i v_{2i+1} (c = a + ib, the 2x2 blocks [[a, -b], [b, a]] with the 2x2 identity above them). An
// analytic g gives g(J) = sum_p g^(p)(c) / p! (eps Nil)^p, so with x = -h c (jordan_engine.py:1-12, combine.py:143-190):
//   flow   exp(-h J) = e^x sum_p (-h eps)^p / p! Nil^p                         (exact at any step)
//   leaf   s_t = phi(-h J) v = sum_p (-h)^p u_p(x) (eps Nil)^p v,  u_p = phi^(p) / p!
// with phi(y) = (e^y - 1) / y (the exact integral: jordan_closed, plane_closed, block_series and van_loan's level 1),
// or, for the series leaf of order q (series_leaf.py:72-113 at level 1: sum_{p<=q} (-h)^p A^p v / (p+1)!),
// u_r = sum_{n=r..q} C(n, r) x^(n-r) / (n+1)!, the r-th derivative over r! of the degree-q Taylor polynomial of phi.
// u_r for the exact leaf: the entire series sum_j x^j / ((j + r + 1) j!) / r! below |x| = 2, else the recurrence
// phi^(r) = (e^x - r phi^(r-1)) / x from (e^x - 1) / x, in float64.
//
// Passes: chunk summaries from a zero state; a float64 carry scan over chunks per (sample, chain) (a workgroup each:
// runs of chunks composed in parallel, then chained), the chunk's flow taken in closed form over its clock span (the
// chain's flows commute); the rows from the carries. Adjoint: each chunk's own rows from a zero cotangent (its
// cotangent on the carry-in state), a float64 reverse scan over chunks (the same parallel scan), then each chunk
// from the cotangent at its end with the states recomputed from its carry into LDS: dv, dh and the chain-parameter
// partials (c, eps), summed in a fixed order (deterministic). Gradients of A land on the entries the chain is read
// from (A[f, f], A[f+1, f] and the coupling A[f, f+1] or A[f, f+2], f the chain's first row), as the reference's
// closed-form leaf and jordan_flows read them; a parametrisation of uniform chains gets its exact parameter gradient
// from them.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "ews_hip.h"

namespace ews {
namespace chain {

struct zd {
  double re, im;
};
__device__ __forceinline__ zd Z(double r, double i = 0.0) { return zd{r, i}; }
__device__ __forceinline__ zd operator+(zd a, zd b) { return zd{a.re + b.re, a.im + b.im}; }
__device__ __forceinline__ zd operator-(zd a, zd b) { return zd{a.re - b.re, a.im - b.im}; }
__device__ __forceinline__ zd operator*(zd a, zd b) {
  return zd{fma(a.re, b.re, -a.im * b.im), fma(a.re, b.im, a.im * b.re)};
}
__device__ __forceinline__ zd operator*(double s, zd a) { return zd{s * a.re, s * a.im}; }
__device__ __forceinline__ zd& operator+=(zd& a, zd b) {
  a.re += b.re;
  a.im += b.im;
  return a;
}
__device__ __forceinline__ zd cj(zd a) { return zd{a.re, -a.im}; }
__device__ __forceinline__ zd cjm(zd a, zd b) {  // conj(a) b
  return zd{fma(a.re, b.re, a.im * b.im), fma(a.re, b.im, -a.im * b.re)};
}
__device__ __forceinline__ double redot(zd a, zd b) { return fma(a.re, b.re, a.im * b.im); }  // Re(conj(a) b)
__device__ __forceinline__ zd zdiv(zd a, zd b) {  // Smith's algorithm
  if (fabs(b.re) >= fabs(b.im)) {
    const double r = b.im / b.re, den = b.re + b.im * r;
    return zd{(a.re + a.im * r) / den, (a.im - a.re * r) / den};
  }
  const double r = b.re / b.im, den = b.im + b.re * r;
  return zd{(a.re * r + a.im) / den, (a.im * r - a.re) / den};
}
__device__ __forceinline__ zd zexp(zd a) {
  double s, c;
  sincos(a.im, &s, &c);
  const double m = exp(a.re);
  return zd{m * c, m * s};
}

constexpr int kTaylor = 28;       // terms of the phi^(r) series (|x| <= 2: the tail is below 1e-20)
constexpr double kSwitch = 2.0;   // |x| above which the recurrence from e^x takes over
constexpr int kMaxT = 64;         // longest chunk (the adjoint's LDS holds a chunk of states per lane)

struct CArgs {
  int B, L, n, d, K, size, cplx, M;  // M: coordinates per chain (complex for complex chains)
  int T, C, KP, CPW;                 // chunk length and count; lanes per chunk (power of 2 >= K); chunks per wave
  int flow_mode, leaf_mode, readout, lvl0, W, q;
  const float* path;
  const float* clock;
  const float* A;
  float* out;
  const float* gout;
  double* carries;  // (B, C+1, K, M) complex: the state before each chunk, and after the last
  double* summ;     // (B, C, K, M) complex: each chunk from a zero state
  double* mu;       // (B, C, K, M) complex: the chunk's own rows' cotangent on its carry-in state
  double* mt;       // (B, C, K, M) complex: the cotangent at the chunk's end from the later chunks
  float* dv;        // (B, n, d) per-interval increment cotangents
  float* dh;        // (B, n) per-interval step cotangents (every chain's)
  double* pp;       // (B, C, K, 5): partials of Re c, Im c, eps, and of the reference steps theta1-theta0, theta2-theta1
  float* gpath;
  float* gclock;
  float* gA;
};

// the chain's eigenvalue and coupling, read from its first rows (jordan_engine.py:338-353)
__device__ __forceinline__ void chain_params(const CArgs& a, int j, zd& c, double& eps) {
  const int f = j * a.size;
  eps = 0.0;  // a chain of one coordinate (a diagonal entry, a rotation plane) has no coupling
  if (a.cplx) {
    c = Z((double)a.A[(size_t)f * a.d + f], (double)a.A[(size_t)(f + 1) * a.d + f]);
    if (a.M > 1) eps = (double)a.A[(size_t)f * a.d + f + 2];
  } else {
    c = Z((double)a.A[(size_t)f * a.d + f]);
    if (a.M > 1) eps = (double)a.A[(size_t)f * a.d + f + 1];
  }
}

// the clock step of interval t under a flow mode (chen_scan.py:155-168): its own, or the shared reference step
// theta1 - theta0 (cached) / theta2 - theta1 with interval 0 taking none (cached with basepoint)
__device__ __forceinline__ double mode_step(const float* th, int L, int t, double h_own, int mode) {
  if (mode == EWS_FLOW_PER_INTERVAL) return h_own;
  if (mode == EWS_FLOW_CACHED) return (double)th[1] - (double)th[0];
  if (t == 0 || L < 3) return 0.0;
  return (double)th[2] - (double)th[1];
}

// u[r] = phi^(r)(x) / r!, r = 0..R: exact (q = 0) or of the degree-q Taylor polynomial of phi
template <int R>
__device__ __forceinline__ void u_table(zd x, int q, zd* u) {
#pragma unroll
  for (int r = 0; r <= R; ++r) u[r] = Z(0.0);
  if (q > 0) {
#pragma unroll
    for (int r = 0; r <= R; ++r) {
      if (r > q) continue;
      // sum_{m=0..q-r} a_m x^m, a_m = C(m+r, r) / (m+r+1)!, by Horner from the top coefficient
      double top = 1.0;  // C(q, r) / (q+1)!
      for (int i = 1; i <= q + 1; ++i) top /= (double)i;
      for (int i = 0; i < r; ++i) top = top * (double)(q - i) / (double)(i + 1);
      zd acc = Z(top);
      double am = top;
      for (int m = q - r - 1; m >= 0; --m) {
        am = am * (double)(m + 1) * (double)(m + r + 2) / (double)(m + r + 1);
        acc = acc * x + Z(am);
      }
      u[r] = acc;
    }
    return;
  }
  if (x.re * x.re + x.im * x.im <= kSwitch * kSwitch) {
    zd t = Z(1.0);  // x^j / j!
    for (int j = 0; j < kTaylor; ++j) {
#pragma unroll
      for (int r = 0; r <= R; ++r) u[r] += (1.0 / (double)(j + r + 1)) * t;
      t = (1.0 / (double)(j + 1)) * (t * x);
    }
    double f = 1.0;
#pragma unroll
    for (int r = 1; r <= R; ++r) {
      f *= (double)r;
      u[r] = (1.0 / f) * u[r];
    }
  } else {
    const zd e = zexp(x);
    zd ph = zdiv(e - Z(1.0), x);
    u[0] = ph;
    double f = 1.0;
#pragma unroll
    for (int r = 1; r <= R; ++r) {
      ph = zdiv(e - (double)r * ph, x);
      f *= (double)r;
      u[r] = (1.0 / f) * ph;
    }
  }
}

// one interval's coefficients: leaf g[p] = (-hl)^p u_p(-hl c), flow e[p] = e^{-hf c} (-hf eps)^p / p!
template <int M>
struct Coef {
  zd g[M], e[M];
};
template <int M>
__device__ __forceinline__ void coefs(zd c, double eps, double hl, double hf, int q, Coef<M>& k) {
  zd u[M];
  u_table<M - 1>(Z(-hl) * c, q, u);
  double hp = 1.0;
#pragma unroll
  for (int p = 0; p < M; ++p) {
    k.g[p] = hp * u[p];
    hp *= -hl;
  }
  k.e[0] = zexp(Z(-hf) * c);
#pragma unroll
  for (int p = 1; p < M; ++p) k.e[p] = (-hf * eps / (double)p) * k.e[p - 1];
}
// the step S <- E S + s with s = sum_p g[p] (eps Nil)^p v
template <int M>
__device__ __forceinline__ void step(const Coef<M>& k, double eps, const zd* v, zd* S) {
  zd ew[M];  // eps^p
  ew[0] = Z(1.0);
#pragma unroll
  for (int p = 1; p < M; ++p) ew[p] = eps * ew[p - 1];
#pragma unroll
  for (int i = 0; i < M; ++i) {
    zd acc = Z(0.0);
#pragma unroll
    for (int p = 0; p + i < M; ++p) acc += k.e[p] * S[i + p] + k.g[p] * (ew[p].re * v[i + p]);
    S[i] = acc;
  }
}
// the chunk's flow over a clock span tau: e^{-tau c} sum_p (-tau eps)^p / p! Nil^p
template <int M>
__device__ __forceinline__ void span_flow(zd c, double eps, double tau, zd* F) {
  F[0] = zexp(Z(-tau) * c);
#pragma unroll
  for (int p = 1; p < M; ++p) F[p] = (-tau * eps / (double)p) * F[p - 1];
}
// the flow span of chunk cc under the flow mode
__device__ __forceinline__ double chunk_span(const CArgs& a, const float* th, int cc) {
  const int t0 = cc * a.T, t1 = min(t0 + a.T, a.n);
  if (a.flow_mode == EWS_FLOW_PER_INTERVAL) return (double)th[t1] - (double)th[t0];
  const double hr = mode_step(th, a.L, 1, 0.0, a.flow_mode);
  const int nstep = (a.flow_mode == EWS_FLOW_CACHED_BASEPOINT && t0 == 0) ? t1 - 1 : t1 - t0;
  return hr * (double)nstep;
}

// knot row t of the chain's coordinates (complex coordinates of a complex chain)
template <int M, bool CPLX>
__device__ __forceinline__ void load_knot(const CArgs& a, int b, int t, int j, zd* x) {
  const float* r = a.path + ((size_t)b * a.L + t) * a.d + (size_t)j * a.size;
#pragma unroll
  for (int i = 0; i < M; ++i) x[i] = CPLX ? Z((double)r[2 * i], (double)r[2 * i + 1]) : Z((double)r[i]);
}

struct Lane {
  int b, j, c, t0, Tc;
  bool live, group;  // live: a real chain of an existing chunk; group: the lane's chunk exists
};
__device__ __forceinline__ Lane lane_of(const CArgs& a) {
  Lane l;
  const int lane = threadIdx.x;
  l.b = blockIdx.y;
  l.j = lane % a.KP;
  l.c = blockIdx.x * a.CPW + lane / a.KP;
  l.group = l.c < a.C;
  l.live = l.group && l.j < a.K;
  l.t0 = l.c * a.T;
  l.Tc = l.group ? min(a.T, a.n - l.t0) : 0;
  return l;
}
__device__ __forceinline__ size_t st_off(const CArgs& a, int b, int c, int j) {  // (B, C(+1), K, M) complex rows
  return (((size_t)b * (a.C + 1) + c) * a.K + j) * a.M * 2;
}
__device__ __forceinline__ size_t ch_off(const CArgs& a, int b, int c, int j) {  // (B, C, K, M)
  return (((size_t)b * a.C + c) * a.K + j) * a.M * 2;
}
template <int M>
__device__ __forceinline__ void ld_state(const double* p, zd* S) {
#pragma unroll
  for (int i = 0; i < M; ++i) S[i] = Z(p[2 * i], p[2 * i + 1]);
}
template <int M>
__device__ __forceinline__ void st_state(double* p, const zd* S) {
#pragma unroll
  for (int i = 0; i < M; ++i) {
    p[2 * i] = S[i].re;
    p[2 * i + 1] = S[i].im;
  }
}

// ------------------------------------------------------------------------------------------------ forward
// ROWS false: the chunk's summary from a zero state; true: the prefix rows from the chunk's carry
template <int M, bool CPLX, bool ROWS>
__device__ __forceinline__ void fwd_body(const CArgs& a) {
  const Lane l = lane_of(a);
  if (!l.live) return;
  zd c;
  double eps;
  chain_params(a, l.j, c, eps);
  zd S[M];
  if (ROWS) {
    ld_state<M>(a.carries + st_off(a, l.b, l.c, l.j), S);
  } else {
#pragma unroll
    for (int i = 0; i < M; ++i) S[i] = Z(0.0);
  }
  const float* th = a.clock + (size_t)l.b * a.L;
  zd x0[M], x1[M], v[M];
  load_knot<M, CPLX>(a, l.b, l.t0, l.j, x0);
  double th0 = (double)th[l.t0];
  Coef<M> k;
  const bool fixed = a.flow_mode != EWS_FLOW_PER_INTERVAL && a.leaf_mode != EWS_FLOW_PER_INTERVAL;
  if (fixed) coefs<M>(c, eps, mode_step(th, a.L, 1, 0.0, a.leaf_mode), mode_step(th, a.L, 1, 0.0, a.flow_mode), a.q, k);
  for (int s = 0; s < l.Tc; ++s) {
    const int t = l.t0 + s;
    load_knot<M, CPLX>(a, l.b, t + 1, l.j, x1);
    const double th1 = (double)th[t + 1], h = th1 - th0;
#pragma unroll
    for (int i = 0; i < M; ++i) v[i] = x1[i] - x0[i];
    if (!fixed || (t <= 1 && (a.flow_mode == EWS_FLOW_CACHED_BASEPOINT || a.leaf_mode == EWS_FLOW_CACHED_BASEPOINT)))
      coefs<M>(c, eps, mode_step(th, a.L, t, h, a.leaf_mode), mode_step(th, a.L, t, h, a.flow_mode), a.q, k);
    step<M>(k, eps, v, S);
    if (ROWS) {
      float* row = a.out + ((size_t)l.b * a.n + t) * a.W + a.lvl0 + (size_t)l.j * a.size;
#pragma unroll
      for (int i = 0; i < M; ++i) {
        if (CPLX) {
          row[2 * i] = (float)S[i].re;
          row[2 * i + 1] = (float)S[i].im;
        } else {
          row[i] = (float)S[i].re;
        }
      }
      if (a.lvl0 && l.j == 0) a.out[((size_t)l.b * a.n + t) * a.W] = 1.0f;
    }
#pragma unroll
    for (int i = 0; i < M; ++i) x0[i] = x1[i];
    th0 = th1;
  }
  if (!ROWS) st_state<M>(a.summ + ch_off(a, l.b, l.c, l.j), S);
}
template <int M, bool CPLX>
__global__ __launch_bounds__(64) void k_summary(CArgs a) {
  fwd_body<M, CPLX, false>(a);
}
template <int M, bool CPLX>
__global__ __launch_bounds__(64) void k_rows(CArgs a) {
  fwd_body<M, CPLX, true>(a);
}

// ---- carry scans over the chunks: a workgroup per (sample, chain), its 256 threads each owning a run of
// consecutive chunks. A chunk acts on the chain's state as S -> F S + z (F its flow over the chunk's clock span, a
// polynomial in Nil; z its summary) and, in the adjoint, on the cotangent as X -> F^H X + m with the chunks taken
// from the last. Each thread composes its run into one such map, thread 0 chains the 256 maps from the initial
// state in order (float64, fixed order), and each thread re-walks its run from its start state writing the carries
// (cotangents). The maps compose as (F2, z2) o (F1, z1) = (F2 F1, F2 z1 + z2) (adjoint: F2^H z1 + z2), the flows
// being polynomials in Nil that commute.
constexpr int kCarryThreads = 256;

template <int M>
__device__ __forceinline__ void nil_apply(const zd* F, const zd* S, zd* o) {  // (F S)_i = sum_p F[p] S_{i+p}
#pragma unroll
  for (int i = 0; i < M; ++i) {
    zd acc = Z(0.0);
#pragma unroll
    for (int p = 0; p + i < M; ++p) acc += F[p] * S[i + p];
    o[i] = acc;
  }
}
template <int M>
__device__ __forceinline__ void nil_apply_h(const zd* F, const zd* X, zd* o) {  // (F^H X)_k = sum_p conj(F[p]) X_{k-p}
#pragma unroll
  for (int k = 0; k < M; ++k) {
    zd acc = Z(0.0);
#pragma unroll
    for (int p = 0; p <= k; ++p) acc += cjm(F[p], X[k - p]);
    o[k] = acc;
  }
}
template <int M>
__device__ __forceinline__ void nil_mul(const zd* F2, const zd* F1, zd* o) {  // product of polynomials in Nil
#pragma unroll
  for (int r = 0; r < M; ++r) {
    zd acc = Z(0.0);
#pragma unroll
    for (int p = 0; p <= r; ++p) acc += F2[p] * F1[r - p];
    o[r] = acc;
  }
}
// the map of chunk cc (application order: ascending chunks forward, descending in the adjoint)
template <int M, bool BWD>
__device__ __forceinline__ void chunk_map(const CArgs& a, int b, int j, zd c, double eps, const float* th, int cc,
                                          zd* F, zd* z) {
  span_flow<M>(c, eps, chunk_span(a, th, cc), F);
  if (!BWD) {
    ld_state<M>(a.summ + ch_off(a, b, cc, j), z);
  } else if (a.readout != EWS_READOUT_TERMINAL) {
    ld_state<M>(a.mu + ch_off(a, b, cc, j), z);
  } else {
#pragma unroll
    for (int i = 0; i < M; ++i) z[i] = Z(0.0);
  }
}
template <int M, bool BWD>
__device__ __forceinline__ void map_apply(const zd* F, const zd* z, zd* S) {
  zd o[M];
  if (BWD) nil_apply_h<M>(F, S, o);
  else nil_apply<M>(F, S, o);
#pragma unroll
  for (int i = 0; i < M; ++i) S[i] = o[i] + z[i];
}
template <int M, bool CPLX, bool BWD>
__device__ __forceinline__ void carry_scan(const CArgs& a) {
  __shared__ double s_map[kCarryThreads][4 * M];  // each thread's composed map: F, then z (complex)
  __shared__ double s_in[kCarryThreads][2 * M];   // each thread's start state
  const int b = blockIdx.x / a.K, j = blockIdx.x % a.K, tid = threadIdx.x;
  zd c;
  double eps;
  chain_params(a, j, c, eps);
  const float* th = a.clock + (size_t)b * a.L;
  const int nth = blockDim.x, per = (a.C + nth - 1) / nth, nrun = (a.C + per - 1) / per;
  const int q0 = tid * per, q1 = min(a.C, q0 + per);  // the thread's run, in application order
  zd AF[M], Az[M], F[M], z[M], t[M];
#pragma unroll
  for (int i = 0; i < M; ++i) {
    AF[i] = Z(i == 0 ? 1.0 : 0.0);
    Az[i] = Z(0.0);
  }
  for (int q = q0; q < q1; ++q) {
    const int cc = BWD ? a.C - 1 - q : q;
    chunk_map<M, BWD>(a, b, j, c, eps, th, cc, F, z);
    nil_mul<M>(F, AF, t);  // the chunk after the run so far
#pragma unroll
    for (int i = 0; i < M; ++i) AF[i] = t[i];
    map_apply<M, BWD>(F, z, Az);
  }
  st_state<M>(&s_map[tid][0], AF);
  st_state<M>(&s_map[tid][2 * M], Az);
  __syncthreads();
  if (tid == 0) {
    zd S[M];
    if (BWD && a.readout == EWS_READOUT_TERMINAL) {
      const float* r = a.gout + (size_t)b * a.W + a.lvl0 + (size_t)j * a.size;
#pragma unroll
      for (int i = 0; i < M; ++i) S[i] = CPLX ? Z((double)r[2 * i], (double)r[2 * i + 1]) : Z((double)r[i]);
    } else {
#pragma unroll
      for (int i = 0; i < M; ++i) S[i] = Z(0.0);
    }
    for (int u = 0; u < nrun; ++u) {  // the threads past nrun own no chunk
      st_state<M>(&s_in[u][0], S);
      ld_state<M>(&s_map[u][0], F);
      ld_state<M>(&s_map[u][2 * M], z);
      map_apply<M, BWD>(F, z, S);
    }
  }
  __syncthreads();
  if (tid >= nrun) return;
  zd S[M];
  ld_state<M>(&s_in[tid][0], S);
  for (int q = q0; q < q1; ++q) {
    const int cc = BWD ? a.C - 1 - q : q;
    if (BWD) st_state<M>(a.mt + ch_off(a, b, cc, j), S);  // the cotangent at the chunk's end
    else st_state<M>(a.carries + st_off(a, b, cc, j), S);  // the state before the chunk
    chunk_map<M, BWD>(a, b, j, c, eps, th, cc, F, z);
    map_apply<M, BWD>(F, z, S);
    if (!BWD && cc == a.C - 1) st_state<M>(a.carries + st_off(a, b, a.C, j), S);
  }
}
template <int M, bool CPLX>
__global__ __launch_bounds__(kCarryThreads) void k_carry(CArgs a) {
  carry_scan<M, CPLX, false>(a);
}

// the terminal row: the state after the last chunk
template <int M, bool CPLX>
__global__ void k_terminal(CArgs a) {
  const int e = blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= a.B * a.W) return;
  const int b = e / a.W, col = e % a.W;
  if (a.lvl0 && col == 0) {
    a.out[e] = 1.0f;
    return;
  }
  const int r = col - a.lvl0, j = r / a.size, w = r % a.size;
  const double* s = a.carries + st_off(a, b, a.C, j);
  a.out[e] = (float)(CPLX ? s[w] : s[2 * w]);  // complex coordinate i at (2i, 2i+1) = (re, im); real: re
}

// ------------------------------------------------------------------------------------------------ adjoint
// the row cotangent of interval t on the chain's coordinates (G = dl/dRe + i dl/dIm for complex coordinates)
template <int M, bool CPLX>
__device__ __forceinline__ void load_g(const CArgs& a, int b, int t, int j, zd* g) {
  const float* r = a.gout + ((size_t)b * a.n + t) * a.W + a.lvl0 + (size_t)j * a.size;
#pragma unroll
  for (int i = 0; i < M; ++i) g[i] = CPLX ? Z((double)r[2 * i], (double)r[2 * i + 1]) : Z((double)r[i]);
}
// Lam <- E^H Lam
template <int M>
__device__ __forceinline__ void adj_flow(const zd* e, zd* Lam) {
  zd o[M];
#pragma unroll
  for (int i = 0; i < M; ++i) o[i] = Z(0.0);
#pragma unroll
  for (int i = 0; i < M; ++i)
#pragma unroll
    for (int p = 0; p + i < M; ++p) o[i + p] += cjm(e[p], Lam[i]);
#pragma unroll
  for (int i = 0; i < M; ++i) Lam[i] = o[i];
}

// the chunk's own rows from a zero cotangent at its end: the cotangent on its carry-in state
template <int M, bool CPLX>
__global__ __launch_bounds__(64) void k_local(CArgs a) {
  const Lane l = lane_of(a);
  if (!l.live) return;
  zd c;
  double eps;
  chain_params(a, l.j, c, eps);
  const float* th = a.clock + (size_t)l.b * a.L;
  zd Lam[M], g[M], e[M];
#pragma unroll
  for (int i = 0; i < M; ++i) Lam[i] = Z(0.0);
  for (int s = l.Tc - 1; s >= 0; --s) {
    const int t = l.t0 + s;
    load_g<M, CPLX>(a, l.b, t, l.j, g);
#pragma unroll
    for (int i = 0; i < M; ++i) Lam[i] += g[i];
    const double hf = mode_step(th, a.L, t, (double)th[t + 1] - (double)th[t], a.flow_mode);
    span_flow<M>(c, eps, hf, e);
    adj_flow<M>(e, Lam);
  }
  st_state<M>(a.mu + ch_off(a, l.b, l.c, l.j), Lam);
}

// the reverse carry scan: mt[c] = the cotangent at chunk c's end from the later chunks (the terminal row's at the
// last chunk); mt[c-1] = F_c^H mt[c] + mu[c]
template <int M, bool CPLX>
__global__ __launch_bounds__(kCarryThreads) void k_carry_bwd(CArgs a) {
  carry_scan<M, CPLX, true>(a);
}

// each chunk from the cotangent at its end: states from the carry into LDS, then the steps in reverse with dv, dh
// and the chain-parameter partials
template <int M, bool CPLX>
__global__ __launch_bounds__(64) void k_full(CArgs a) {
  extern __shared__ float2 s_st[];  // [64 lanes][T][M] states before each step
  const Lane l = lane_of(a);
  if (!l.group) return;  // the lanes of one chunk stay together: the dh sums exchange across them
  const bool live = l.live;
  float2* my = s_st + (size_t)threadIdx.x * a.T * M;
  zd c = Z(0.0);
  double eps = 0.0;
  if (live) chain_params(a, l.j, c, eps);
  const float* th = a.clock + (size_t)l.b * a.L;
  // 1. the states S_{t-1} of the chunk's steps, from its carry
  zd S[M], x0[M], x1[M], v[M];
  Coef<M> k;
  if (live) {
    ld_state<M>(a.carries + st_off(a, l.b, l.c, l.j), S);
    load_knot<M, CPLX>(a, l.b, l.t0, l.j, x0);
    double th0 = (double)th[l.t0];
    for (int s = 0; s < l.Tc; ++s) {
      const int t = l.t0 + s;
#pragma unroll
      for (int i = 0; i < M; ++i) my[s * M + i] = float2{(float)S[i].re, (float)S[i].im};
      load_knot<M, CPLX>(a, l.b, t + 1, l.j, x1);
      const double th1 = (double)th[t + 1], h = th1 - th0;
#pragma unroll
      for (int i = 0; i < M; ++i) v[i] = x1[i] - x0[i];
      coefs<M>(c, eps, mode_step(th, a.L, t, h, a.leaf_mode), mode_step(th, a.L, t, h, a.flow_mode), a.q, k);
      step<M>(k, eps, v, S);
#pragma unroll
      for (int i = 0; i < M; ++i) x0[i] = x1[i];
      th0 = th1;
    }
  }
  // 2. the steps in reverse from the cotangent at the chunk's end
  zd Lam[M], g[M], Gc = Z(0.0);
  double deps = 0.0, dref0 = 0.0, dref1 = 0.0;
  if (live) {
    ld_state<M>(a.mt + ch_off(a, l.b, l.c, l.j), Lam);
    load_knot<M, CPLX>(a, l.b, l.t0 + l.Tc, l.j, x1);
  }
  for (int s = l.Tc - 1; s >= 0; --s) {
    const int t = l.t0 + s;
    double dh_own = 0.0;
    if (live) {
      if (a.readout != EWS_READOUT_TERMINAL) {
        load_g<M, CPLX>(a, l.b, t, l.j, g);
#pragma unroll
        for (int i = 0; i < M; ++i) Lam[i] += g[i];
      }
      load_knot<M, CPLX>(a, l.b, t, l.j, x0);
#pragma unroll
      for (int i = 0; i < M; ++i) v[i] = x1[i] - x0[i];
      const double h = (double)th[t + 1] - (double)th[t];
      const double hl = mode_step(th, a.L, t, h, a.leaf_mode), hf = mode_step(th, a.L, t, h, a.flow_mode);
      zd u[M + 1];
      u_table<M>(Z(-hl) * c, a.q, u);
      zd ew[M];  // eps^p, as reals
      ew[0] = Z(1.0);
#pragma unroll
      for (int p = 1; p < M; ++p) ew[p] = eps * ew[p - 1];
      // leaf: s_i = sum_p z_p eps^p v_{i+p}, z_p = (-hl)^p u_p(-hl c)
      zd dv[M];
#pragma unroll
      for (int i = 0; i < M; ++i) dv[i] = Z(0.0);
      double hp = 1.0, hq = 0.0, dhl = 0.0;  // (-hl)^p, (-hl)^(p-1)
#pragma unroll
      for (int p = 0; p < M; ++p) {
        const zd zp = hp * u[p];
        zd Gz = Z(0.0);  // cotangent of z_p
#pragma unroll
        for (int i = 0; i + p < M; ++i) {
          Gz += cjm(ew[p].re * v[i + p], Lam[i]);
          dv[i + p] += (ew[p].re) * cjm(zp, Lam[i]);
          if (p > 0) deps += (double)p * ew[p - 1].re * redot(Lam[i], zp * v[i + p]);
        }
        // dz_p / dc = -hl (p+1) (-hl)^p u_{p+1}; dz_p / dhl = -p (-hl)^(p-1) u_p - c (p+1) (-hl)^p u_{p+1}
        const zd dzc = (-hl * (double)(p + 1) * hp) * u[p + 1];
        Gc += cjm(dzc, Gz);
        const zd dzh = (-(double)p * hq) * u[p] - ((double)(p + 1) * hp) * (c * u[p + 1]);
        dhl += redot(Gz, dzh);
        hq = hp;
        hp *= -hl;
      }
      // flow: (E S)_i = sum_p e_p S_{i+p}, e_p = e^{-hf c} (-hf eps)^p / p!
      zd Sp[M];
#pragma unroll
      for (int i = 0; i < M; ++i) {
        const float2 w = my[s * M + i];
        Sp[i] = Z((double)w.x, (double)w.y);
      }
      zd e[M];
      span_flow<M>(c, eps, hf, e);
      const zd ef = e[0];
      double dhf = 0.0;
      double xp = 1.0, fp = 1.0;  // (-hf eps)^(p-1), (p-1)!
#pragma unroll
      for (int p = 0; p < M; ++p) {
        zd Ge = Z(0.0);
#pragma unroll
        for (int i = 0; i + p < M; ++i) Ge += cjm(Sp[i + p], Lam[i]);
        Gc += cjm((-hf) * e[p], Ge);
        zd deh = Z(0.0) - c * e[p];
        if (p > 0) {
          deh += (-eps * xp / fp) * ef;
          deps += redot(Ge, (-hf * xp / fp) * ef);
          xp *= -hf * eps;
          fp *= (double)p;
        }
        dhf += redot(Ge, deh);
      }
      adj_flow<M>(e, Lam);
      // increment cotangent of the interval
      float* dvr = a.dv + ((size_t)l.b * a.n + t) * a.d + (size_t)l.j * a.size;
#pragma unroll
      for (int i = 0; i < M; ++i) {
        if (CPLX) {
          dvr[2 * i] = (float)dv[i].re;
          dvr[2 * i + 1] = (float)dv[i].im;
        } else {
          dvr[i] = (float)dv[i].re;
        }
      }
      // steps: the interval's own, or the shared reference steps (theta1 - theta0: cached; theta2 - theta1:
      // cached with basepoint, interval 0 none)
      if (a.leaf_mode == EWS_FLOW_PER_INTERVAL) dh_own += dhl;
      else if (a.leaf_mode == EWS_FLOW_CACHED) dref0 += dhl;
      else if (t > 0) dref1 += dhl;
      if (a.flow_mode == EWS_FLOW_PER_INTERVAL) dh_own += dhf;
      else if (a.flow_mode == EWS_FLOW_CACHED) dref0 += dhf;
      else if (t > 0) dref1 += dhf;
#pragma unroll
      for (int i = 0; i < M; ++i) x1[i] = x0[i];
    }
    // dh of the interval: every chain of the sample, summed across the chunk's lane group
    double acc = dh_own;
    for (int o = 1; o < a.KP; o <<= 1) acc += __shfl_xor(acc, o, 64);
    if (l.j == 0) a.dh[(size_t)l.b * a.n + t] = (float)acc;
  }
  if (live) {
    double* pp = a.pp + (((size_t)l.b * a.C + l.c) * a.K + l.j) * 5;
    pp[0] = Gc.re;
    pp[1] = Gc.im;
    pp[2] = deps;
    pp[3] = dref0;
    pp[4] = dref1;
  }
}

// knot gradients: dX_t = dv_{t-1} - dv_t; dtheta_t = dh_{t-1} - dh_t, plus the reference steps' shares (summed over
// the sample's chunks and chains in order)
__device__ __forceinline__ void knot_clock(const CArgs& a, size_t b, size_t t) {
  double g = (t > 0 ? (double)a.dh[b * a.n + t - 1] : 0.0) - (t < (size_t)a.n ? (double)a.dh[b * a.n + t] : 0.0);
  if (t <= 2 && (a.flow_mode != EWS_FLOW_PER_INTERVAL || a.leaf_mode != EWS_FLOW_PER_INTERVAL)) {
    double r0 = 0.0, r1 = 0.0;
    for (size_t i = 0; i < (size_t)a.C * a.K; ++i) {
      r0 += a.pp[(b * a.C * a.K + i) * 5 + 3];
      r1 += a.pp[(b * a.C * a.K + i) * 5 + 4];
    }
    if (t == 1) g += r0 - r1;
    else if (t == 0) g -= r0;
    else g += r1;
  }
  a.gclock[b * a.L + t] = (float)g;
}
__global__ void k_knots(CArgs a) {
  const size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  const size_t per = (size_t)a.L * (a.d + 1);
  if (e >= (size_t)a.B * per) return;
  const size_t b = e / per, r = e % per, t = r / (a.d + 1), ch = r % (a.d + 1);
  if (ch < (size_t)a.d) {
    const float lo = t > 0 ? a.dv[(b * a.n + t - 1) * a.d + ch] : 0.0f;
    const float hi = t < (size_t)a.n ? a.dv[(b * a.n + t) * a.d + ch] : 0.0f;
    a.gpath[(b * a.L + t) * a.d + ch] = lo - hi;
  } else if (a.gclock) {
    knot_clock(a, b, t);
  }
}
// the same for d % 4 == 0 and 16-byte aligned rows: the path columns four at a time (a thread per sample, knot and
// float4), then the clock column, a thread per (sample, knot), in threads B L d / 4 ..
__global__ void k_knots4(CArgs a) {
  const size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  const size_t d4 = (size_t)a.d / 4, np = (size_t)a.B * a.L * d4;
  if (e < np) {
    const size_t b = e / ((size_t)a.L * d4), r = e % ((size_t)a.L * d4), t = r / d4, q = r % d4;
    const float4* dv4 = reinterpret_cast<const float4*>(a.dv);
    const float4 z = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    const float4 lo = t > 0 ? dv4[(b * a.n + t - 1) * d4 + q] : z;
    const float4 hi = t < (size_t)a.n ? dv4[(b * a.n + t) * d4 + q] : z;
    reinterpret_cast<float4*>(a.gpath)[(b * a.L + t) * d4 + q] =
        make_float4(lo.x - hi.x, lo.y - hi.y, lo.z - hi.z, lo.w - hi.w);
  } else if (a.gclock && e < np + (size_t)a.B * a.L) {
    const size_t k = e - np;
    knot_clock(a, k / a.L, k % a.L);
  }
}

// grad_A: zero, then each chain's entries from the partials (one workgroup per chain and component, float64 sums in
// a fixed order)
__global__ void k_zero_a(CArgs a) {
  const int e = blockIdx.x * blockDim.x + threadIdx.x;
  if (e < a.d * a.d) a.gA[e] = 0.0f;
}
__global__ __launch_bounds__(256) void k_params(CArgs a) {
  __shared__ double red[256];
  const int j = blockIdx.x / 3, comp = blockIdx.x % 3, tid = threadIdx.x;
  if ((!a.cplx && comp == 1) || (comp == 2 && a.M == 1)) return;  // uniform across the workgroup
  const size_t tot = (size_t)a.B * a.C;
  double acc = 0.0;
  for (size_t it = tid; it < tot; it += 256) acc += a.pp[(it * a.K + j) * 5 + comp];
  red[tid] = acc;
  __syncthreads();
  for (int o = 128; o > 0; o >>= 1) {
    if (tid < o) red[tid] += red[tid + o];
    __syncthreads();
  }
  if (tid == 0) {
    const int f = j * a.size;
    size_t idx;
    if (comp == 0) idx = (size_t)f * a.d + f;
    else if (comp == 1) idx = (size_t)(f + 1) * a.d + f;
    else idx = a.cplx ? (size_t)f * a.d + f + 2 : (size_t)f * a.d + f + 1;
    a.gA[idx] = (float)red[0];
  }
}

}  // namespace chain

namespace {

using chain::CArgs;

int chain_check(const ews_chain_desc* s) {
  if (!s) return EWS_ERR_NULL;
  if (s->batch < 1 || s->length < 2 || s->dim < 1) return EWS_ERR_SHAPE;
  if (s->kind == EWS_JORDAN_REAL) {
    if (s->size < 1 || s->size > 4) return EWS_ERR_OPTION;
  } else if (s->kind == EWS_JORDAN_COMPLEX) {
    if (s->size != 2 && s->size != 4 && s->size != 6 && s->size != 8) return EWS_ERR_OPTION;
  } else {
    return EWS_ERR_OPTION;
  }
  if (s->dim % s->size || s->dim / s->size > 64) return EWS_ERR_SHAPE;
  for (int m : {s->flow_mode, s->leaf_mode})
    if (m != EWS_FLOW_PER_INTERVAL && m != EWS_FLOW_CACHED && m != EWS_FLOW_CACHED_BASEPOINT) return EWS_ERR_OPTION;
  if (s->readout != EWS_READOUT_PREFIX && s->readout != EWS_READOUT_TERMINAL) return EWS_ERR_OPTION;
  if (s->series_q < 0 || s->series_q > 48) return EWS_ERR_OPTION;
  if (s->chunk < 0 || s->chunk > chain::kMaxT) return EWS_ERR_SHAPE;
  return EWS_OK;
}

CArgs chain_args(const ews_chain_desc* s) {
  CArgs a{};
  a.B = s->batch;
  a.L = s->length;
  a.n = s->length - 1;
  a.d = s->dim;
  a.size = s->size;
  a.cplx = s->kind == EWS_JORDAN_COMPLEX;
  a.M = a.cplx ? s->size / 2 : s->size;
  a.K = s->dim / s->size;
  a.T = s->chunk ? s->chunk : 32;
  a.C = (a.n + a.T - 1) / a.T;
  a.KP = 1;
  while (a.KP < a.K) a.KP <<= 1;
  a.CPW = 64 / a.KP;
  a.flow_mode = s->flow_mode;
  a.leaf_mode = s->leaf_mode;
  a.readout = s->readout;
  a.lvl0 = s->level0 ? 1 : 0;
  a.W = a.lvl0 + a.d;
  a.q = s->series_q;
  return a;
}

size_t al256c(size_t x) { return (x + 255) & ~(size_t)255; }
size_t carries_bytes(const CArgs& a) { return al256c((size_t)a.B * (a.C + 1) * a.K * a.M * 16); }
size_t chunk_state_bytes(const CArgs& a) { return al256c((size_t)a.B * a.C * a.K * a.M * 16); }

// the workspace: summaries (forward); mu, mt, dv, dh and the partials (backward)
struct WsOff {
  size_t summ, mu, mt, dv, dh, pp, total;
};
WsOff ws_off(const CArgs& a) {
  WsOff w{};
  size_t o = 0;
  w.summ = o; o += chunk_state_bytes(a);
  w.mu = o; o += chunk_state_bytes(a);
  w.mt = o; o += chunk_state_bytes(a);
  w.dv = o; o += al256c((size_t)a.B * a.n * a.d * 4);
  w.dh = o; o += al256c((size_t)a.B * a.n * 4);
  w.pp = o; o += al256c((size_t)a.B * a.C * a.K * 5 * 8);
  w.total = o;
  return w;
}

// threads of a carry-scan workgroup: one per chunk up to 256, in whole wavefronts
int carry_threads(int C) { return std::min(chain::kCarryThreads, std::max(64, (C + 63) / 64 * 64)); }

#define EWS_CHAIN_LAUNCH(KERNEL, GRID, BLK, LDS, ST, A)                                                       \
  do {                                                                                                        \
    const bool cp = (A).cplx != 0;                                                                            \
    switch ((A).M) {                                                                                          \
      case 1:                                                                                                 \
        if (cp) hipLaunchKernelGGL((KERNEL<1, true>), GRID, BLK, LDS, ST, A);                                  \
        else hipLaunchKernelGGL((KERNEL<1, false>), GRID, BLK, LDS, ST, A);                                    \
        break;                                                                                                \
      case 2:                                                                                                 \
        if (cp) hipLaunchKernelGGL((KERNEL<2, true>), GRID, BLK, LDS, ST, A);                                  \
        else hipLaunchKernelGGL((KERNEL<2, false>), GRID, BLK, LDS, ST, A);                                    \
        break;                                                                                                \
      case 3:                                                                                                 \
        if (cp) hipLaunchKernelGGL((KERNEL<3, true>), GRID, BLK, LDS, ST, A);                                  \
        else hipLaunchKernelGGL((KERNEL<3, false>), GRID, BLK, LDS, ST, A);                                    \
        break;                                                                                                \
      default:                                                                                                \
        if (cp) hipLaunchKernelGGL((KERNEL<4, true>), GRID, BLK, LDS, ST, A);                                  \
        else hipLaunchKernelGGL((KERNEL<4, false>), GRID, BLK, LDS, ST, A);                                    \
        break;                                                                                                \
    }                                                                                                         \
    if (hipGetLastError() != hipSuccess) return EWS_ERR_LAUNCH;                                               \
  } while (0)

// the adjoint's LDS (a chunk of states per lane) can exceed the 64 KB a launch gets without asking
template <int M, bool CPLX>
int allow_lds(size_t bytes) {
  return hipFuncSetAttribute(reinterpret_cast<const void*>(&chain::k_full<M, CPLX>),
                             hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes) == hipSuccess
             ? EWS_OK
             : EWS_ERR_LAUNCH;
}
int allow_full_lds(const CArgs& a, size_t bytes) {
  switch (a.M * 2 + (a.cplx ? 1 : 0)) {
    case 2: return allow_lds<1, false>(bytes);
    case 3: return allow_lds<1, true>(bytes);
    case 4: return allow_lds<2, false>(bytes);
    case 5: return allow_lds<2, true>(bytes);
    case 6: return allow_lds<3, false>(bytes);
    case 7: return allow_lds<3, true>(bytes);
    case 8: return allow_lds<4, false>(bytes);
    default: return allow_lds<4, true>(bytes);
  }
}

}  // namespace
}  // namespace ews

extern "C" {

size_t ews_chain_residual_bytes(const ews_chain_desc* desc) {
  if (ews::chain_check(desc) != EWS_OK) return 0;
  return ews::carries_bytes(ews::chain_args(desc));
}

size_t ews_chain_workspace_bytes(const ews_chain_desc* desc) {
  if (ews::chain_check(desc) != EWS_OK) return 0;
  return ews::ws_off(ews::chain_args(desc)).total;
}

int ews_chain_forward(const ews_chain_desc* desc, const void* path, const float* clock, const float* A, float* out,
                      void* residual, void* workspace, ews_stream_t stream) {
  const int rc = ews::chain_check(desc);
  if (rc != EWS_OK) return rc;
  if (!path || !clock || !A || !out || !residual || !workspace) return EWS_ERR_NULL;
  ews::chain::CArgs a = ews::chain_args(desc);
  a.path = (const float*)path;
  a.clock = clock;
  a.A = A;
  a.out = out;
  a.carries = (double*)residual;
  a.summ = (double*)((char*)workspace + ews::ws_off(a).summ);
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid((a.C + a.CPW - 1) / a.CPW, a.B), blk(64);
  EWS_CHAIN_LAUNCH(ews::chain::k_summary, grid, blk, 0, st, a);
  const dim3 ct(ews::carry_threads(a.C));
  EWS_CHAIN_LAUNCH(ews::chain::k_carry, dim3(a.B * a.K), ct, 0, st, a);
  if (a.readout == EWS_READOUT_PREFIX) {
    EWS_CHAIN_LAUNCH(ews::chain::k_rows, grid, blk, 0, st, a);
  } else {
    const dim3 gt((a.B * a.W + 255) / 256);
    EWS_CHAIN_LAUNCH(ews::chain::k_terminal, gt, dim3(256), 0, st, a);
  }
  return EWS_OK;
}

int ews_chain_backward(const ews_chain_desc* desc, const void* path, const float* clock, const float* A,
                       const void* residual, const float* grad_out, float* grad_path, float* grad_clock,
                       float* grad_A, void* workspace, ews_stream_t stream) {
  const int rc = ews::chain_check(desc);
  if (rc != EWS_OK) return rc;
  if (!path || !clock || !A || !residual || !grad_out || !grad_path || !grad_A || !workspace) return EWS_ERR_NULL;
  ews::chain::CArgs a = ews::chain_args(desc);
  a.path = (const float*)path;
  a.clock = clock;
  a.A = A;
  a.gout = grad_out;
  a.carries = (double*)residual;
  const ews::WsOff w = ews::ws_off(a);
  char* ws = (char*)workspace;
  a.summ = (double*)(ws + w.summ);
  a.mu = (double*)(ws + w.mu);
  a.mt = (double*)(ws + w.mt);
  a.dv = (float*)(ws + w.dv);
  a.dh = (float*)(ws + w.dh);
  a.pp = (double*)(ws + w.pp);
  a.gpath = grad_path;
  a.gclock = grad_clock;
  a.gA = grad_A;
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid((a.C + a.CPW - 1) / a.CPW, a.B), blk(64);
  if (a.readout == EWS_READOUT_PREFIX) EWS_CHAIN_LAUNCH(ews::chain::k_local, grid, blk, 0, st, a);
  EWS_CHAIN_LAUNCH(ews::chain::k_carry_bwd, dim3(a.B * a.K), dim3(ews::carry_threads(a.C)), 0, st, a);
  const size_t lds = (size_t)64 * a.T * a.M * sizeof(float2);
  if (lds > 65536 && ews::allow_full_lds(a, lds) != EWS_OK) return EWS_ERR_LAUNCH;
  EWS_CHAIN_LAUNCH(ews::chain::k_full, grid, blk, lds, st, a);
  if (a.d % 4 == 0 && ((uintptr_t)grad_path & 15) == 0) {  // dv rows sit at 256-byte aligned offsets
    const size_t kt = (size_t)a.B * a.L * (a.d / 4 + 1);
    hipLaunchKernelGGL(ews::chain::k_knots4, dim3((unsigned)((kt + 255) / 256)), dim3(256), 0, st, a);
  } else {
    const size_t kt = (size_t)a.B * a.L * (a.d + 1);
    hipLaunchKernelGGL(ews::chain::k_knots, dim3((unsigned)((kt + 255) / 256)), dim3(256), 0, st, a);
  }
  if (hipGetLastError() != hipSuccess) return EWS_ERR_LAUNCH;
  hipLaunchKernelGGL(ews::chain::k_zero_a, dim3((a.d * a.d + 255) / 256), dim3(256), 0, st, a);
  if (hipGetLastError() != hipSuccess) return EWS_ERR_LAUNCH;
  hipLaunchKernelGGL(ews::chain::k_params, dim3(a.K * 3), dim3(256), 0, st, a);
  return hipGetLastError() == hipSuccess ? EWS_OK : EWS_ERR_LAUNCH;
}

}  // extern "C"
