// Closed-form local terms of uniform Jordan chains (the leaves jordan_closed / jordan_closed_tables of
// ews/core/kernels/jordan_engine.py), exact at any clock step, forward and adjoint, in float64 on the device.
//
// A chain is J = c I + eps Nil with (Nil v)_i = v_{i+1}: a real chain of n coordinates (c = lambda real), or a
// complex chain of k coordinates P_i = v_{2i} + i v_{2i+1} (c = a + ib). An analytic g gives
// g(J) = sum_{p<n} g^(p)(c) / p! (eps Nil)^p, so with x = -h c (jordan_engine.py:246-321):
//     level 1:  s1 = sum_p (-h)^p phi^(p)(x_j) / p!  w_j[p],            w_j[p]_i = eps^p P_{i+p}
//     level 2:  B_il = sum_{p,q} (-h)^(p+q) D^(p,q)(x_j, x_k) / (p! q!)  w_j[p]_i w_k[q]_l
//               A_il = the same with D^(p,q)(x_j, conj(x_k)) and conj(w_k[q]_l)  (complex chains)
// phi(y) = (e^y - 1)/y, D(x, delta) = (phi(x + delta) - phi(x)) / delta = exp[0, x, x + delta], and D^(p,q) its
// derivatives in x and delta. A complex pair block is written as real 2x2 blocks from A = U conj(W), B = U W
// (jordan_engine.py:79-91); a real chain's block is B itself. The flat layout puts chain j's coordinates at
// rows j*size .. (jordan_engine.py:281-285).
//
// Tables, as the reference evaluates them (jordan_engine.py:175-243): phi^(r)(y) by its entire series
// sum_j y^j / ((j + r + 1) j!) when |y| <= 8 (64 terms), otherwise by the recurrence phi^(r) = (e^y - r phi^(r-1))/y
// from expm1(y)/y (stable for Re y <= 0 at these orders); D^(p,q) by its expansion in delta,
// sum_s delta^s phi^(p+q+1+s)(x) / (s! (q+s+1)) (10 terms), when |delta| < 1/4, otherwise by Leibniz on
// (phi^(p)(x + delta) - phi^(p)(x)) / delta with the pair tables at x + delta (24 series terms up to |y| = 1.5).
//
// Adjoint: one wavefront per interval, a lane per chain pair (j, k); the coefficients' derivatives are the tables
// one order up (d phi^(p)/dx = phi^(p+1), dD^(p,q)/dx = D^(p+1,q), dD^(p,q)/d delta = D^(p,q+1)). Complex
// cotangents are carried as G = dl/dRe + i dl/dIm: a holomorphic factor z(c) passes G conj(z'(c)) to c, an
// antiholomorphic one z(conj(c)) passes conj(G) z'. The lanes' partials are summed per chain in a fixed order.
#include <hip/hip_runtime.h>

#include "ews_hip.h"

namespace ews {
namespace jordan {

// ------------------------------------------------------------------------------------------------ complex double
struct zd {
  double re, im;
};
__device__ __forceinline__ zd Z(double r, double i = 0.0) { return zd{r, i}; }
__device__ __forceinline__ zd operator+(zd a, zd b) { return zd{a.re + b.re, a.im + b.im}; }
__device__ __forceinline__ zd operator-(zd a, zd b) { return zd{a.re - b.re, a.im - b.im}; }
__device__ __forceinline__ zd operator-(zd a) { return zd{-a.re, -a.im}; }
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
__device__ __forceinline__ double zabs(zd a) { return hypot(a.re, a.im); }
__device__ __forceinline__ zd zdiv(zd a, zd b) {  // Smith's algorithm
  if (fabs(b.re) >= fabs(b.im)) {
    const double r = b.im / b.re, den = b.re + b.im * r;
    return zd{(a.re + a.im * r) / den, (a.im - a.re * r) / den};
  }
  const double r = b.re / b.im, den = b.im + b.re * r;
  return zd{(a.re * r + a.im) / den, (a.im * r - a.re) / den};
}
__device__ __forceinline__ zd zexp(zd a) {
  const double m = exp(a.re);
  return zd{m * cos(a.im), m * sin(a.im)};
}
__device__ __forceinline__ double redot(zd a, zd b) { return a.re * b.re + a.im * b.im; }  // Re(conj(a) b)

__device__ __forceinline__ double ipow(double x, int p) {
  double r = 1.0;
  for (int i = 0; i < p; ++i) r *= x;
  return r;
}
__device__ __forceinline__ double fact(int n) {
  double r = 1.0;
  for (int i = 2; i <= n; ++i) r *= (double)i;
  return r;
}

// phi^(r)(y), r = 0..R
template <int R>
__device__ __forceinline__ void phi_table(zd y, double sw, int nterms, zd* out) {
#pragma unroll
  for (int r = 0; r <= R; ++r) out[r] = Z(0.0);
  if (zabs(y) <= sw) {
    zd t = Z(1.0);  // y^j / j!
    for (int j = 0; j < nterms; ++j) {
#pragma unroll
      for (int r = 0; r <= R; ++r) out[r] += (1.0 / (double)(j + r + 1)) * t;
      t = (1.0 / (double)(j + 1)) * (t * y);
    }
  } else {
    const zd e = zexp(y);
    out[0] = zdiv(e - Z(1.0), y);
#pragma unroll
    for (int r = 1; r <= R; ++r) out[r] = zdiv(e - (double)r * out[r - 1], y);
  }
}

constexpr double kPhiSwitch = 8.0;
constexpr int kPhiTerms = 64;
constexpr double kPairSwitch = 1.5;
constexpr int kPairTerms = 24;
constexpr int kPairS = 10;
constexpr double kPairDelta0 = 0.25;

// D^(p,q)(x, delta) for p <= PM, q <= QM; tabx = phi^(r)(x) for r = 0..PM + QM + kPairS
template <int PM, int QM>
__device__ __forceinline__ void pair_table(const zd* tabx, zd x, zd delta, zd (*D)[QM + 1]) {
  if (zabs(delta) < kPairDelta0) {
    zd dp[kPairS];  // delta^s / s!
    dp[0] = Z(1.0);
#pragma unroll
    for (int s = 1; s < kPairS; ++s) dp[s] = (1.0 / (double)s) * (dp[s - 1] * delta);
#pragma unroll
    for (int p = 0; p <= PM; ++p)
#pragma unroll
      for (int q = 0; q <= QM; ++q) {
        zd acc = Z(0.0);
#pragma unroll
        for (int s = 0; s < kPairS; ++s) acc += (1.0 / (double)(q + s + 1)) * (dp[s] * tabx[p + q + 1 + s]);
        D[p][q] = acc;
      }
  } else {
    zd txd[PM + QM + 1];
    phi_table<PM + QM>(x + delta, kPairSwitch, kPairTerms, txd);
    const zd inv = zdiv(Z(1.0), delta);
    zd ip[QM + 2];  // inv^m
    ip[0] = Z(1.0);
#pragma unroll
    for (int m = 1; m <= QM + 1; ++m) ip[m] = ip[m - 1] * inv;
#pragma unroll
    for (int p = 0; p <= PM; ++p)
#pragma unroll
      for (int q = 0; q <= QM; ++q) {
        zd acc = Z(0.0);
#pragma unroll
        for (int s = 0; s <= q; ++s) {
          const zd F = s == 0 ? txd[p] - tabx[p] : txd[p + s];
          double binom = 1.0;
          for (int u = 0; u < s; ++u) binom = binom * (double)(q - u) / (double)(u + 1);
          const double coef = binom * (((q - s) & 1) ? -1.0 : 1.0) * fact(q - s);
          acc += coef * (ip[q - s + 1] * F);
        }
        D[p][q] = acc;
      }
  }
}

// ------------------------------------------------------------------------------------------------ arguments
struct JArgs {
  int B, L, n, d, N, K, cplx, size;
  const float* path;
  const float* clock;
  const float* A;
  float* levels;
  const float* glevels;
  float* dv;     // (B, n, d) per-interval path cotangents
  float* dh;     // (B, n) per-interval step cotangents
  double* pp;    // (B, n, K, 3) chain-parameter partials: Re c, Im c, eps
  float* gpath;
  float* gclock;
  float* gA;
};

// the chain's coordinates in the interval, its eigenvalue and coupling
template <bool CPLX, int NC>
__device__ __forceinline__ void load_chain(const JArgs& a, size_t row, int j, zd* P, zd& c, double& eps) {
  constexpr int CS = CPLX ? 2 * NC : NC;
  const int f = j * CS;
  const float* x0 = a.path + row * a.d;
  const float* x1 = x0 + a.d;
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    if (CPLX) {
      P[i] = Z((double)x1[f + 2 * i] - (double)x0[f + 2 * i], (double)x1[f + 2 * i + 1] - (double)x0[f + 2 * i + 1]);
    } else {
      P[i] = Z((double)x1[f + i] - (double)x0[f + i]);
    }
  }
  eps = 0.0;  // a chain of one coordinate (a diagonal entry, a rotation plane) has no coupling
  if (CPLX) {
    c = Z((double)a.A[f * a.d + f], (double)a.A[(f + 1) * a.d + f]);
    if (NC > 1) eps = (double)a.A[f * a.d + f + 2];
  } else {
    c = Z((double)a.A[f * a.d + f]);
    if (NC > 1) eps = (double)a.A[f * a.d + f + 1];
  }
}

// w[p]_i = eps^p P_{i+p}
template <int NC>
__device__ __forceinline__ zd wv(const zd* P, double eps, int p, int i) {
  return i + p < NC ? ipow(eps, p) * P[i + p] : Z(0.0);
}

// ------------------------------------------------------------------------------------------------ forward
// one thread per (interval, chain pair); the pairs (j, 0) also write chain j's level 1
template <bool CPLX, int NC>
__global__ __launch_bounds__(128) void k_fwd(JArgs a) {
  constexpr int CS = CPLX ? 2 * NC : NC;
  constexpr int RX = 2 * (NC - 1) + kPairS;  // phi^(r)(x_j) orders of the pair expansion
  const int K = a.K, KK = K * K;
  const size_t tid = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (tid >= (size_t)a.B * a.n * KK) return;
  const int pr = (int)(tid % KK), j = pr / K, k = pr % K;
  const size_t it = tid / KK, b = it / a.n, t = it % a.n;
  const size_t row = b * a.L + t;
  const double h = (double)a.clock[row + 1] - (double)a.clock[row];
  zd Pj[NC], Pk[NC], cjv, ckv;
  double ej, ek;
  load_chain<CPLX, NC>(a, row, j, Pj, cjv, ej);
  load_chain<CPLX, NC>(a, row, k, Pk, ckv, ek);
  const zd xj = (-h) * cjv, xk = (-h) * ckv;
  zd tabx[RX + 1];
  phi_table<RX>(xj, kPhiSwitch, kPhiTerms, tabx);
  const int Dl = a.d + (a.N == 2 ? a.d * a.d : 0);
  float* out = a.levels + it * Dl;
  if (k == 0) {
#pragma unroll
    for (int i = 0; i < NC; ++i) {
      zd s = Z(0.0);
#pragma unroll
      for (int p = 0; p < NC; ++p) s += (ipow(-h, p) / fact(p)) * (tabx[p] * wv<NC>(Pj, ej, p, i));
      if (CPLX) {
        out[j * CS + 2 * i] = (float)s.re;
        out[j * CS + 2 * i + 1] = (float)s.im;
      } else {
        out[j * CS + i] = (float)s.re;
      }
    }
  }
  if (a.N < 2) return;
  zd QB[NC][NC], QA[NC][NC];
  {
    zd D[NC][NC];
    pair_table<NC - 1, NC - 1>(tabx, xj, xk, D);
#pragma unroll
    for (int i = 0; i < NC; ++i)
#pragma unroll
      for (int l = 0; l < NC; ++l) {
        zd acc = Z(0.0);
#pragma unroll
        for (int p = 0; p < NC; ++p)
#pragma unroll
          for (int q = 0; q < NC; ++q)
            acc += (ipow(-h, p + q) / (fact(p) * fact(q))) * (D[p][q] * (wv<NC>(Pj, ej, p, i) * wv<NC>(Pk, ek, q, l)));
        QB[i][l] = acc;
      }
  }
  if (CPLX) {
    zd D[NC][NC];
    pair_table<NC - 1, NC - 1>(tabx, xj, cj(xk), D);
#pragma unroll
    for (int i = 0; i < NC; ++i)
#pragma unroll
      for (int l = 0; l < NC; ++l) {
        zd acc = Z(0.0);
#pragma unroll
        for (int p = 0; p < NC; ++p)
#pragma unroll
          for (int q = 0; q < NC; ++q)
            acc += (ipow(-h, p + q) / (fact(p) * fact(q))) *
                   (D[p][q] * (wv<NC>(Pj, ej, p, i) * cj(wv<NC>(Pk, ek, q, l))));
        QA[i][l] = acc;
      }
  }
  float* o2 = out + a.d;
#pragma unroll
  for (int i = 0; i < NC; ++i)
#pragma unroll
    for (int l = 0; l < NC; ++l) {
      if (CPLX) {
        const int r0 = j * CS + 2 * i, c0 = k * CS + 2 * l;
        o2[r0 * a.d + c0] = (float)(0.5 * (QA[i][l].re + QB[i][l].re));
        o2[r0 * a.d + c0 + 1] = (float)(0.5 * (QB[i][l].im - QA[i][l].im));
        o2[(r0 + 1) * a.d + c0] = (float)(0.5 * (QA[i][l].im + QB[i][l].im));
        o2[(r0 + 1) * a.d + c0 + 1] = (float)(0.5 * (QA[i][l].re - QB[i][l].re));
      } else {
        o2[(j * CS + i) * a.d + k * CS + l] = (float)QB[i][l].re;
      }
    }
}

// ------------------------------------------------------------------------------------------------ adjoint
// Cotangents of one pair part Q_il = sum_pq c_pq w_j[p]_i (conj) w_k[q]_l, c_pq = s_pq D^(p,q)(x_j, delta) with
// s_pq = (-h)^(p+q) / (p! q!) and delta = x_k (B part) or conj(x_k) (A part, ANTI): accumulates the P cotangents
// of both chains (through w), their eps cotangents, the c cotangents and the step cotangent.
template <int NC, bool ANTI>
__device__ __forceinline__ void pair_adjoint(const zd (*G)[NC], const zd (*D)[NC + 1], double h, const zd* Pj,
                                             const zd* Pk, double ej, double ek, zd cjv, zd ckv, zd* dPj, zd* dPk,
                                             double& dej, double& dek, zd& gcj, zd& gck, double& dh) {
  const zd ckd = ANTI ? cj(ckv) : ckv;  // the node delta = -h ckd
#pragma unroll
  for (int p = 0; p < NC; ++p)
#pragma unroll
    for (int q = 0; q < NC; ++q) {
      const double s = ipow(-h, p + q) / (fact(p) * fact(q));
      const double ds = (p + q) ? -(double)(p + q) * ipow(-h, p + q - 1) / (fact(p) * fact(q)) : 0.0;
      const zd c = s * D[p][q];
      zd Gc = Z(0.0);
#pragma unroll
      for (int i = 0; i < NC; ++i) {
        const zd wj = wv<NC>(Pj, ej, p, i);
#pragma unroll
        for (int l = 0; l < NC; ++l) {
          const zd wk = wv<NC>(Pk, ek, q, l);
          const zd g = G[i][l];
          zd Gwj, Gwk;
          if (ANTI) {  // z = c wj conj(wk)
            Gc += g * (cj(wj) * wk);
            Gwj = g * (cj(c) * wk);
            Gwk = cj(g) * (c * wj);
          } else {  // z = c wj wk
            Gc += g * cj(wj * wk);
            Gwj = g * cj(c * wk);
            Gwk = g * cj(c * wj);
          }
          if (i + p < NC) {
            dPj[i + p] += ipow(ej, p) * Gwj;
            if (p) dej += (double)p * ipow(ej, p - 1) * redot(Gwj, Pj[i + p]);
          }
          if (l + q < NC) {
            dPk[l + q] += ipow(ek, q) * Gwk;
            if (q) dek += (double)q * ipow(ek, q - 1) * redot(Gwk, Pk[l + q]);
          }
        }
      }
      // c_pq(h, c_j, c_k): dc/dc_j = s (-h) D^(p+1,q) (holomorphic), dc/d ckd = s (-h) D^(p,q+1)
      gcj += Gc * cj((s * (-h)) * D[p + 1][q]);
      const zd fk = (s * (-h)) * D[p][q + 1];
      gck += ANTI ? cj(Gc) * fk : Gc * cj(fk);
      const zd dcdh = ds * D[p][q] + s * (D[p + 1][q] * (-cjv) + D[p][q + 1] * (-ckd));
      dh += redot(Gc, dcdh);
    }
}

template <bool CPLX, int NC>
__global__ __launch_bounds__(64) void k_bwd(JArgs a) {
  constexpr int CS = CPLX ? 2 * NC : NC;
  constexpr int RX = 2 * NC + kPairS;  // one order above the forward's
  __shared__ zd s_dvj[64][NC], s_dvk[64][NC], s_gcj[64], s_gck[64];
  __shared__ double s_dej[64], s_dek[64], s_dh[64];
  const int K = a.K, KK = K * K, lane = threadIdx.x;
  const bool act = lane < KK;
  const int j = act ? lane / K : 0, k = act ? lane % K : 0;
  for (size_t it = blockIdx.x; it < (size_t)a.B * a.n; it += gridDim.x) {
    const size_t b = it / a.n, t = it % a.n, row = b * a.L + t;
    zd dPj[NC], dPk[NC], gcj = Z(0.0), gck = Z(0.0);
    double dej = 0.0, dek = 0.0, dh = 0.0;
#pragma unroll
    for (int i = 0; i < NC; ++i) dPj[i] = dPk[i] = Z(0.0);
    if (act) {
      const double h = (double)a.clock[row + 1] - (double)a.clock[row];
      zd Pj[NC], Pk[NC], cjv, ckv;
      double ej, ek;
      load_chain<CPLX, NC>(a, row, j, Pj, cjv, ej);
      load_chain<CPLX, NC>(a, row, k, Pk, ckv, ek);
      const zd xj = (-h) * cjv, xk = (-h) * ckv;
      zd tabx[RX + 1];
      phi_table<RX>(xj, kPhiSwitch, kPhiTerms, tabx);
      const int Dl = a.d + (a.N == 2 ? a.d * a.d : 0);
      const float* gl = a.glevels + it * Dl;
      if (a.N == 2) {
        const float* g2 = gl + a.d;
        zd GB[NC][NC], GA[NC][NC];
#pragma unroll
        for (int i = 0; i < NC; ++i)
#pragma unroll
          for (int l = 0; l < NC; ++l) {
            if (CPLX) {
              const int r0 = j * CS + 2 * i, c0 = k * CS + 2 * l;
              const double g00 = g2[r0 * a.d + c0], g01 = g2[r0 * a.d + c0 + 1];
              const double g10 = g2[(r0 + 1) * a.d + c0], g11 = g2[(r0 + 1) * a.d + c0 + 1];
              GA[i][l] = Z(0.5 * (g00 + g11), 0.5 * (g10 - g01));
              GB[i][l] = Z(0.5 * (g00 - g11), 0.5 * (g01 + g10));
            } else {
              GB[i][l] = Z((double)g2[(j * CS + i) * a.d + k * CS + l]);
            }
          }
        {
          zd D[NC + 1][NC + 1];
          pair_table<NC, NC>(tabx, xj, xk, D);
          pair_adjoint<NC, false>(GB, D, h, Pj, Pk, ej, ek, cjv, ckv, dPj, dPk, dej, dek, gcj, gck, dh);
        }
        if (CPLX) {
          zd D[NC + 1][NC + 1];
          pair_table<NC, NC>(tabx, xj, cj(xk), D);
          pair_adjoint<NC, true>(GA, D, h, Pj, Pk, ej, ek, cjv, ckv, dPj, dPk, dej, dek, gcj, gck, dh);
        }
      }
      if (k == 0) {  // level 1 of chain j: s1_i = sum_p a_p w_j[p]_i, a_p = (-h)^p phi^(p)(x_j) / p!
        zd G1[NC];
#pragma unroll
        for (int i = 0; i < NC; ++i)
          G1[i] = CPLX ? Z((double)gl[j * CS + 2 * i], (double)gl[j * CS + 2 * i + 1]) : Z((double)gl[j * CS + i]);
#pragma unroll
        for (int p = 0; p < NC; ++p) {
          const double s = ipow(-h, p) / fact(p);
          const double ds = p ? -(double)p * ipow(-h, p - 1) / fact(p) : 0.0;
          const zd ap = s * tabx[p];
          zd Ga = Z(0.0);
#pragma unroll
          for (int i = 0; i < NC; ++i) {
            const zd w = wv<NC>(Pj, ej, p, i);
            Ga += G1[i] * cj(w);
            const zd Gw = G1[i] * cj(ap);
            if (i + p < NC) {
              dPj[i + p] += ipow(ej, p) * Gw;
              if (p) dej += (double)p * ipow(ej, p - 1) * redot(Gw, Pj[i + p]);
            }
          }
          gcj += Ga * cj((s * (-h)) * tabx[p + 1]);
          dh += redot(Ga, ds * tabx[p] + s * (tabx[p + 1] * (-cjv)));
        }
      }
    }
#pragma unroll
    for (int i = 0; i < NC; ++i) {
      s_dvj[lane][i] = dPj[i];
      s_dvk[lane][i] = dPk[i];
    }
    s_gcj[lane] = gcj;
    s_gck[lane] = gck;
    s_dej[lane] = dej;
    s_dek[lane] = dek;
    s_dh[lane] = dh;
    __syncthreads();
    if (lane < K) {  // chain m = lane: its shares as the first factor (pairs (m, k)) and as the second (pairs (j, m))
      const int m = lane;
      zd dP[NC], gc = Z(0.0);
      double de = 0.0;
#pragma unroll
      for (int i = 0; i < NC; ++i) dP[i] = Z(0.0);
      for (int q = 0; q < K; ++q) {
#pragma unroll
        for (int i = 0; i < NC; ++i) dP[i] += s_dvj[m * K + q][i];
        gc += s_gcj[m * K + q];
        de += s_dej[m * K + q];
      }
      for (int q = 0; q < K; ++q) {
#pragma unroll
        for (int i = 0; i < NC; ++i) dP[i] += s_dvk[q * K + m][i];
        gc += s_gck[q * K + m];
        de += s_dek[q * K + m];
      }
      float* dvo = a.dv + it * a.d + m * CS;
#pragma unroll
      for (int i = 0; i < NC; ++i) {
        if (CPLX) {
          dvo[2 * i] = (float)dP[i].re;
          dvo[2 * i + 1] = (float)dP[i].im;
        } else {
          dvo[i] = (float)dP[i].re;
        }
      }
      double* ppo = a.pp + (it * K + m) * 3;
      ppo[0] = gc.re;
      ppo[1] = gc.im;
      ppo[2] = de;
    }
    if (lane == 0) {
      double acc = 0.0;
      for (int q = 0; q < KK; ++q) acc += s_dh[q];
      a.dh[it] = (float)acc;
    }
    __syncthreads();
  }
}

// knot gradients from the interval cotangents: dX_t = dv_{t-1} - dv_t, dtheta_t = dh_{t-1} - dh_t
__global__ void k_knots(JArgs a) {
  const size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  const size_t per = (size_t)a.L * (a.d + 1);
  if (e >= (size_t)a.B * per) return;
  const size_t b = e / per, r = e % per, t = r / (a.d + 1), ch = r % (a.d + 1);
  if (ch < (size_t)a.d) {
    const float lo = t > 0 ? a.dv[(b * a.n + t - 1) * a.d + ch] : 0.0f;
    const float hi = t < (size_t)a.n ? a.dv[(b * a.n + t) * a.d + ch] : 0.0f;
    a.gpath[(b * a.L + t) * a.d + ch] = lo - hi;
  } else if (a.gclock) {
    const float lo = t > 0 ? a.dh[b * a.n + t - 1] : 0.0f;
    const float hi = t < (size_t)a.n ? a.dh[b * a.n + t] : 0.0f;
    a.gclock[b * a.L + t] = lo - hi;
  }
}

// grad_A: zero, then the chain entries from the per-interval partials (one workgroup per chain and component,
// a fixed order of float64 sums)
__global__ void k_zero_a(JArgs a) {
  const int e = blockIdx.x * blockDim.x + threadIdx.x;
  if (e < a.d * a.d) a.gA[e] = 0.0f;
}
__global__ __launch_bounds__(256) void k_params(JArgs a) {
  __shared__ double red[256];
  const int m = blockIdx.x / 3, comp = blockIdx.x % 3, tid = threadIdx.x;
  // a real chain has no imaginary part, a chain of one coordinate no coupling (uniform across the workgroup)
  if ((!a.cplx && comp == 1) || (comp == 2 && a.size == (a.cplx ? 2 : 1))) return;
  const size_t tot = (size_t)a.B * a.n;
  double acc = 0.0;
  for (size_t it = tid; it < tot; it += 256) acc += a.pp[(it * a.K + m) * 3 + comp];
  red[tid] = acc;
  __syncthreads();
  for (int o = 128; o > 0; o >>= 1) {
    if (tid < o) red[tid] += red[tid + o];
    __syncthreads();
  }
  if (tid == 0) {
    const int f = m * a.size;
    int idx;
    if (comp == 0) idx = f * a.d + f;                             // lambda / a
    else if (comp == 1) idx = (f + 1) * a.d + f;                  // b
    else idx = a.cplx ? f * a.d + f + 2 : f * a.d + f + 1;        // eps
    a.gA[idx] = (float)red[0];
  }
}

}  // namespace jordan

namespace {

using jordan::JArgs;

int check_desc(const ews_jordan_desc* s, int& nc) {
  if (!s) return EWS_ERR_NULL;
  if (s->batch < 1 || s->length < 2 || s->dim < 1 || s->dim > 16) return EWS_ERR_SHAPE;
  if (s->depth != 1 && s->depth != 2) return EWS_ERR_DEPTH;
  if (s->kind == EWS_JORDAN_REAL) {
    if (s->size < 1 || s->size > 4) return EWS_ERR_OPTION;
    nc = s->size;
  } else if (s->kind == EWS_JORDAN_COMPLEX) {
    if (s->size != 2 && s->size != 4 && s->size != 6 && s->size != 8) return EWS_ERR_OPTION;
    nc = s->size / 2;
  } else {
    return EWS_ERR_OPTION;
  }
  if (s->dim % s->size) return EWS_ERR_SHAPE;
  if (s->dim / s->size > 8) return EWS_ERR_SHAPE;  // the adjoint's wavefront holds every chain pair (K^2 <= 64)
  return EWS_OK;
}

size_t al256(size_t x) { return (x + 255) & ~(size_t)255; }

JArgs make(const ews_jordan_desc* s) {
  JArgs a{};
  a.B = s->batch;
  a.L = s->length;
  a.n = s->length - 1;
  a.d = s->dim;
  a.N = s->depth;
  a.size = s->size;
  a.K = s->dim / s->size;
  a.cplx = s->kind == EWS_JORDAN_COMPLEX;
  return a;
}

template <bool CPLX>
int launch_fwd(const JArgs& a, int nc, hipStream_t st) {
  const size_t tot = (size_t)a.B * a.n * a.K * a.K;
  const dim3 grid((unsigned)((tot + 127) / 128)), blk(128);
  if (nc == 1) hipLaunchKernelGGL((jordan::k_fwd<CPLX, 1>), grid, blk, 0, st, a);
  else if (nc == 2) hipLaunchKernelGGL((jordan::k_fwd<CPLX, 2>), grid, blk, 0, st, a);
  else if (nc == 3) hipLaunchKernelGGL((jordan::k_fwd<CPLX, 3>), grid, blk, 0, st, a);
  else hipLaunchKernelGGL((jordan::k_fwd<CPLX, 4>), grid, blk, 0, st, a);
  return hipGetLastError() == hipSuccess ? EWS_OK : EWS_ERR_LAUNCH;
}

template <bool CPLX>
int launch_bwd(const JArgs& a, int nc, hipStream_t st) {
  const size_t tot = (size_t)a.B * a.n;
  const dim3 grid((unsigned)(tot < 65536 ? tot : 65536)), blk(64);
  if (nc == 1) hipLaunchKernelGGL((jordan::k_bwd<CPLX, 1>), grid, blk, 0, st, a);
  else if (nc == 2) hipLaunchKernelGGL((jordan::k_bwd<CPLX, 2>), grid, blk, 0, st, a);
  else if (nc == 3) hipLaunchKernelGGL((jordan::k_bwd<CPLX, 3>), grid, blk, 0, st, a);
  else hipLaunchKernelGGL((jordan::k_bwd<CPLX, 4>), grid, blk, 0, st, a);
  return hipGetLastError() == hipSuccess ? EWS_OK : EWS_ERR_LAUNCH;
}

}  // namespace
}  // namespace ews

extern "C" {

int ews_jordan_local_terms(const ews_jordan_desc* desc, const float* path, const float* clock, const float* A,
                           float* levels, ews_stream_t stream) {
  int nc = 0;
  const int rc = ews::check_desc(desc, nc);
  if (rc != EWS_OK) return rc;
  if (!path || !clock || !A || !levels) return EWS_ERR_NULL;
  ews::JArgs a = ews::make(desc);
  a.path = path;
  a.clock = clock;
  a.A = A;
  a.levels = levels;
  return a.cplx ? ews::launch_fwd<true>(a, nc, (hipStream_t)stream) : ews::launch_fwd<false>(a, nc, (hipStream_t)stream);
}

size_t ews_jordan_workspace_bytes(const ews_jordan_desc* desc) {
  int nc = 0;
  if (ews::check_desc(desc, nc) != EWS_OK) return 0;
  const size_t bn = (size_t)desc->batch * (desc->length - 1), K = desc->dim / desc->size;
  return ews::al256(bn * desc->dim * 4) + ews::al256(bn * 4) + ews::al256(bn * K * 3 * 8);
}

int ews_jordan_local_terms_backward(const ews_jordan_desc* desc, const float* path, const float* clock,
                                    const float* A, const float* grad_levels, float* grad_path, float* grad_clock,
                                    float* grad_A, void* workspace, ews_stream_t stream) {
  int nc = 0;
  const int rc = ews::check_desc(desc, nc);
  if (rc != EWS_OK) return rc;
  if (!path || !clock || !A || !grad_levels || !grad_path || !grad_A || !workspace) return EWS_ERR_NULL;
  ews::JArgs a = ews::make(desc);
  a.path = path;
  a.clock = clock;
  a.A = A;
  a.glevels = grad_levels;
  a.gpath = grad_path;
  a.gclock = grad_clock;
  a.gA = grad_A;
  const size_t bn = (size_t)a.B * a.n;
  char* w = (char*)workspace;
  a.dv = (float*)w;
  a.dh = (float*)(w + ews::al256(bn * a.d * 4));
  a.pp = (double*)(w + ews::al256(bn * a.d * 4) + ews::al256(bn * 4));
  hipStream_t st = (hipStream_t)stream;
  int r = a.cplx ? ews::launch_bwd<true>(a, nc, st) : ews::launch_bwd<false>(a, nc, st);
  if (r != EWS_OK) return r;
  const size_t kt = (size_t)a.B * a.L * (a.d + 1);
  hipLaunchKernelGGL(ews::jordan::k_knots, dim3((unsigned)((kt + 255) / 256)), dim3(256), 0, st, a);
  if (hipGetLastError() != hipSuccess) return EWS_ERR_LAUNCH;
  hipLaunchKernelGGL(ews::jordan::k_zero_a, dim3((a.d * a.d + 255) / 256), dim3(256), 0, st, a);
  if (hipGetLastError() != hipSuccess) return EWS_ERR_LAUNCH;
  hipLaunchKernelGGL(ews::jordan::k_params, dim3(a.K * 3), dim3(256), 0, st, a);
  return hipGetLastError() == hipSuccess ? EWS_OK : EWS_ERR_LAUNCH;
}

}  // extern "C"
