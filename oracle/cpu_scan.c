/* CPU restatement of the reference's rotation-plane EWS path: closed-form plane leaf + sequential modified-Chen
 * combine, forward and adjoint. TEST INFRASTRUCTURE ONLY: used as the float64 full-size checker by tests/ and,
 * built with REAL=float, as the CPU baseline timed by bench.py. The product never links or calls it.
 *
 * Restates, in the reference's real 2x2-block formulation:
 *   local terms   ews/core/kernels/plane_engine.py:134-152 (phi, divided differences :29-78, blocks :95-116)
 *   combine       plane_engine.py:164-170 (_combine_n2: S2 <- R S2 R^T + (R S1) s1^T + s2), the sequential
 *                 form of ews/core/chen_scan.py:124-152 / the lax.scan branch of plane_prefix (:188-196)
 *   flows         per interval, or one shared step (ews/core/chen_scan.py:155-168)
 *   readout       prefix rows with the level-0 constant (ews/core/output_format.py:22-30)
 * Gradients: the adjoint of the block recursion; the scalar coefficients' derivatives in (h, d, w) analytically,
 * by the chain rule through the nodes x = -h conj(z_j) and delta = -h conj(z_k) (B) or -h z_k (A), with
 *   dphi/dx = exp[0, x, x],  dD/dx = int_0^1 a^2 phi(delta a) e^{x a} da,  dD/ddelta = int_0^1 a^2 phi'(delta a) e^{x a} da
 * (D(x, delta) = int_0^1 a phi(delta a) e^{x a} da, the simplex integral with the inner variable done in closed
 * form), evaluated by 24-point Gauss-Legendre quadrature. No finite differences: a central difference of the
 * direct divided-difference branch loses ~1e-13 / step to cancellation.
 */
#include <complex.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifndef REAL
#define REAL double
#endif

typedef double complex cplx;

/* phi family (plane_engine.py:23-78), float64 guards */
static cplx phi(cplx x) {
  if (cabs(x) < 1e-3) return 1 + x * (1.0 / 2 + x * (1.0 / 6 + x * (1.0 / 24 + x * (1.0 / 120 + x / 720))));
  return (cexp(x) - 1) / x;
}
static cplx dphi(cplx x) {
  if (cabs(x) < 3e-2) return 1.0 / 2 + x * (1.0 / 3 + x * (1.0 / 8 + x * (1.0 / 30 + x * (1.0 / 144 + x / 840))));
  return (cexp(x) * (x - 1) + 1) / (x * x);
}
static cplx d2phi(cplx x) {
  if (cabs(x) < 1e-1) return 1.0 / 3 + x * (1.0 / 4 + x * (1.0 / 10 + x * (1.0 / 36 + x * (1.0 / 168 + x / 960))));
  return (cexp(x) * (x * x - 2 * x + 2) - 2) / (x * x * x);
}
static cplx d3phi(cplx x) {
  if (cabs(x) < 2.5e-1)
    return 1.0 / 4 + x * (1.0 / 5 + x * (1.0 / 12 + x * (1.0 / 42 + x * (1.0 / 192 + x / 1080))));
  return (cexp(x) * (x * x * x - 3 * x * x + 6 * x - 6) + 6) / (x * x * x * x);
}
static cplx divdiff(cplx x, cplx delta) {
  if (cabs(delta) < 4e-4) return dphi(x) + delta * (d2phi(x) / 2 + delta * d3phi(x) / 6);
  return (phi(x + delta) - phi(x)) / delta;
}

/* 24-point Gauss-Legendre nodes / weights on [0, 1] (computed once by Newton iteration on P_24) */
#define GL_N 24
static double gl_x[GL_N], gl_w[GL_N];
static int gl_ready = 0;
static void gl_init(void) {
  if (gl_ready) return;
  const int n = GL_N;
  for (int i = 0; i < n; ++i) {
    double x = cos(M_PI * (i + 0.75) / (n + 0.5)), dp = 0.0;
    for (int it = 0; it < 100; ++it) {
      double p0 = 1.0, p1 = x;
      for (int k = 2; k <= n; ++k) {
        const double p2 = ((2.0 * k - 1.0) * x * p1 - (k - 1.0) * p0) / k;
        p0 = p1;
        p1 = p2;
      }
      dp = n * (x * p1 - p0) / (x * x - 1.0);
      const double dx = p1 / dp;
      x -= dx;
      if (fabs(dx) < 1e-16) break;
    }
    gl_x[i] = 0.5 * (1.0 - x);
    gl_w[i] = 1.0 / ((1.0 - x * x) * dp * dp);
  }
  gl_ready = 1;
}

/* partial derivatives of D(x, delta) = int_0^1 a phi(delta a) e^{x a} da */
static void divdiff_derivs(cplx x, cplx delta, cplx* Dx, cplx* Dd) {
  cplx sx = 0, sd = 0;
  for (int i = 0; i < GL_N; ++i) {
    const double a = gl_x[i];
    const cplx e = cexp(x * a) * (gl_w[i] * a * a);
    sx += e * phi(delta * a);
    sd += e * dphi(delta * a);
  }
  *Dx = sx;
  *Dd = sd;
}

/* coefficients of one interval for planes j, k: rho_j, phi_j, IA_jk, IB_jk (complex) */
typedef struct {
  cplx rho, ph, IA, IB;
} Coef;

static cplx zc(double d, double w) { return d - I * w; }  /* conj(z), z = d + i w */

static cplx c_rho(double h, double dj, double wj) { return cexp(-h * zc(dj, wj)); }
static cplx c_phi(double h, double dj, double wj) { return phi(-h * zc(dj, wj)); }
static cplx c_IA(double h, double dj, double wj, double dk, double wk) {
  return divdiff(-h * zc(dj, wj), -h * (dk + I * wk));
}
static cplx c_IB(double h, double dj, double wj, double dk, double wk) {
  return divdiff(-h * zc(dj, wj), -h * zc(dk, wk));
}

/* A_j real 2x2 of exp(-h A_j) from rho: [[Re, -Im], [Im, Re]] (rot_blocks, plane_engine.py:95-100) */
static void rotm(cplx rho, double R[4]) {
  R[0] = creal(rho);
  R[1] = -cimag(rho);
  R[2] = cimag(rho);
  R[3] = creal(rho);
}

/* real 2x2 block from complex A = u conj(w), B = u w parts (_blocks_from_AB, plane_engine.py:111-116) */
static void blocks_from_AB(cplx A, cplx B, double q[4]) {
  q[0] = (creal(A) + creal(B)) / 2;
  q[1] = (cimag(B) - cimag(A)) / 2;
  q[2] = (cimag(A) + cimag(B)) / 2;
  q[3] = (creal(A) - creal(B)) / 2;
}

#define IDX2(j, k, a, b) ((((2 * (j) + (a)) * m) + 2 * (k) + (b)))

/* flow step actually used at interval t (cached modes share one step) */
static double flow_h(const REAL* th, int t, int L, int flow_mode) {
  if (flow_mode == 0) return (double)th[t + 1] - (double)th[t];
  if (flow_mode == 1) return (double)th[1] - (double)th[0];
  return (double)th[2] - (double)th[1];
}

/* one sample: forward prefix into states (L-1, m + m*m) in double; returns nothing */
static void planes_forward_one(int L, int m, const REAL* X, const REAL* th, const double* dw, int flow_mode,
                               double* states) {
  const int K = m / 2, D = m + m * m;
  double* S = calloc(D, sizeof(double));
  double* Sn = calloc(D, sizeof(double));
  for (int t = 0; t < L - 1; ++t) {
    const double h = (double)th[t + 1] - (double)th[t];
    const double hf = flow_h(th, t, L, flow_mode);
    double R[32][4], s1[32][2], c[32][2];
    cplx p[32];
    for (int j = 0; j < K; ++j) {
      p[j] = ((double)X[(t + 1) * m + 2 * j] - (double)X[t * m + 2 * j]) +
             I * ((double)X[(t + 1) * m + 2 * j + 1] - (double)X[t * m + 2 * j + 1]);
      rotm(c_rho(hf, dw[2 * j], dw[2 * j + 1]), R[j]);
      const cplx s = c_phi(h, dw[2 * j], dw[2 * j + 1]) * p[j];
      s1[j][0] = creal(s);
      s1[j][1] = cimag(s);
      c[j][0] = R[j][0] * S[2 * j] + R[j][1] * S[2 * j + 1];
      c[j][1] = R[j][2] * S[2 * j] + R[j][3] * S[2 * j + 1];
    }
    for (int j = 0; j < K; ++j)
      for (int k = 0; k < K; ++k) {
        const cplx A = c_IA(h, dw[2 * j], dw[2 * j + 1], dw[2 * k], dw[2 * k + 1]) * p[j] * conj(p[k]);
        const cplx B = c_IB(h, dw[2 * j], dw[2 * j + 1], dw[2 * k], dw[2 * k + 1]) * p[j] * p[k];
        double q[4];
        blocks_from_AB(A, B, q);
        /* R_j S_jk R_k^T */
        double P[4], T[4];
        for (int a = 0; a < 2; ++a)
          for (int b = 0; b < 2; ++b) P[2 * a + b] = S[m + IDX2(j, k, a, b)];
        for (int a = 0; a < 2; ++a)
          for (int b = 0; b < 2; ++b) T[2 * a + b] = R[j][2 * a] * P[b] + R[j][2 * a + 1] * P[2 + b];
        for (int a = 0; a < 2; ++a)
          for (int b = 0; b < 2; ++b)
            Sn[m + IDX2(j, k, a, b)] =
                T[2 * a] * R[k][2 * b] + T[2 * a + 1] * R[k][2 * b + 1] + c[j][a] * s1[k][b] + q[2 * a + b];
      }
    for (int j = 0; j < K; ++j) {
      Sn[2 * j] = c[j][0] + s1[j][0];
      Sn[2 * j + 1] = c[j][1] + s1[j][1];
    }
    memcpy(S, Sn, D * sizeof(double));
    memcpy(states + (size_t)t * D, S, D * sizeof(double));
  }
  free(S);
  free(Sn);
}

/* Forward: path (B, L, m), clock (B, L), dw (m/2, 2) -> out (B, L-1, 1 + m + m^2), prefix rows with level 0. */
void cpu_planes_forward(int B, int L, int m, int flow_mode, const REAL* path, const REAL* clock, const REAL* dwr,
                        REAL* out) {
  const int D = m + m * m, W = D + 1, K = m / 2;
  double dw[64];
  for (int i = 0; i < 2 * K; ++i) dw[i] = dwr[i];
#pragma omp parallel for schedule(dynamic, 1)
  for (int b = 0; b < B; ++b) {
    double* st = malloc((size_t)(L - 1) * D * sizeof(double));
    planes_forward_one(L, m, path + (size_t)b * L * m, clock + (size_t)b * L, dw, flow_mode, st);
    for (int t = 0; t < L - 1; ++t) {
      REAL* row = out + ((size_t)b * (L - 1) + t) * W;
      row[0] = 1;
      for (int i = 0; i < D; ++i) row[1 + i] = (REAL)st[(size_t)t * D + i];
    }
    free(st);
  }
}

/* Backward of the prefix readout: gout (B, L-1, W) -> dpath (B, L, m), dclock (B, L), ddw (m/2, 2). */
void cpu_planes_backward(int B, int L, int m, int flow_mode, const REAL* path, const REAL* clock, const REAL* dwr,
                         const REAL* gout, REAL* dpath, REAL* dclock, REAL* ddw_out) {
  const int D = m + m * m, W = D + 1, K = m / 2;
  double dw[64];
  for (int i = 0; i < 2 * K; ++i) dw[i] = dwr[i];
  double* ddw_all = calloc((size_t)B * 2 * K, sizeof(double));
  gl_init();
#pragma omp parallel for schedule(dynamic, 1)
  for (int b = 0; b < B; ++b) {
    const REAL* X = path + (size_t)b * L * m;
    const REAL* th = clock + (size_t)b * L;
    double* st = malloc((size_t)(L - 1) * D * sizeof(double));
    planes_forward_one(L, m, X, th, dw, flow_mode, st);
    double* lam = calloc(D, sizeof(double));
    double* lamn = calloc(D, sizeof(double));
    double* dv = calloc((size_t)(L - 1) * m, sizeof(double));
    double* dh = calloc((size_t)(L - 1), sizeof(double));
    double dhf_shared = 0.0;
    double* ddw = ddw_all + (size_t)b * 2 * K;
    for (int t = L - 2; t >= 0; --t) {
      const REAL* g = gout + ((size_t)b * (L - 1) + t) * W + 1;
      for (int i = 0; i < D; ++i) lam[i] += (double)g[i];
      const double* Sp = t > 0 ? st + (size_t)(t - 1) * D : NULL; /* state before interval t */
      const double h = (double)th[t + 1] - (double)th[t];
      const double hf = flow_h(th, t, L, flow_mode);
      double R[32][4], s1[32][2], c[32][2], S1p[32][2];
      cplx p[32], rho[32], ph[32];
      for (int j = 0; j < K; ++j) {
        p[j] = ((double)X[(t + 1) * m + 2 * j] - (double)X[t * m + 2 * j]) +
               I * ((double)X[(t + 1) * m + 2 * j + 1] - (double)X[t * m + 2 * j + 1]);
        rho[j] = c_rho(hf, dw[2 * j], dw[2 * j + 1]);
        ph[j] = c_phi(h, dw[2 * j], dw[2 * j + 1]);
        rotm(rho[j], R[j]);
        const cplx s = ph[j] * p[j];
        s1[j][0] = creal(s);
        s1[j][1] = cimag(s);
        S1p[j][0] = Sp ? Sp[2 * j] : 0.0;
        S1p[j][1] = Sp ? Sp[2 * j + 1] : 0.0;
        c[j][0] = R[j][0] * S1p[j][0] + R[j][1] * S1p[j][1];
        c[j][1] = R[j][2] * S1p[j][0] + R[j][3] * S1p[j][1];
      }
      double gc[32][2], gs1[32][2], gR[32][4];
      cplx gp[32];
      for (int j = 0; j < K; ++j) {
        gc[j][0] = lam[2 * j];
        gc[j][1] = lam[2 * j + 1];
        gs1[j][0] = lam[2 * j];
        gs1[j][1] = lam[2 * j + 1];
        gp[j] = 0;
        for (int e = 0; e < 4; ++e) gR[j][e] = 0;
      }
      for (int j = 0; j < K; ++j)
        for (int k = 0; k < K; ++k) {
          double Lb[4], P[4];
          for (int a = 0; a < 2; ++a)
            for (int bb = 0; bb < 2; ++bb) {
              Lb[2 * a + bb] = lam[m + IDX2(j, k, a, bb)];
              P[2 * a + bb] = Sp ? Sp[m + IDX2(j, k, a, bb)] : 0.0;
            }
          /* cross term c_j s1_k^T */
          for (int a = 0; a < 2; ++a)
            for (int bb = 0; bb < 2; ++bb) {
              gc[j][a] += Lb[2 * a + bb] * s1[k][bb];
              gs1[k][bb] += Lb[2 * a + bb] * c[j][a];
            }
          /* flow R_j P R_k^T: cotangent of P is R_j^T Lb R_k; of R_j: Lb R_k P^T; of R_k: Lb^T R_j P */
          double RkPt[4], RjP[4];
          for (int a = 0; a < 2; ++a)
            for (int bb = 0; bb < 2; ++bb) {
              RkPt[2 * a + bb] = R[k][2 * a] * P[2 * bb] + R[k][2 * a + 1] * P[2 * bb + 1]; /* (R_k P^T)[a][bb] */
              RjP[2 * a + bb] = R[j][2 * a] * P[bb] + R[j][2 * a + 1] * P[2 + bb];
            }
          for (int a = 0; a < 2; ++a)
            for (int bb = 0; bb < 2; ++bb) {
              gR[j][2 * a + bb] += Lb[2 * a] * RkPt[bb] + Lb[2 * a + 1] * RkPt[2 + bb];
              gR[k][2 * a + bb] += Lb[a] * RjP[bb] + Lb[2 + a] * RjP[2 + bb];
            }
          double Ln[4];
          for (int a = 0; a < 2; ++a)
            for (int bb = 0; bb < 2; ++bb) {
              /* (R_j^T Lb R_k)[a][bb] */
              double acc = 0;
              for (int x = 0; x < 2; ++x)
                for (int y = 0; y < 2; ++y) acc += R[j][2 * x + a] * Lb[2 * x + y] * R[k][2 * y + bb];
              Ln[2 * a + bb] = acc;
            }
          for (int e = 0; e < 4; ++e) lamn[m + IDX2(j, k, e / 2, e % 2)] = Ln[e];
          /* local block from A = IA p_j conj(p_k), B = IB p_j p_k */
          const cplx gA = 0.5 * ((Lb[0] + Lb[3]) + I * (Lb[2] - Lb[1]));
          const cplx gB = 0.5 * ((Lb[0] - Lb[3]) + I * (Lb[1] + Lb[2]));
          const double dj = dw[2 * j], wj = dw[2 * j + 1], dk = dw[2 * k], wk = dw[2 * k + 1];
          const cplx IA = c_IA(h, dj, wj, dk, wk), IB = c_IB(h, dj, wj, dk, wk);
          const cplx e1 = p[j] * conj(p[k]), f1 = p[j] * p[k];
          const cplx ge = conj(IA) * gA, gf = conj(IB) * gB;
          gp[j] += p[k] * ge + conj(p[k]) * gf;
          gp[k] += conj(ge) * p[j] + conj(p[j]) * gf;
          const cplx gIA = conj(e1) * gA, gIB = conj(f1) * gB;
          /* coefficient derivatives: d/dh, d/dd_j, d/dw_j, d/dd_k, d/dw_k through the nodes */
          const cplx xj = -h * zc(dj, wj), dlB = -h * zc(dk, wk), dlA = -h * (dk + I * wk);
          cplx DxA, DdA, DxB, DdB;
          divdiff_derivs(xj, dlA, &DxA, &DdA);
          divdiff_derivs(xj, dlB, &DxB, &DdB);
          cplx dA[5], dB[5];
          dA[0] = DxA * (-zc(dj, wj)) + DdA * (-(dk + I * wk));
          dB[0] = DxB * (-zc(dj, wj)) + DdB * (-zc(dk, wk));
          dA[1] = -h * DxA;
          dB[1] = -h * DxB;
          dA[2] = I * h * DxA;
          dB[2] = I * h * DxB;
          dA[3] = -h * DdA;
          dB[3] = -h * DdB;
          dA[4] = -I * h * DdA;
          dB[4] = I * h * DdB;
          dh[t] += creal(conj(gIA) * dA[0] + conj(gIB) * dB[0]);
          ddw[2 * j] += creal(conj(gIA) * dA[1] + conj(gIB) * dB[1]);
          ddw[2 * j + 1] += creal(conj(gIA) * dA[2] + conj(gIB) * dB[2]);
          ddw[2 * k] += creal(conj(gIA) * dA[3] + conj(gIB) * dB[3]);
          ddw[2 * k + 1] += creal(conj(gIA) * dA[4] + conj(gIB) * dB[4]);
        }
      for (int j = 0; j < K; ++j) {
        /* c_j = R_j S1p_j: cotangents of R_j and S1p_j */
        for (int a = 0; a < 2; ++a)
          for (int bb = 0; bb < 2; ++bb) gR[j][2 * a + bb] += gc[j][a] * S1p[j][bb];
        lamn[2 * j] = R[j][0] * gc[j][0] + R[j][2] * gc[j][1];
        lamn[2 * j + 1] = R[j][1] * gc[j][0] + R[j][3] * gc[j][1];
        /* s1_j = phi_j p_j */
        const cplx gs = gs1[j][0] + I * gs1[j][1];
        gp[j] += conj(ph[j]) * gs;
        const cplx gph = conj(p[j]) * gs;
        /* R from rho = a + ib: R = [[a, -b], [b, a]] */
        const cplx grho = (gR[j][0] + gR[j][3]) + I * (gR[j][2] - gR[j][1]);
        const double dj = dw[2 * j], wj = dw[2 * j + 1];
        const cplx xj = -h * zc(dj, wj), xf = -hf * zc(dj, wj);
        const cplx dphx = dphi(xj), erx = cexp(xf);
        const cplx dph_h = dphx * (-zc(dj, wj)), dph_d = -h * dphx, dph_w = I * h * dphx;
        const cplx dr_h = erx * (-zc(dj, wj)), dr_d = -hf * erx, dr_w = I * hf * erx;
        dh[t] += creal(conj(gph) * dph_h);
        if (flow_mode == 0) dh[t] += creal(conj(grho) * dr_h);
        else dhf_shared += creal(conj(grho) * dr_h);
        ddw[2 * j] += creal(conj(gph) * dph_d + conj(grho) * dr_d);
        ddw[2 * j + 1] += creal(conj(gph) * dph_w + conj(grho) * dr_w);
        dv[(size_t)t * m + 2 * j] = creal(gp[j]);
        dv[(size_t)t * m + 2 * j + 1] = cimag(gp[j]);
      }
      memcpy(lam, lamn, D * sizeof(double));
    }
    for (int t = 0; t < L; ++t) {
      for (int ch = 0; ch < m; ++ch) {
        double gsum = 0;
        if (t >= 1) gsum += dv[(size_t)(t - 1) * m + ch];
        if (t < L - 1) gsum -= dv[(size_t)t * m + ch];
        dpath[((size_t)b * L + t) * m + ch] = (REAL)gsum;
      }
      double gsum = 0;
      if (t >= 1) gsum += dh[t - 1];
      if (t < L - 1) gsum -= dh[t];
      if (flow_mode != 0) {
        const int r = flow_mode == 1 ? 0 : 1;
        if (t == r + 1) gsum += dhf_shared;
        if (t == r) gsum -= dhf_shared;
      }
      dclock[(size_t)b * L + t] = (REAL)gsum;
    }
    free(st);
    free(lam);
    free(lamn);
    free(dv);
    free(dh);
  }
  for (int i = 0; i < 2 * K; ++i) {
    double s = 0;
    for (int b = 0; b < B; ++b) s += ddw_all[(size_t)b * 2 * K + i];
    ddw_out[i] = (REAL)s;
  }
  free(ddw_all);
}
