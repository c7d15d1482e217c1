// Scalar numerics of the EWS local terms for diagonal and rotation-plane generators, shared by the HIP kernels
// and by a host build used in CPU tests.
//
// For a clock step h and generator eigenvalue mu (real diagonal: mu = lambda_i; rotation plane
// A_j = [[d, w], [-w, d]] acting as multiplication by conj(z_j), z_j = d + i w), every coefficient of the
// interval's local term is a divided difference of exp at nodes proportional to h
// (Hermite-Genocchi: exp[a_0..a_n] = integral over the n-simplex of exp(sum t_i a_i)):
//   flow        rho   = e^x                 x = -h mu
//   level 1     phi   = exp[0, x]           = (e^x - 1) / x
//   level 2     D     = exp[0, x, y]        y = x + x' (the later factor's node)
// The reference writes D(x, delta) = (phi(x + delta) - phi(x)) / delta (ews/core/kernels/plane_engine.py:65-78);
// the two are equal. Node derivatives are divided differences with a repeated node:
//   d phi / dx = exp[0, x, x],  dD/dx|_y = exp[0, x, x, y],  dD/dy|_x = exp[0, x, y, y].
// Evaluation: joint Taylor series when every node lies in the unit disk; otherwise the recursive
// divided-difference formula divided by the node of largest modulus, whose two-node pieces are computed
// around the nearer node (e^t phi(s) = exp[t, t + s]) so no quotient cancels catastrophically.
#pragma once

#include <math.h>
#include <stdint.h>

#if defined(__HIPCC__)
#define EWS_HD __host__ __device__ __forceinline__
#else
#define EWS_HD inline
#endif

namespace ews {

struct cf {
  float re, im;
};

EWS_HD cf mk(float r, float i) { return cf{r, i}; }
EWS_HD cf operator+(cf a, cf b) { return cf{a.re + b.re, a.im + b.im}; }
EWS_HD cf operator-(cf a, cf b) { return cf{a.re - b.re, a.im - b.im}; }
EWS_HD cf operator-(cf a) { return cf{-a.re, -a.im}; }
EWS_HD cf operator*(cf a, cf b) { return cf{a.re * b.re - a.im * b.im, a.re * b.im + a.im * b.re}; }
EWS_HD cf operator*(float s, cf a) { return cf{s * a.re, s * a.im}; }
EWS_HD cf operator*(cf a, float s) { return cf{s * a.re, s * a.im}; }
EWS_HD cf operator+(cf a, float s) { return cf{a.re + s, a.im}; }
EWS_HD cf operator-(cf a, float s) { return cf{a.re - s, a.im}; }
EWS_HD cf& operator+=(cf& a, cf b) { a.re += b.re; a.im += b.im; return a; }
EWS_HD cf& operator-=(cf& a, cf b) { a.re -= b.re; a.im -= b.im; return a; }
EWS_HD cf conj(cf a) { return cf{a.re, -a.im}; }
EWS_HD float conj(float a) { return a; }
EWS_HD float absv(float a) { return fabsf(a); }
EWS_HD float absv(cf a) { return sqrtf(a.re * a.re + a.im * a.im); }
EWS_HD float re(float a) { return a; }
EWS_HD float re(cf a) { return a.re; }
EWS_HD float im(float) { return 0.0f; }
EWS_HD float im(cf a) { return a.im; }
EWS_HD cf operator/(cf a, cf b) {
  // Smith's algorithm: no overflow for |b| large
  if (fabsf(b.re) >= fabsf(b.im)) {
    float r = b.im / b.re, den = b.re + b.im * r;
    return cf{(a.re + a.im * r) / den, (a.im - a.re * r) / den};
  }
  float r = b.re / b.im, den = b.im + b.re * r;
  return cf{(a.re * r + a.im) / den, (a.im * r - a.re) / den};
}
EWS_HD float expv(float x) { return expf(x); }
EWS_HD cf expv(cf x) {
  float m = expf(x.re);
  return cf{m * cosf(x.im), m * sinf(x.im)};
}
template <class T> EWS_HD T one();
template <> EWS_HD float one<float>() { return 1.0f; }
template <> EWS_HD cf one<cf>() { return cf{1.0f, 0.0f}; }
template <class T> EWS_HD T zero();
template <> EWS_HD float zero<float>() { return 0.0f; }
template <> EWS_HD cf zero<cf>() { return cf{0.0f, 0.0f}; }

// 1 / n! for n = 0..20
#define EWS_INVFACT                                                                                    \
  {1.0f, 1.0f, 0.5f, 1.6666667e-1f, 4.1666668e-2f, 8.3333338e-3f, 1.3888889e-3f, 1.9841270e-4f,         \
   2.4801587e-5f, 2.7557319e-6f, 2.7557319e-7f, 2.5052108e-8f, 2.0876757e-9f, 1.6059044e-10f,           \
   1.1470746e-11f, 7.6471637e-13f, 4.7794773e-14f, 2.8114573e-15f, 1.5619207e-16f, 8.2206352e-18f,      \
   4.1103176e-19f}

EWS_HD float invfact(int n) {
  const float t[21] = EWS_INVFACT;
  return t[n];
}

// phi(s) = exp[0, s] = sum_n s^n / (n+1)!
template <class T> EWS_HD T phi1(T s) {
  if (absv(s) < 0.5f) {
    T acc = invfact(12) * one<T>();
    for (int n = 10; n >= 0; --n) acc = acc * s + invfact(n + 1) * one<T>();
    return acc;
  }
  return (expv(s) - 1.0f) / s;
}

// exp[0, s, s] = phi'(s) = sum_n (n+1) s^n / (n+2)!
template <class T> EWS_HD T dphi1(T s) {
  if (absv(s) < 1.0f) {
    T acc = (14.0f * invfact(15)) * one<T>();
    for (int n = 12; n >= 0; --n) acc = acc * s + ((float)(n + 1) * invfact(n + 2)) * one<T>();
    return acc;
  }
  return (expv(s) * (s - 1.0f) + 1.0f) / (s * s);
}

// exp[0, 0, s] = (e^s - 1 - s) / s^2 = sum_n s^n / (n+2)!
template <class T> EWS_HD T phi2(T s) {
  if (absv(s) < 1.0f) {
    T acc = invfact(15) * one<T>();
    for (int n = 12; n >= 0; --n) acc = acc * s + invfact(n + 2) * one<T>();
    return acc;
  }
  return (expv(s) - 1.0f - s) / (s * s);
}

template <class T> struct Node1 {
  T e;   // e^x
  T p;   // exp[0, x]
  T dp;  // exp[0, x, x]
};

template <class T> EWS_HD Node1<T> node1(T x) {
  Node1<T> o;
  o.e = expv(x);
  if (absv(x) < 0.5f) {
    T acc = invfact(12) * one<T>();
    for (int n = 10; n >= 0; --n) acc = acc * x + invfact(n + 1) * one<T>();
    o.p = acc;
  } else {
    o.p = (o.e - 1.0f) / x;
  }
  if (absv(x) < 1.0f) {
    T acc = (14.0f * invfact(15)) * one<T>();
    for (int n = 12; n >= 0; --n) acc = acc * x + ((float)(n + 1) * invfact(n + 2)) * one<T>();
    o.dp = acc;
  } else {
    o.dp = (o.e * (x - 1.0f) + 1.0f) / (x * x);
  }
  return o;
}

template <class T> struct DD3 {
  T d;   // exp[0, x, y]
  T dx;  // exp[0, x, x, y]
  T dy;  // exp[0, x, y, y]
};

// Divided differences of exp at {0, x, y} and their node derivatives.
template <class T, bool DERIV> EWS_HD DD3<T> dd3(T x, T y) {
  DD3<T> o;
  const float ax = absv(x), ay = absv(y);
  if (ax <= 1.0f && ay <= 1.0f) {
    // exp[nodes] = sum_m h_m(nodes) / (m + #nodes - 1)!, h_m the complete homogeneous polynomials
    T a = one<T>(), bpow = one<T>();
    T h2 = one<T>(), h3x = one<T>(), h3y = one<T>();
    T s2 = invfact(2) * one<T>();
    T s3x = invfact(3) * one<T>();
    T s3y = invfact(3) * one<T>();
    for (int m = 1; m <= 13; ++m) {
      a = a * x;
      h2 = h2 * y + a;
      s2 += invfact(m + 2) * h2;
      if (DERIV) {
        bpow = bpow * y;
        h3x = h3x * y + (float)(m + 1) * a;
        h3y = h3y * x + (float)(m + 1) * bpow;
        s3x += invfact(m + 3) * h3x;
        s3y += invfact(m + 3) * h3y;
      }
    }
    o.d = s2;
    o.dx = s3x;
    o.dy = s3y;
    return o;
  }
  if (ay >= ax) {
    // orderings (0,x,y), (0,x,x,y), (0,x,y,y): divide by y; pieces around x with s = y - x
    T s = y - x;
    T ex = expv(x);
    Node1<T> nx = node1(x);
    o.d = (ex * phi1(s) - nx.p) / y;
    if (DERIV) {
      o.dx = (ex * phi2(s) - nx.dp) / y;
      o.dy = (ex * dphi1(s) - o.d) / y;
    }
  } else {
    // orderings (0,y,x), (0,y,x,x), (0,y,y,x): divide by x; pieces around y with s = x - y
    T s = x - y;
    T ey = expv(y);
    Node1<T> ny = node1(y);
    o.d = (ey * phi1(s) - ny.p) / x;
    if (DERIV) {
      o.dx = (ey * dphi1(s) - o.d) / x;
      o.dy = (ey * phi2(s) - ny.dp) / x;
    }
  }
  return o;
}

// Order-q truncations: the series leaf (ews/core/series_leaf.py:8-25) on a diagonal or plane generator. Its
// letters are b_p = x^p / p! times the increment, so each level-k coefficient is the degree-<= q Taylor
// polynomial of the exact divided difference in the nodes:
//   phi_q(x)   = sum_{n <= q} x^n / (n+1)!
//   D_q(x, y)  = sum_{m <= q} h_m(x, y) / (m+2)!        (h_m homogeneous of degree m in (x, x' = y - x))
// Node derivatives are the derivatives of these polynomials (degree q - 1): dphi_q = sum_{n < q} (n+1) x^n/(n+2)!,
// dD_q/dx = sum_{m < q} h_m(x, x, y)/(m+3)!, dD_q/dy = sum_{m < q} h_m(x, y, y)/(m+3)!. Each sum is accumulated
// in increasing degree with the factorials folded into the running terms (no 1/n! table, no underflow at q = 40).
// q <= 0 selects the exact functions above.
template <class T> EWS_HD Node1<T> node1q(T x, int q) {
  if (q <= 0) return node1(x);
  Node1<T> o;
  o.e = expv(x);
  T t = one<T>();         // x^n / (n+1)!
  T u = 0.5f * one<T>();  // x^n / (n+2)!
  T p = t;
  T dp = zero<T>();
  if (q >= 1) dp = u;
  for (int n = 1; n <= q; ++n) {
    t = t * x * (1.0f / (float)(n + 1));
    p += t;
    if (n < q) {
      u = u * x * (1.0f / (float)(n + 2));
      dp += (float)(n + 1) * u;
    }
  }
  o.p = p;
  o.dp = dp;
  return o;
}

template <class T, bool DERIV> EWS_HD DD3<T> dd3q(T x, T y, int q) {
  if (q <= 0) return dd3<T, DERIV>(x, y);
  DD3<T> o;
  T a = 0.5f * one<T>();  // x^m / (m+2)!
  T g = a;                // h_m(x, y) / (m+2)!
  T dsum = g;
  const float s6 = 1.0f / 6.0f;
  T bx = s6 * one<T>(), by = s6 * one<T>();  // x^m / (m+3)!, y^m / (m+3)!
  T gx = bx, gy = by;                        // h_m(x, x, y) / (m+3)!, h_m(x, y, y) / (m+3)!
  T sx = zero<T>(), sy = zero<T>();
  if (DERIV && q >= 1) {
    sx = gx;
    sy = gy;
  }
  for (int m = 1; m <= q; ++m) {
    const float r = 1.0f / (float)(m + 2);
    a = a * x * r;
    g = y * g * r + a;
    dsum += g;
    if (DERIV && m < q) {
      const float r3 = 1.0f / (float)(m + 3);
      bx = bx * x * r3;
      by = by * y * r3;
      gx = y * gx * r3 + (float)(m + 1) * bx;
      gy = x * gy * r3 + (float)(m + 1) * by;
      sx += gx;
      sy += gy;
    }
  }
  o.d = dsum;
  o.dx = sx;
  o.dy = sy;
  return o;
}

}  // namespace ews
