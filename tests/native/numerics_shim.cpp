// Host build of the kernels' scalar numerics (csrc/ews_numerics.h) for CPU tests: plain arrays in, arrays out.
#include "ews_numerics.h"

using ews::cf;

extern "C" {
void shim_node1_c(int n, const float* x, float* out) {  // out: n x 6 (e, p, dp as re/im)
  for (int i = 0; i < n; ++i) {
    ews::Node1<cf> r = ews::node1(cf{x[2 * i], x[2 * i + 1]});
    float v[6] = {r.e.re, r.e.im, r.p.re, r.p.im, r.dp.re, r.dp.im};
    for (int j = 0; j < 6; ++j) out[6 * i + j] = v[j];
  }
}
void shim_dd3_c(int n, const float* x, const float* y, float* out) {  // out: n x 6 (d, dx, dy)
  for (int i = 0; i < n; ++i) {
    ews::DD3<cf> r = ews::dd3<cf, true>(cf{x[2 * i], x[2 * i + 1]}, cf{y[2 * i], y[2 * i + 1]});
    float v[6] = {r.d.re, r.d.im, r.dx.re, r.dx.im, r.dy.re, r.dy.im};
    for (int j = 0; j < 6; ++j) out[6 * i + j] = v[j];
  }
}
void shim_dd3_r(int n, const float* x, const float* y, float* out) {  // out: n x 3
  for (int i = 0; i < n; ++i) {
    ews::DD3<float> r = ews::dd3<float, true>(x[i], y[i]);
    out[3 * i] = r.d;
    out[3 * i + 1] = r.dx;
    out[3 * i + 2] = r.dy;
  }
}
void shim_node1q_c(int n, int q, const float* x, float* out) {  // order-q truncation; out: n x 6
  for (int i = 0; i < n; ++i) {
    ews::Node1<cf> r = ews::node1q(cf{x[2 * i], x[2 * i + 1]}, q);
    float v[6] = {r.e.re, r.e.im, r.p.re, r.p.im, r.dp.re, r.dp.im};
    for (int j = 0; j < 6; ++j) out[6 * i + j] = v[j];
  }
}
void shim_dd3q_c(int n, int q, const float* x, const float* y, float* out) {  // order-q truncation; out: n x 6
  for (int i = 0; i < n; ++i) {
    ews::DD3<cf> r = ews::dd3q<cf, true>(cf{x[2 * i], x[2 * i + 1]}, cf{y[2 * i], y[2 * i + 1]}, q);
    float v[6] = {r.d.re, r.d.im, r.dx.re, r.dx.im, r.dy.re, r.dy.im};
    for (int j = 0; j < 6; ++j) out[6 * i + j] = v[j];
  }
}
}
