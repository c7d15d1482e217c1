// EWS Chen scan for diagonal and rotation-plane generators on MI355X (gfx950): fused local terms + chunked
// modified-Chen recursion, forward and hand-written adjoint.
//
// Math (reference sign: flow exp(-h A)). Rotation plane j acts on p_j = v_{2j} + i v_{2j+1} as multiplication
// by conj(z_j); with x_j = -h conj(z_j) the interval's flow is rho_j = e^{x_j} and its level-1 local term
// phi(x_j) p_j (ews/core/kernels/plane_engine.py:134-152). A level-2 block (j, k) of the real (d, d) tensor is
// carried as two complex numbers SA_jk (the u conj(w) part) and SB_jk (the u w part):
//     SB <- rho_j rho_k SB       + c_j s1_k       + D(x_j, x_j + x_k)       p_j p_k
//     SA <- rho_j conj(rho_k) SA + c_j conj(s1_k) + D(x_j, x_j + conj(x_k)) p_j conj(p_k)
// with c_j = rho_j S1_j (the flowed level 1) and D(x, y) = exp[0, x, y]; this is the Chen step
// S2 <- M S2 M^T + (M S1) s1^T + s2 (ews/core/chen_scan.py:124-152, pallas_combine.py:300-303) diagonalised
// plane by plane. A real diagonal A is the same recursion with real scalars and only the B channel.
//
// Parallel structure: one workgroup per (sample, chunk of T intervals); one lane per level-2 element pair
// (j, k) (lanes with k == 0 also own plane j's level 1). Passes:
//   forward  F1 chunk summaries from a zero carry -> F2 float64 carry scan over chunks per sample ->
//            F3 chunk outputs from the true carry (prefix rows, or mean/max partials) [-> F4 mean/max reduce]
//   backward B1 chunk-local adjoints with zero incoming cotangent -> B2 float64 reverse adjoint scan ->
//            B3 full adjoint per chunk (forward states recomputed from the chunk's carry, 8-step
//            checkpoints) -> B4 knot gradients and parameter reductions.
// Per-step coefficients: when every clock step of a chunk is within 2^-16 / (2 max|mu|) of the chunk mean
// (a uniform clock in float32), coefficients are first-order Taylor models in h around the mean (error
// below float32 rounding); otherwise they are evaluated exactly per step.
#include <hip/hip_runtime.h>

#include <type_traits>

#include "ews_hip.h"
#include "ews_numerics.h"

namespace ews {

// ------------------------------------------------------------------------------------------- float64 complex
struct cd {
  double re, im;
};
__device__ __forceinline__ cd operator+(cd a, cd b) { return cd{a.re + b.re, a.im + b.im}; }
__device__ __forceinline__ cd operator*(cd a, cd b) {
  return cd{a.re * b.re - a.im * b.im, a.re * b.im + a.im * b.re};
}
__device__ __forceinline__ cd conj(cd a) { return cd{a.re, -a.im}; }
__device__ __forceinline__ double conj(double a) { return a; }
__device__ __forceinline__ cd dexp(cd x) {
  double m = exp(x.re);
  return cd{m * cos(x.im), m * sin(x.im)};
}
__device__ __forceinline__ double dexp(double x) { return exp(x); }

template <bool CPLX> struct Types;
template <> struct Types<true> {
  using T = cf;
  using TD = cd;
};
template <> struct Types<false> {
  using T = float;
  using TD = double;
};

__device__ __forceinline__ cd to_d(cf a) { return cd{(double)a.re, (double)a.im}; }
__device__ __forceinline__ double to_d(float a) { return (double)a; }
__device__ __forceinline__ cf to_f(cd a) { return cf{(float)a.re, (float)a.im}; }
__device__ __forceinline__ float to_f(double a) { return (float)a; }

// ------------------------------------------------------------------------------------------- arguments
struct DiagArgs {
  int B, L, n_int, d, K;  // K: planes (complex) or channels (real)
  int N, flow_mode, readout;
  int T, C;               // chunk length, chunk count
  int W, off1, off2, lvl0, D, npar;
  int path_bf16;
  const void* path;
  const float* clock;
  const float* params;
  float* out;
  const float* gout;
  // residual
  double* carries;  // (B, C+1, D)
  int* argmax;      // (B, W)
  // workspace
  float* summ;      // (B, C, D)
  float* mu;        // (B, C, D)
  float* mt;        // (B, C, D)
  float* red;       // (B, C, W)
  int* red_idx;     // (B, C, W)
  float* dv;        // (B, n_int, d)
  float* dh;        // (B, n_int)
  float* gp;        // (B, C, npar)
  float* gph;       // (B, C)
  // backward outputs
  float* dpath;
  float* dclock;
  float* dparams;
};

enum { MODE_SUMMARY = 0, MODE_PREFIX = 1, MODE_REDUCE = 2 };

// plane parameter u_j = -conj(z_j) = (-d_j, w_j) (planes) or -lambda_j (real): nodes are h * u
__device__ __forceinline__ cf load_u(const float* params, int j, cf*) {
  return cf{-params[2 * j], params[2 * j + 1]};
}
__device__ __forceinline__ float load_u(const float* params, int j, float*) { return -params[j]; }

template <class T> __device__ __forceinline__ T lds_p(const float* s_v, int t, int d, int j);
template <> __device__ __forceinline__ cf lds_p<cf>(const float* s_v, int t, int d, int j) {
  const float2 v = *reinterpret_cast<const float2*>(s_v + t * d + 2 * j);
  return cf{v.x, v.y};
}
template <> __device__ __forceinline__ float lds_p<float>(const float* s_v, int t, int d, int j) {
  return s_v[t * d + j];
}

__device__ __forceinline__ float load_path(const DiagArgs& a, size_t idx) {
  if (a.path_bf16) {
    const unsigned short u = reinterpret_cast<const unsigned short*>(a.path)[idx];
    return __uint_as_float(((unsigned)u) << 16);
  }
  return reinterpret_cast<const float*>(a.path)[idx];
}

// Increments v_t = X_{t+1} - X_t and clock steps h_t = theta_{t+1} - theta_t of chunk intervals [t0, t0+Tc).
__device__ __forceinline__ void load_chunk(const DiagArgs& a, int b, int t0, int Tc, float* s_v, float* s_h) {
  const size_t base = ((size_t)b * a.L + t0) * a.d;
  for (int i = threadIdx.x; i < Tc * a.d; i += blockDim.x) {
    s_v[i] = load_path(a, base + i + a.d) - load_path(a, base + i);
  }
  const float* th = a.clock + (size_t)b * a.L + t0;
  for (int i = threadIdx.x; i < Tc; i += blockDim.x) s_h[i] = th[i + 1] - th[i];
}

// ------------------------------------------------------------------------------------------- coefficients
template <class T> struct Coef {
  T rho, phi_j, phi_k, IA, IB, lamA, lamB;
};
template <class T> struct CoefD {
  T rho1, phi_j1, phi_k1, IA1, IB1, lamA1, lamB1;  // d/dh
  T dphi_j, dphi_k, DxA, DyA, DxB, DyB;           // node derivatives
};

template <class T> __device__ __forceinline__ T conj_if(T x, bool) { return x; }
__device__ __forceinline__ cf conjc(cf x) { return conj(x); }
__device__ __forceinline__ float conjc(float x) { return x; }

// Exact coefficients at clock step h (flows at hf: h per interval, the shared step when cached).
template <class T, bool CPLX, int N, bool DERIV>
__device__ __forceinline__ void eval_coef(float h, float hf, bool per_int, T uj, T uk, Coef<T>& c, CoefD<T>& q) {
  const T xj = h * uj;
  const Node1<T> nj = node1(xj);
  c.phi_j = nj.p;
  hf = per_int ? h : hf;  // flows use the interval's own step unless they are cached
  c.rho = per_int ? nj.e : expv(hf * uj);
  if (DERIV) {
    q.dphi_j = nj.dp;
    q.phi_j1 = nj.dp * uj;
    q.rho1 = per_int ? c.rho * uj : zero<T>();
  }
  if (N == 2) {
    const T xk = h * uk;
    const Node1<T> nk = node1(xk);
    c.phi_k = nk.p;
    const T ub = uj + uk;
    const DD3<T> db = dd3<T, DERIV>(xj, h * ub);
    c.IB = db.d;
    c.lamB = expv(hf * ub);
    if (DERIV) {
      q.dphi_k = nk.dp;
      q.phi_k1 = nk.dp * uk;
      q.DxB = db.dx;
      q.DyB = db.dy;
      q.IB1 = db.dx * uj + db.dy * ub;
      q.lamB1 = per_int ? c.lamB * ub : zero<T>();
    }
    if (CPLX) {
      const T ua = uj + conjc(uk);
      const DD3<T> da = dd3<T, DERIV>(xj, h * ua);
      c.IA = da.d;
      c.lamA = expv(hf * ua);
      if (DERIV) {
        q.DxA = da.dx;
        q.DyA = da.dy;
        q.IA1 = da.dx * uj + da.dy * ua;
        q.lamA1 = per_int ? c.lamA * ua : zero<T>();
      }
    }
  }
}

// First-order model c(h_t) = c0 + c1 (h_t - hbar) of every h-dependent coefficient.
template <class T, bool CPLX, int N>
__device__ __forceinline__ void lin_coef(const Coef<T>& c0, const CoefD<T>& q, float dlt, bool per_int, Coef<T>& c) {
  c.phi_j = c0.phi_j + q.phi_j1 * dlt;
  c.rho = per_int ? c0.rho + q.rho1 * dlt : c0.rho;
  if (N == 2) {
    c.phi_k = c0.phi_k + q.phi_k1 * dlt;
    c.IB = c0.IB + q.IB1 * dlt;
    c.lamB = per_int ? c0.lamB + q.lamB1 * dlt : c0.lamB;
    if (CPLX) {
      c.IA = c0.IA + q.IA1 * dlt;
      c.lamA = per_int ? c0.lamA + q.lamA1 * dlt : c0.lamA;
    }
  }
}

// One forward Chen step of the lane's elements.
template <class T, bool CPLX, int N>
__device__ __forceinline__ void fwd_step(const Coef<T>& c, T pj, T pk, T& S1, T& SA, T& SB) {
  const T cj = c.rho * S1;
  if (N == 2) {
    const T s1k = c.phi_k * pk;
    SB = c.lamB * SB + cj * s1k + c.IB * (pj * pk);
    if (CPLX) SA = c.lamA * SA + cj * conjc(s1k) + c.IA * (pj * conjc(pk));
  }
  S1 = cj + c.phi_j * pj;
}

// Chunk setup shared by all chunk kernels: the uniform-clock test and the reference step.
struct ChunkClock {
  float hbar, href;
  bool fast, per_int;
};

template <class T>
__device__ __forceinline__ ChunkClock chunk_clock(const DiagArgs& a, int b, int Tc, const float* s_h) {
  ChunkClock cc;
  float s = 0.0f;
  for (int t = 0; t < Tc; ++t) s += s_h[t];
  cc.hbar = s / (float)Tc;
  float dmax = 0.0f;
  bool finite = true;
  for (int t = 0; t < Tc; ++t) {
    const float dl = fabsf(s_h[t] - cc.hbar);
    dmax = fmaxf(dmax, dl);
    finite = finite && (dl <= 3.0e38f);
  }
  float R = 0.0f;
  T dummy{};
  for (int j = 0; j < a.K; ++j) R = fmaxf(R, absv(load_u(a.params, j, &dummy)));
  cc.fast = finite && (dmax * 2.0f * R < 1.52587890625e-5f);  // 2^-16
  cc.per_int = a.flow_mode == EWS_FLOW_PER_INTERVAL;
  const float* th = a.clock + (size_t)b * a.L;
  if (a.flow_mode == EWS_FLOW_CACHED) {
    cc.href = th[1] - th[0];
  } else if (a.flow_mode == EWS_FLOW_CACHED_BASEPOINT) {
    cc.href = a.L > 2 ? th[2] - th[1] : 0.0f;
  } else {
    cc.href = 0.0f;
  }
  return cc;
}

struct LaneMap {
  int j, k;
  bool active, plane;
};
__device__ __forceinline__ LaneMap lane_map(const DiagArgs& a, int tid) {
  LaneMap m;
  const int P = (a.N == 2) ? a.K * a.K : a.K;
  m.active = tid < P;
  const int t = m.active ? tid : 0;
  m.j = (a.N == 2) ? t / a.K : t;
  m.k = (a.N == 2) ? t % a.K : 0;
  m.plane = m.active && m.k == 0;
  return m;
}

// kernel-layout state offsets: level 1 plane j, level-2 pair (j, k)
template <bool CPLX> __device__ __forceinline__ int st1(int j) { return CPLX ? 2 * j : j; }
template <bool CPLX> __device__ __forceinline__ int st2(const DiagArgs& a, int j, int k) {
  return CPLX ? a.d + 4 * (j * a.K + k) : a.d + j * a.d + k;
}

template <bool CPLX, class T> __device__ __forceinline__ T ldT(const float* p);
template <> __device__ __forceinline__ cf ldT<true, cf>(const float* p) { return cf{p[0], p[1]}; }
template <> __device__ __forceinline__ float ldT<false, float>(const float* p) { return p[0]; }
template <bool CPLX, class T> __device__ __forceinline__ T ldTd(const double* p);
template <> __device__ __forceinline__ cf ldTd<true, cf>(const double* p) { return cf{(float)p[0], (float)p[1]}; }
template <> __device__ __forceinline__ float ldTd<false, float>(const double* p) { return (float)p[0]; }
__device__ __forceinline__ void stT(float* p, cf v) {
  p[0] = v.re;
  p[1] = v.im;
}
__device__ __forceinline__ void stT(float* p, float v) { p[0] = v; }

// Output row element indices of the lane's values (level 1 of plane j; the level-2 block (j, k)).
template <bool CPLX>
__device__ __forceinline__ void out_values(const DiagArgs& a, int j, int k, cf S1, cf SA, cf SB, int* idx,
                                           float* val, int& n1, int& n2);

// ------------------------------------------------------------------------------------------- F1 / F3
template <bool CPLX, int N, int MODE, int MAXT>
__global__ __launch_bounds__(MAXT) void k_chunk_fwd(DiagArgs a) {
  using T = typename Types<CPLX>::T;
  extern __shared__ float smem[];
  float* s_v = smem;
  float* s_h = s_v + a.T * a.d;
  const int c = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
  const int t0 = c * a.T;
  const int Tc = min(a.T, a.n_int - t0);
  load_chunk(a, b, t0, Tc, s_v, s_h);
  __syncthreads();
  const LaneMap m = lane_map(a, tid);
  if (!m.active) return;
  const ChunkClock cc = chunk_clock<T>(a, b, Tc, s_h);
  T dummy{};
  const T uj = load_u(a.params, m.j, &dummy);
  const T uk = load_u(a.params, m.k, &dummy);

  T S1 = zero<T>(), SA = zero<T>(), SB = zero<T>();
  if (MODE != MODE_SUMMARY) {
    const double* cr = a.carries + ((size_t)b * (a.C + 1) + c) * a.D;
    S1 = ldTd<CPLX, T>(cr + st1<CPLX>(m.j));
    if (N == 2) {
      const double* p2 = cr + st2<CPLX>(a, m.j, m.k);
      if (CPLX) {
        SA = ldTd<CPLX, T>(p2);
        SB = ldTd<CPLX, T>(p2 + 2);
      } else {
        SB = ldTd<CPLX, T>(p2);
      }
    }
  }
  Coef<T> c0;
  CoefD<T> q;
  if (cc.fast) eval_coef<T, CPLX, N, true>(cc.hbar, cc.href, cc.per_int, uj, uk, c0, q);

  // reduce-mode accumulators: [level-1 re, im][level-2 q00, q01, q10, q11]
  float acc[6];
  int arg[6];
  const bool is_max = a.readout == EWS_READOUT_MAX;
#pragma unroll
  for (int i = 0; i < 6; ++i) {
    acc[i] = is_max ? -INFINITY : 0.0f;
    arg[i] = 0;
  }

  for (int t = 0; t < Tc; ++t) {
    const float h = s_h[t];
    Coef<T> co;
    if (cc.fast) {
      lin_coef<T, CPLX, N>(c0, q, h - cc.hbar, cc.per_int, co);
    } else {
      CoefD<T> qq;
      eval_coef<T, CPLX, N, false>(h, cc.href, cc.per_int, uj, uk, co, qq);
    }
    const T pj = lds_p<T>(s_v, t, a.d, m.j);
    const T pk = (N == 2) ? lds_p<T>(s_v, t, a.d, m.k) : zero<T>();
    fwd_step<T, CPLX, N>(co, pj, pk, S1, SA, SB);
    if (MODE == MODE_SUMMARY) continue;
    // the lane's output values in the row layout
    float v[6];
    int n1 = 0;
    if (m.plane) {
      v[0] = re(S1);
      v[1] = im(S1);
      n1 = CPLX ? 2 : 1;
    }
    if (N == 2) {
      if constexpr (CPLX) {
        const cf sa = SA, sb = SB;
        v[2] = 0.5f * (sa.re + sb.re);
        v[3] = 0.5f * (sb.im - sa.im);
        v[4] = 0.5f * (sa.im + sb.im);
        v[5] = 0.5f * (sa.re - sb.re);
      } else {
        v[2] = re(SB);
      }
    }
    if (MODE == MODE_PREFIX) {
      float* row = a.out + ((size_t)b * a.n_int + t0 + t) * a.W;
      if (a.lvl0 && tid == 0) row[0] = 1.0f;
      if (m.plane) {
        row[a.off1 + st1<CPLX>(m.j)] = v[0];
        if (CPLX) row[a.off1 + st1<CPLX>(m.j) + 1] = v[1];
      }
      if (N == 2) {
        if (CPLX) {
          float* r0 = row + a.off2 + (2 * m.j) * a.d + 2 * m.k;
          r0[0] = v[2];
          r0[1] = v[3];
          r0[a.d] = v[4];
          r0[a.d + 1] = v[5];
        } else {
          row[a.off2 + m.j * a.d + m.k] = v[2];
        }
      }
    } else {  // MODE_REDUCE
      const int tg = t0 + t;
#pragma unroll
      for (int i = 0; i < 6; ++i) {
        const bool use = (i < 2) ? (i < n1) : (N == 2 && (CPLX || i == 2));
        if (!use) continue;
        if (is_max) {
          if (v[i] > acc[i]) {
            acc[i] = v[i];
            arg[i] = tg;
          }
        } else {
          acc[i] += v[i];
        }
      }
    }
  }

  if (MODE == MODE_SUMMARY) {
    float* sp = a.summ + ((size_t)b * a.C + c) * a.D;
    if (m.plane) stT(sp + st1<CPLX>(m.j), S1);
    if (N == 2) {
      float* p2 = sp + st2<CPLX>(a, m.j, m.k);
      if (CPLX) {
        stT(p2, SA);
        stT(p2 + 2, SB);
      } else {
        stT(p2, SB);
      }
    }
  } else if (MODE == MODE_REDUCE) {
    float* rp = a.red + ((size_t)b * a.C + c) * a.W;
    int* ip = a.red_idx + ((size_t)b * a.C + c) * a.W;
    if (m.plane) {
      const int e = a.off1 + st1<CPLX>(m.j);
      rp[e] = acc[0];
      ip[e] = arg[0];
      if (CPLX) {
        rp[e + 1] = acc[1];
        ip[e + 1] = arg[1];
      }
    }
    if (N == 2) {
      if (CPLX) {
        const int e0 = a.off2 + (2 * m.j) * a.d + 2 * m.k;
        const int es[4] = {e0, e0 + 1, e0 + a.d, e0 + a.d + 1};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          rp[es[i]] = acc[2 + i];
          ip[es[i]] = arg[2 + i];
        }
      } else {
        const int e = a.off2 + m.j * a.d + m.k;
        rp[e] = acc[2];
        ip[e] = arg[2];
      }
    }
  }
}

// ------------------------------------------------------------------------------------------- F2
// Exact chunk flow (float64): per-interval flows multiply to exp(u (theta_end - theta_start)).
__device__ __forceinline__ double chunk_tau(const DiagArgs& a, int b, int c, int Tc) {
  const float* th = a.clock + (size_t)b * a.L;
  const int t0 = c * a.T;
  if (a.flow_mode == EWS_FLOW_PER_INTERVAL) return (double)th[t0 + Tc] - (double)th[t0];
  if (a.flow_mode == EWS_FLOW_CACHED) return ((double)th[1] - (double)th[0]) * Tc;
  const double h1 = a.L > 2 ? (double)th[2] - (double)th[1] : 0.0;
  return h1 * (Tc - (t0 == 0 ? 1 : 0));
}

__device__ __forceinline__ cd load_ud(const float* params, int j, cd*) {
  return cd{-(double)params[2 * j], (double)params[2 * j + 1]};
}
__device__ __forceinline__ double load_ud(const float* params, int j, double*) { return -(double)params[j]; }
__device__ __forceinline__ cd mul_s(cd a, double s) { return cd{a.re * s, a.im * s}; }
__device__ __forceinline__ double mul_s(double a, double s) { return a * s; }
__device__ __forceinline__ cd ldD(const float* p, cd*) { return cd{(double)p[0], (double)p[1]}; }
__device__ __forceinline__ double ldD(const float* p, double*) { return (double)p[0]; }
__device__ __forceinline__ cd ldDD(const double* p, cd*) { return cd{p[0], p[1]}; }
__device__ __forceinline__ double ldDD(const double* p, double*) { return p[0]; }
__device__ __forceinline__ void stD(double* p, cd v) {
  p[0] = v.re;
  p[1] = v.im;
}
__device__ __forceinline__ void stD(double* p, double v) { p[0] = v; }
__device__ __forceinline__ double dre(cd a) { return a.re; }
__device__ __forceinline__ double dre(double a) { return a; }
__device__ __forceinline__ double dim_(cd a) { return a.im; }
__device__ __forceinline__ double dim_(double) { return 0.0; }
__device__ __forceinline__ cd operator-(cd a, cd b) { return cd{a.re - b.re, a.im - b.im}; }

// Write one row of the readout layout from a float64 kernel-layout state (terminal readout).
template <bool CPLX, int N>
__device__ __forceinline__ void write_row_d(const DiagArgs& a, const LaneMap& m, float* row,
                                            typename Types<CPLX>::TD S1, typename Types<CPLX>::TD SA,
                                            typename Types<CPLX>::TD SB, int tid) {
  if (a.lvl0 && tid == 0) row[0] = 1.0f;
  if (m.plane) {
    row[a.off1 + st1<CPLX>(m.j)] = (float)dre(S1);
    if (CPLX) row[a.off1 + st1<CPLX>(m.j) + 1] = (float)dim_(S1);
  }
  if (N == 2) {
    if (CPLX) {
      float* r0 = row + a.off2 + (2 * m.j) * a.d + 2 * m.k;
      r0[0] = (float)(0.5 * (dre(SA) + dre(SB)));
      r0[1] = (float)(0.5 * (dim_(SB) - dim_(SA)));
      r0[a.d] = (float)(0.5 * (dim_(SA) + dim_(SB)));
      r0[a.d + 1] = (float)(0.5 * (dre(SA) - dre(SB)));
    } else {
      row[a.off2 + m.j * a.d + m.k] = (float)dre(SB);
    }
  }
}

template <bool CPLX, int N, int MAXT>
__global__ __launch_bounds__(MAXT) void k_carry_scan(DiagArgs a) {
  using TD = typename Types<CPLX>::TD;
  const int b = blockIdx.x, tid = threadIdx.x;
  const LaneMap m = lane_map(a, tid);
  if (!m.active) return;
  TD dummy{};
  const TD uj = load_ud(a.params, m.j, &dummy);
  const TD uk = load_ud(a.params, m.k, &dummy);
  TD S1{}, SA{}, SB{};
  for (int c = 0; c < a.C; ++c) {
    double* cr = a.carries + ((size_t)b * (a.C + 1) + c) * a.D;
    if (m.plane) stD(cr + st1<CPLX>(m.j), S1);
    if (N == 2) {
      double* p2 = cr + st2<CPLX>(a, m.j, m.k);
      if (CPLX) {
        stD(p2, SA);
        stD(p2 + 2, SB);
      } else {
        stD(p2, SB);
      }
    }
    const int Tc = min(a.T, a.n_int - c * a.T);
    const double tau = chunk_tau(a, b, c, Tc);
    const float* sp = a.summ + ((size_t)b * a.C + c) * a.D;
    const TD Fj = dexp(mul_s(uj, tau));
    const TD l1j = ldD(sp + st1<CPLX>(m.j), &dummy);
    const TD cj = Fj * S1;
    if (N == 2) {
      const TD l1k = ldD(sp + st1<CPLX>(m.k), &dummy);
      const float* p2 = sp + st2<CPLX>(a, m.j, m.k);
      const TD lamB = dexp(mul_s(uj + uk, tau));
      if (CPLX) {
        const TD lamA = dexp(mul_s(uj + conj(uk), tau));
        SA = lamA * SA + cj * conj(l1k) + ldD(p2, &dummy);
        SB = lamB * SB + cj * l1k + ldD(p2 + 2, &dummy);
      } else {
        SB = lamB * SB + cj * l1k + ldD(p2, &dummy);
      }
    }
    S1 = cj + l1j;
  }
  double* cr = a.carries + ((size_t)b * (a.C + 1) + a.C) * a.D;
  if (m.plane) stD(cr + st1<CPLX>(m.j), S1);
  if (N == 2) {
    double* p2 = cr + st2<CPLX>(a, m.j, m.k);
    if (CPLX) {
      stD(p2, SA);
      stD(p2 + 2, SB);
    } else {
      stD(p2, SB);
    }
  }
  if (a.readout == EWS_READOUT_TERMINAL) write_row_d<CPLX, N>(a, m, a.out + (size_t)b * a.W, S1, SA, SB, tid);
}

// ------------------------------------------------------------------------------------------- F4
__global__ void k_reduce_readout(DiagArgs a) {
  const int b = blockIdx.x;
  const bool is_max = a.readout == EWS_READOUT_MAX;
  for (int e = threadIdx.x; e < a.W; e += blockDim.x) {
    if (a.lvl0 && e == 0) {
      a.out[(size_t)b * a.W] = 1.0f;
      if (is_max) a.argmax[(size_t)b * a.W] = 0;
      continue;
    }
    if (is_max) {
      float best = -INFINITY;
      int bi = 0;
      for (int c = 0; c < a.C; ++c) {
        const float v = a.red[((size_t)b * a.C + c) * a.W + e];
        if (v > best) {
          best = v;
          bi = a.red_idx[((size_t)b * a.C + c) * a.W + e];
        }
      }
      a.out[(size_t)b * a.W + e] = best;
      a.argmax[(size_t)b * a.W + e] = bi;
    } else {
      double s = 0.0;
      for (int c = 0; c < a.C; ++c) s += (double)a.red[((size_t)b * a.C + c) * a.W + e];
      a.out[(size_t)b * a.W + e] = (float)(s / (double)a.n_int);
    }
  }
}

// ------------------------------------------------------------------------------------------- cotangents
// Cotangents of the lane's state at interval tg from the readout's cotangent (complex convention
// gamma = dL/dRe + i dL/dIm). Level 2 (complex): the row layout's block (j, k) is
// q00 = (ReSA + ReSB)/2, q01 = (ImSB - ImSA)/2, q10 = (ImSA + ImSB)/2, q11 = (ReSA - ReSB)/2.
template <bool CPLX, int N, class T>
__device__ __forceinline__ void gamma_at(const DiagArgs& a, const LaneMap& m, int b, int tg, T& g1, T& gA,
                                         T& gB) {
  g1 = zero<T>();
  gA = zero<T>();
  gB = zero<T>();
  const float* row;
  float scale = 1.0f;
  const int* am = nullptr;
  if (a.readout == EWS_READOUT_PREFIX) {
    row = a.gout + ((size_t)b * a.n_int + tg) * a.W;
  } else if (a.readout == EWS_READOUT_TERMINAL) {
    if (tg != a.n_int - 1) return;
    row = a.gout + (size_t)b * a.W;
  } else if (a.readout == EWS_READOUT_MEAN) {
    row = a.gout + (size_t)b * a.W;
    scale = 1.0f / (float)a.n_int;
  } else {
    row = a.gout + (size_t)b * a.W;
    am = a.argmax + (size_t)b * a.W;
  }
  auto G = [&](int e) -> float {
    if (am && am[e] != tg) return 0.0f;
    return row[e] * scale;
  };
  if (m.plane) {
    const int e = a.off1 + st1<CPLX>(m.j);
    if constexpr (CPLX) {
      g1 = cf{G(e), G(e + 1)};
    } else {
      g1 = G(e);
    }
  }
  if constexpr (N == 2) {
    if constexpr (CPLX) {
      const int e0 = a.off2 + (2 * m.j) * a.d + 2 * m.k;
      const float g00 = G(e0), g01 = G(e0 + 1), g10 = G(e0 + a.d), g11 = G(e0 + a.d + 1);
      gA = cf{0.5f * (g00 + g11), 0.5f * (g10 - g01)};
      gB = cf{0.5f * (g00 - g11), 0.5f * (g01 + g10)};
    } else {
      gB = G(a.off2 + m.j * a.d + m.k);
    }
  }
}

// ------------------------------------------------------------------------------------------- B1
// Chunk-local adjoint with zero incoming cotangent: the cotangent mu(c) on the chunk's carry-in.
// Level 1 uses linearity: each lane carries its pair's share of the plane cotangent, summed at the end.
template <bool CPLX, int N, int MAXT>
__global__ __launch_bounds__(MAXT) void k_chunk_bwd_local(DiagArgs a) {
  using T = typename Types<CPLX>::T;
  extern __shared__ float smem[];
  float* s_v = smem;
  float* s_h = s_v + a.T * a.d;
  float* s_red = s_h + a.T;  // MAXT * 2
  const int c = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
  const int t0 = c * a.T;
  const int Tc = min(a.T, a.n_int - t0);
  load_chunk(a, b, t0, Tc, s_v, s_h);
  __syncthreads();
  const LaneMap m = lane_map(a, tid);
  const ChunkClock cc = chunk_clock<T>(a, b, Tc, s_h);
  T dummy{};
  const T uj = load_u(a.params, m.j, &dummy);
  const T uk = load_u(a.params, m.k, &dummy);
  Coef<T> c0;
  CoefD<T> q;
  if (cc.fast) eval_coef<T, CPLX, N, true>(cc.hbar, cc.href, cc.per_int, uj, uk, c0, q);
  T L1 = zero<T>(), LA = zero<T>(), LB = zero<T>();
  if (m.active) {
    for (int t = Tc - 1; t >= 0; --t) {
      T g1, gA, gB;
      gamma_at<CPLX, N>(a, m, b, t0 + t, g1, gA, gB);
      L1 += g1;
      LA += gA;
      LB += gB;
      const float h = s_h[t];
      Coef<T> co;
      if (cc.fast) {
        lin_coef<T, CPLX, N>(c0, q, h - cc.hbar, cc.per_int, co);
      } else {
        CoefD<T> qq;
        eval_coef<T, CPLX, N, false>(h, cc.href, cc.per_int, uj, uk, co, qq);
      }
      T toC = zero<T>();
      if (N == 2) {
        const T pk = lds_p<T>(s_v, t, a.d, m.k);
        const T s1k = co.phi_k * pk;
        toC = conjc(s1k) * LB;
        if (CPLX) toC += s1k * LA;
        LB = conjc(co.lamB) * LB;
        if (CPLX) LA = conjc(co.lamA) * LA;
      }
      L1 = conjc(co.rho) * (L1 + toC);
    }
  }
  float* mp = a.mu + ((size_t)b * a.C + c) * a.D;
  if (N == 2) {
    // plane cotangent = sum over the row's lanes
    if (m.active) stT(s_red + 2 * tid, L1);
    __syncthreads();
    if (m.plane) {
      T s = zero<T>();
      for (int k = 0; k < a.K; ++k) s += ldT<CPLX, T>(s_red + 2 * (m.j * a.K + k));
      stT(mp + st1<CPLX>(m.j), s);
    }
    if (m.active) {
      float* p2 = mp + st2<CPLX>(a, m.j, m.k);
      if (CPLX) {
        stT(p2, LA);
        stT(p2 + 2, LB);
      } else {
        stT(p2, LB);
      }
    }
  } else if (m.active) {
    stT(mp + st1<CPLX>(m.j), L1);
  }
}

// ------------------------------------------------------------------------------------------- B2
// Reverse float64 scan of chunk cotangents: X(c) = mu(c) + J_c^T X(c+1); writes mt[c-1] = X(c) (the cotangent
// on chunk c-1's end state coming from chunks >= c) and mt[C-1] = 0.
template <bool CPLX, int N, int MAXT>
__global__ __launch_bounds__(MAXT) void k_adjoint_scan(DiagArgs a) {
  using TD = typename Types<CPLX>::TD;
  __shared__ double s_red[2 * MAXT];
  const int b = blockIdx.x, tid = threadIdx.x;
  const LaneMap m = lane_map(a, tid);
  TD dummy{};
  const TD uj = load_ud(a.params, m.j, &dummy);
  const TD uk = load_ud(a.params, m.k, &dummy);
  TD X1{}, XA{}, XB{};
  // mt[C-1] = 0
  {
    float* mp = a.mt + ((size_t)b * a.C + (a.C - 1)) * a.D;
    for (int i = tid; i < a.D; i += blockDim.x) mp[i] = 0.0f;
  }
  for (int c = a.C - 1; c >= 1; --c) {
    const int Tc = min(a.T, a.n_int - c * a.T);
    const double tau = chunk_tau(a, b, c, Tc);
    const TD Fj = dexp(mul_s(uj, tau));
    TD toC{};
    if (N == 2 && m.active) {
      // chunk c's zero-carry level-1 increment l1_k = carry1(c+1) - F_k carry1(c)
      const double* cr0 = a.carries + ((size_t)b * (a.C + 1) + c) * a.D;
      const double* cr1 = cr0 + a.D;
      const TD Fk = dexp(mul_s(uk, tau));
      const TD l1k = ldDD(cr1 + st1<CPLX>(m.k), &dummy) - Fk * ldDD(cr0 + st1<CPLX>(m.k), &dummy);
      toC = conj(l1k) * XB;
      if (CPLX) toC = toC + l1k * XA;
      const TD lamB = dexp(mul_s(uj + uk, tau));
      XB = conj(lamB) * XB;
      if (CPLX) {
        const TD lamA = dexp(mul_s(uj + conj(uk), tau));
        XA = conj(lamA) * XA;
      }
    }
    if (N == 2) {
      if (m.active) stD(s_red + 2 * tid, toC);
      __syncthreads();
      if (m.plane) {
        TD s = X1;
        for (int k = 0; k < a.K; ++k) s = s + ldDD(s_red + 2 * (m.j * a.K + k), &dummy);
        X1 = conj(Fj) * s;
      }
      __syncthreads();
    } else if (m.plane) {
      X1 = conj(Fj) * X1;
    }
    // + mu(c)
    const float* mup = a.mu + ((size_t)b * a.C + c) * a.D;
    if (m.plane) X1 = X1 + ldD(mup + st1<CPLX>(m.j), &dummy);
    if (N == 2 && m.active) {
      const float* p2 = mup + st2<CPLX>(a, m.j, m.k);
      if (CPLX) {
        XA = XA + ldD(p2, &dummy);
        XB = XB + ldD(p2 + 2, &dummy);
      } else {
        XB = XB + ldD(p2, &dummy);
      }
    }
    float* mp = a.mt + ((size_t)b * a.C + (c - 1)) * a.D;
    if (m.plane) {
      mp[st1<CPLX>(m.j)] = (float)dre(X1);
      if (CPLX) mp[st1<CPLX>(m.j) + 1] = (float)dim_(X1);
    }
    if (N == 2 && m.active) {
      float* p2 = mp + st2<CPLX>(a, m.j, m.k);
      p2[0] = (float)dre(CPLX ? XA : XB);
      if (CPLX) {
        p2[1] = (float)dim_(XA);
        p2[2] = (float)dre(XB);
        p2[3] = (float)dim_(XB);
      }
    }
  }
}

// ------------------------------------------------------------------------------------------- B3
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ float redot(cf a, cf b) { return a.re * b.re + a.im * b.im; }  // Re(conj(a) b)
__device__ __forceinline__ float redot(float a, float b) { return a * b; }

// parameter gradient of a node h*u with complex cotangent G (already carrying the factor h):
// x-type u = -conj(z) = -(d - i w): (dd, dw) += (-Re G, Im G); z-type u = -z: (dd, dw) += (-Re G, -Im G)
__device__ __forceinline__ void node_to_par(cf G, bool ztype, float& dd, float& dw) {
  dd += -G.re;
  dw += ztype ? -G.im : G.im;
}
__device__ __forceinline__ void node_to_par(float G, bool, float& dd, float&) { dd += -G; }

template <bool CPLX, int N, int MAXT>
__global__ __launch_bounds__(MAXT) void k_chunk_bwd_full(DiagArgs a) {
  using T = typename Types<CPLX>::T;
  constexpr int NS = CPLX ? 6 : 2;  // checkpoint floats per lane
  constexpr int BLK = 8;
  extern __shared__ float smem[];
  float* s_v = smem;
  float* s_h = s_v + a.T * a.d;
  const int nblk = (a.T + BLK - 1) / BLK;
  const int NT = blockDim.x, NW = (NT + 63) / 64;
  float* s_ck = s_h + a.T;                       // nblk * NS * NT
  float* s_rC = s_ck + nblk * NS * NT;           // 2 * NT  (sum over k -> row j)
  float* s_rP = s_rC + 2 * NT;                   // 2 * NT  (sum over k -> row j)
  float* s_cS = s_rP + 2 * NT;                   // 2 * NT  (sum over j -> column k)
  float* s_cP = s_cS + 2 * NT;                   // 2 * NT  (sum over j -> column k)
  float* s_dh = s_cP + 2 * NT;                   // T * NW
  float* s_g = s_dh + a.T * NW;                  // NT * 4 parameter partials
  const int c = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
  const int t0 = c * a.T;
  const int Tc = min(a.T, a.n_int - t0);
  load_chunk(a, b, t0, Tc, s_v, s_h);
  __syncthreads();
  const LaneMap m = lane_map(a, tid);
  const ChunkClock cc = chunk_clock<T>(a, b, Tc, s_h);
  T dummy{};
  const T uj = load_u(a.params, m.j, &dummy);
  const T uk = load_u(a.params, m.k, &dummy);
  const T ua = uj + conjc(uk), ub = uj + uk;
  Coef<T> c0;
  CoefD<T> q0;
  if (cc.fast) eval_coef<T, CPLX, N, true>(cc.hbar, cc.href, cc.per_int, uj, uk, c0, q0);

  // forward pre-pass from the carry: checkpoints of the state before every BLK-th step
  T S1 = zero<T>(), SA = zero<T>(), SB = zero<T>();
  {
    const double* cr = a.carries + ((size_t)b * (a.C + 1) + c) * a.D;
    if (m.active) {
      S1 = ldTd<CPLX, T>(cr + st1<CPLX>(m.j));
      if (N == 2) {
        const double* p2 = cr + st2<CPLX>(a, m.j, m.k);
        if (CPLX) {
          SA = ldTd<CPLX, T>(p2);
          SB = ldTd<CPLX, T>(p2 + 2);
        } else {
          SB = ldTd<CPLX, T>(p2);
        }
      }
    }
  }
  auto ck_store = [&](int blk) {
    float* p = s_ck + (size_t)blk * NS * NT;
    if constexpr (CPLX) {
      const cf s1 = S1, sa = SA, sb = SB;
      p[0 * NT + tid] = s1.re;
      p[1 * NT + tid] = s1.im;
      p[2 * NT + tid] = sa.re;
      p[3 * NT + tid] = sa.im;
      p[4 * NT + tid] = sb.re;
      p[5 * NT + tid] = sb.im;
    } else {
      p[0 * NT + tid] = S1;
      p[1 * NT + tid] = SB;
    }
  };
  auto ck_load = [&](int blk) {
    const float* p = s_ck + (size_t)blk * NS * NT;
    if constexpr (CPLX) {
      S1 = cf{p[0 * NT + tid], p[1 * NT + tid]};
      SA = cf{p[2 * NT + tid], p[3 * NT + tid]};
      SB = cf{p[4 * NT + tid], p[5 * NT + tid]};
    } else {
      S1 = p[0 * NT + tid];
      SB = p[1 * NT + tid];
    }
  };
  auto coef_at = [&](int t, Coef<T>& co, CoefD<T>& qq) {
    if (cc.fast) {
      lin_coef<T, CPLX, N>(c0, q0, s_h[t] - cc.hbar, cc.per_int, co);
      qq = q0;
    } else {
      eval_coef<T, CPLX, N, true>(s_h[t], cc.href, cc.per_int, uj, uk, co, qq);
    }
  };
  for (int t = 0; t < Tc; ++t) {
    if ((t % BLK) == 0) ck_store(t / BLK);
    Coef<T> co;
    CoefD<T> qq;
    coef_at(t, co, qq);
    const T pj = lds_p<T>(s_v, t, a.d, m.j);
    const T pk = (N == 2) ? lds_p<T>(s_v, t, a.d, m.k) : zero<T>();
    fwd_step<T, CPLX, N>(co, pj, pk, S1, SA, SB);
  }
  for (int i = tid; i < a.T * NW; i += NT) s_dh[i] = 0.0f;

  // cotangents on the chunk's end state from later chunks
  T L1 = zero<T>(), LA = zero<T>(), LB = zero<T>();
  {
    const float* mp = a.mt + ((size_t)b * a.C + c) * a.D;
    if (m.plane) L1 = ldT<CPLX, T>(mp + st1<CPLX>(m.j));
    if (N == 2 && m.active) {
      const float* p2 = mp + st2<CPLX>(a, m.j, m.k);
      if (CPLX) {
        LA = ldT<CPLX, T>(p2);
        LB = ldT<CPLX, T>(p2 + 2);
      } else {
        LB = ldT<CPLX, T>(p2);
      }
    }
  }
  // parameter-gradient accumulators (node cotangents times h)
  T Gx = zero<T>(), GyA = zero<T>(), GyB = zero<T>(), Gxp = zero<T>();
  T Sflow = zero<T>(), SflowA = zero<T>(), SflowB = zero<T>();  // cached flows: summed cotangents
  const int wid = tid / 64;

  __syncthreads();
  for (int blk = nblk - 1; blk >= 0; --blk) {
    if (blk * BLK >= Tc) continue;
    // recompute the block's states S(t-1)
    T H1[BLK], HA[BLK], HB[BLK];
    ck_load(blk);
#pragma unroll
    for (int s = 0; s < BLK; ++s) {
      const int t = blk * BLK + s;
      H1[s] = S1;
      HA[s] = SA;
      HB[s] = SB;
      if (t < Tc) {
        Coef<T> co;
        CoefD<T> qq;
        coef_at(t, co, qq);
        const T pj = lds_p<T>(s_v, t, a.d, m.j);
        const T pk = (N == 2) ? lds_p<T>(s_v, t, a.d, m.k) : zero<T>();
        fwd_step<T, CPLX, N>(co, pj, pk, S1, SA, SB);
      }
    }
#pragma unroll
    for (int s = BLK - 1; s >= 0; --s) {
      const int t = blk * BLK + s;
      if (t >= Tc) continue;
      const int tg = t0 + t;
      const float h = s_h[t];
      T g1, gA, gB;
      if (m.active) gamma_at<CPLX, N>(a, m, b, tg, g1, gA, gB);
      else g1 = gA = gB = zero<T>();
      L1 += g1;
      LA += gA;
      LB += gB;
      Coef<T> co;
      CoefD<T> qq;
      coef_at(t, co, qq);
      const T pj = lds_p<T>(s_v, t, a.d, m.j);
      const T pk = (N == 2) ? lds_p<T>(s_v, t, a.d, m.k) : zero<T>();
      const T cj = co.rho * H1[s];
      float dhp = 0.0f;
      if (N == 2) {
        const T s1k = co.phi_k * pk;
        T toC = conjc(s1k) * LB, toS = conjc(cj) * LB;
        const T gf = conjc(co.IB) * LB;
        T toPj = conjc(pk) * gf, toPk = conjc(pj) * gf;
        const T gIB = conjc(pj * pk) * LB;
        const T gLB = conjc(HB[s]) * LB;
        Gx += h * (gIB * conjc(qq.DxB));
        GyB += h * (gIB * conjc(qq.DyB));
        dhp += redot(gIB, qq.IB1);
        if (cc.per_int) {
          GyB += h * (gLB * conjc(co.lamB));
          dhp += redot(gLB, qq.lamB1);
        } else {
          SflowB += gLB;
        }
        if (CPLX) {
          toC += s1k * LA;
          toS += conjc(LA) * cj;
          const T ge = conjc(co.IA) * LA;
          toPj += pk * ge;
          toPk += conjc(ge) * pj;
          const T gIA = conjc(pj * conjc(pk)) * LA;
          const T gLA = conjc(HA[s]) * LA;
          Gx += h * (gIA * conjc(qq.DxA));
          GyA += h * (gIA * conjc(qq.DyA));
          dhp += redot(gIA, qq.IA1);
          if (cc.per_int) {
            GyA += h * (gLA * conjc(co.lamA));
            dhp += redot(gLA, qq.lamA1);
          } else {
            SflowA += gLA;
          }
          LA = conjc(co.lamA) * LA;
        }
        LB = conjc(co.lamB) * LB;
        if (m.active) {
          stT(s_rC + 2 * tid, toC);
          stT(s_rP + 2 * tid, toPj);
          // column arrays are indexed by (k, j) so a plane lane reads a contiguous run
          const int ct = m.k * a.K + m.j;
          stT(s_cS + 2 * ct, toS);
          stT(s_cP + 2 * ct, toPk);
        }
      }
      __syncthreads();
      if (m.plane) {
        T rowC = zero<T>(), rowP = zero<T>(), colS = zero<T>(), colP = zero<T>();
        if (N == 2) {
          for (int kk = 0; kk < a.K; ++kk) {
            rowC += ldT<CPLX, T>(s_rC + 2 * (m.j * a.K + kk));
            rowP += ldT<CPLX, T>(s_rP + 2 * (m.j * a.K + kk));
            colS += ldT<CPLX, T>(s_cS + 2 * (m.j * a.K + kk));
            colP += ldT<CPLX, T>(s_cP + 2 * (m.j * a.K + kk));
          }
        }
        const T gc = L1 + rowC;
        const T gs1 = L1 + colS;
        const T gp = conjc(co.phi_j) * gs1 + rowP + colP;
        float* dvp = a.dv + ((size_t)b * a.n_int + tg) * a.d + st1<CPLX>(m.j);
        dvp[0] = re(gp);
        if (CPLX) dvp[1] = im(gp);
        const T grho = conjc(H1[s]) * gc;
        const T gphi = conjc(pj) * gs1;
        Gxp += h * (gphi * conjc(qq.dphi_j));
        dhp += redot(gphi, qq.phi_j1);
        if (cc.per_int) {
          Gxp += h * (grho * conjc(co.rho));
          dhp += redot(grho, qq.rho1);
        } else {
          Sflow += grho;
        }
        L1 = conjc(co.rho) * gc;
      }
      const float ws = wave_sum(dhp);
      if ((tid & 63) == 0) s_dh[t * NW + wid] = ws;
      __syncthreads();
    }
  }

  // dh of the chunk's intervals (fixed-order sum over waves)
  for (int t = tid; t < Tc; t += NT) {
    float s = 0.0f;
    for (int w = 0; w < NW; ++w) s += s_dh[t * NW + w];
    a.dh[(size_t)b * a.n_int + t0 + t] = s;
  }
  // parameter partials: lane (j, k) -> plane j (row) and plane k (column) contributions, then plane sums
  float pj_d = 0.0f, pj_w = 0.0f, pk_d = 0.0f, pk_w = 0.0f, dhref = 0.0f;
  if (m.active) {
    if (!cc.per_int) {
      // cached flows: every step used the reference step href
      const float hr = cc.href;
      if (N == 2) {
        const T lamB = expv(hr * ub);
        GyB += hr * (SflowB * conjc(lamB));
        dhref += redot(SflowB, lamB * ub);
        if (CPLX) {
          const T lamA = expv(hr * ua);
          GyA += hr * (SflowA * conjc(lamA));
          dhref += redot(SflowA, lamA * ua);
        }
      }
      if (m.plane) {
        const T rho = expv(hr * uj);
        Gxp += hr * (Sflow * conjc(rho));
        dhref += redot(Sflow, rho * uj);
      }
    }
    node_to_par(Gx + Gxp, false, pj_d, pj_w);
    node_to_par(GyB, false, pj_d, pj_w);
    node_to_par(GyB, false, pk_d, pk_w);
    if (CPLX) {
      node_to_par(GyA, false, pj_d, pj_w);
      node_to_par(GyA, true, pk_d, pk_w);
    }
  }
  __syncthreads();
  s_g[4 * tid + 0] = pj_d;
  s_g[4 * tid + 1] = pj_w;
  s_g[4 * tid + 2] = pk_d;
  s_g[4 * tid + 3] = pk_w;
  const float whr = wave_sum(dhref);
  if ((tid & 63) == 0) s_dh[wid] = whr;  // s_dh no longer needed for steps
  __syncthreads();
  if (tid < a.K) {
    const int j = tid;
    float sd = 0.0f, sw = 0.0f;
    const int rows = (a.N == 2) ? a.K : 1;
    for (int kk = 0; kk < rows; ++kk) {
      const int lr = (a.N == 2) ? j * a.K + kk : j;  // lane (j, kk): row contributions
      sd += s_g[4 * lr + 0];
      sw += s_g[4 * lr + 1];
      if (a.N == 2) {
        const int lc = kk * a.K + j;  // lane (kk, j): column contributions
        sd += s_g[4 * lc + 2];
        sw += s_g[4 * lc + 3];
      }
    }
    float* gp = a.gp + ((size_t)b * a.C + c) * a.npar;
    if (CPLX) {
      gp[2 * j] = sd;
      gp[2 * j + 1] = sw;
    } else {
      gp[j] = sd;
    }
  }
  if (tid == 0) {
    float s = 0.0f;
    for (int w = 0; w < NW; ++w) s += s_dh[w];
    a.gph[(size_t)b * a.C + c] = s;
  }
}

// ------------------------------------------------------------------------------------------- B4
__global__ void k_knot_grads(DiagArgs a) {
  const size_t total = (size_t)a.B * a.L;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x) {
    const int b = (int)(i / a.L), t = (int)(i % a.L);
    const float* dvb = a.dv + (size_t)b * a.n_int * a.d;
    for (int ch = 0; ch < a.d; ++ch) {
      float g = 0.0f;
      if (t >= 1) g += dvb[(size_t)(t - 1) * a.d + ch];
      if (t < a.n_int) g -= dvb[(size_t)t * a.d + ch];
      a.dpath[i * a.d + ch] = g;
    }
    const float* dhb = a.dh + (size_t)b * a.n_int;
    float g = 0.0f;
    if (t >= 1) g += dhb[t - 1];
    if (t < a.n_int) g -= dhb[t];
    if (a.flow_mode != EWS_FLOW_PER_INTERVAL) {
      // shared flow step href = theta[r+1] - theta[r]
      const int r = (a.flow_mode == EWS_FLOW_CACHED) ? 0 : 1;
      double hs = 0.0;
      for (int c = 0; c < a.C; ++c) hs += (double)a.gph[(size_t)b * a.C + c];
      if (t == r + 1) g += (float)hs;
      if (t == r) g -= (float)hs;
    }
    a.dclock[i] = g;
  }
}

__global__ void k_param_grads(DiagArgs a) {
  for (int p = threadIdx.x; p < a.npar; p += blockDim.x) {
    double s = 0.0;
    for (int bc = 0; bc < a.B * a.C; ++bc) s += (double)a.gp[(size_t)bc * a.npar + p];
    a.dparams[p] = (float)s;
  }
}

}  // namespace ews

// ================================================================================================= C ABI
namespace {

using namespace ews;

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

struct Plan {
  int B, L, n_int, d, K, N, T, C, D, W, npar;
  bool cplx;
  int NT;
};

int make_plan(const ews_diag_desc* s, Plan& p) {
  if (!s) return EWS_ERR_NULL;
  if (s->structure != EWS_STRUCT_PLANES && s->structure != EWS_STRUCT_REAL_DIAG) return EWS_ERR_OPTION;
  if (s->flow_mode < 0 || s->flow_mode > 2) return EWS_ERR_OPTION;
  if (s->readout < 0 || s->readout > 3) return EWS_ERR_OPTION;
  if (s->path_dtype != EWS_DTYPE_F32 && s->path_dtype != EWS_DTYPE_BF16) return EWS_ERR_OPTION;
  if (s->depth != 1 && s->depth != 2) return EWS_ERR_DEPTH;
  if (s->batch < 1 || s->length < 2 || s->dim < 1) return EWS_ERR_SHAPE;
  p.cplx = s->structure == EWS_STRUCT_PLANES;
  if (p.cplx && (s->dim % 2 != 0 || s->dim > 64)) return EWS_ERR_SHAPE;
  if (!p.cplx && s->dim > 32) return EWS_ERR_SHAPE;
  if ((s->flow_mode == EWS_FLOW_CACHED_BASEPOINT) && s->length < 3) return EWS_ERR_SHAPE;
  p.B = s->batch;
  p.L = s->length;
  p.n_int = p.L - 1;
  p.d = s->dim;
  p.K = p.cplx ? p.d / 2 : p.d;
  p.N = s->depth;
  p.D = p.d + (p.N == 2 ? p.d * p.d : 0);
  p.W = p.D + (s->level0 ? 1 : 0);
  p.npar = p.cplx ? 2 * p.K : p.K;
  const int P = (p.N == 2) ? p.K * p.K : p.K;
  p.NT = ((P + 63) / 64) * 64;
  int T = s->chunk > 0 ? s->chunk : (p.NT >= 512 ? 32 : 64);
  if (T > 256) T = 256;
  p.T = T;
  p.C = (p.n_int + T - 1) / T;
  return EWS_OK;
}

struct WsLayout {
  size_t summ, mu, mt, red, red_idx, dv, dh, gp, gph, total;
};
WsLayout ws_layout(const Plan& p) {
  WsLayout w;
  size_t off = 0;
  const size_t BC = (size_t)p.B * p.C;
  w.summ = off; off += align256(BC * p.D * 4);
  w.mu = off; off += align256(BC * p.D * 4);
  w.mt = off; off += align256(BC * p.D * 4);
  w.red = off; off += align256(BC * p.W * 4);
  w.red_idx = off; off += align256(BC * p.W * 4);
  w.dv = off; off += align256((size_t)p.B * p.n_int * p.d * 4);
  w.dh = off; off += align256((size_t)p.B * p.n_int * 4);
  w.gp = off; off += align256(BC * p.npar * 4);
  w.gph = off; off += align256(BC * 4);
  w.total = off;
  return w;
}
size_t resid_carries_bytes(const Plan& p) { return align256((size_t)p.B * (p.C + 1) * p.D * 8); }

DiagArgs make_args(const ews_diag_desc* s, const Plan& p, const void* path, const float* clock,
                   const float* params, void* residual, void* workspace) {
  DiagArgs a{};
  a.B = p.B; a.L = p.L; a.n_int = p.n_int; a.d = p.d; a.K = p.K; a.N = p.N;
  a.flow_mode = s->flow_mode; a.readout = s->readout; a.T = p.T; a.C = p.C;
  a.W = p.W; a.lvl0 = s->level0 ? 1 : 0; a.off1 = a.lvl0; a.off2 = a.lvl0 + p.d; a.D = p.D; a.npar = p.npar;
  a.path_bf16 = s->path_dtype == EWS_DTYPE_BF16;
  a.path = path; a.clock = clock; a.params = params;
  char* r = (char*)residual;
  a.carries = (double*)r;
  a.argmax = (int*)(r + resid_carries_bytes(p));
  const WsLayout w = ws_layout(p);
  char* ws = (char*)workspace;
  a.summ = (float*)(ws + w.summ); a.mu = (float*)(ws + w.mu); a.mt = (float*)(ws + w.mt);
  a.red = (float*)(ws + w.red); a.red_idx = (int*)(ws + w.red_idx);
  a.dv = (float*)(ws + w.dv); a.dh = (float*)(ws + w.dh);
  a.gp = (float*)(ws + w.gp); a.gph = (float*)(ws + w.gph);
  return a;
}

size_t fwd_lds(const Plan& p) { return (size_t)(p.T * p.d + p.T) * 4; }
size_t bwd_local_lds(const Plan& p) { return fwd_lds(p) + (size_t)2 * p.NT * 4; }
size_t bwd_full_lds(const Plan& p) {
  const int NS = p.cplx ? 6 : 2;
  const int nblk = (p.T + 7) / 8;
  const int NW = p.NT / 64;
  return fwd_lds(p) + ((size_t)nblk * NS * p.NT + 8 * p.NT + (size_t)p.T * NW + 4 * p.NT) * 4;
}

#define EWS_LAUNCH_CHECK()                                  \
  do {                                                      \
    if (hipGetLastError() != hipSuccess) return EWS_ERR_LAUNCH; \
  } while (0)

template <bool CPLX, int N, int MAXT>
int run_forward(const ews_diag_desc* s, const Plan& p, DiagArgs a, hipStream_t st) {
  dim3 grid(p.C, p.B), blk(p.NT);
  hipLaunchKernelGGL((k_chunk_fwd<CPLX, N, MODE_SUMMARY, MAXT>), grid, blk, fwd_lds(p), st, a);
  EWS_LAUNCH_CHECK();
  hipLaunchKernelGGL((k_carry_scan<CPLX, N, MAXT>), dim3(p.B), blk, 0, st, a);
  EWS_LAUNCH_CHECK();
  if (s->readout == EWS_READOUT_PREFIX) {
    hipLaunchKernelGGL((k_chunk_fwd<CPLX, N, MODE_PREFIX, MAXT>), grid, blk, fwd_lds(p), st, a);
    EWS_LAUNCH_CHECK();
  } else if (s->readout == EWS_READOUT_MEAN || s->readout == EWS_READOUT_MAX) {
    hipLaunchKernelGGL((k_chunk_fwd<CPLX, N, MODE_REDUCE, MAXT>), grid, blk, fwd_lds(p), st, a);
    EWS_LAUNCH_CHECK();
    hipLaunchKernelGGL(k_reduce_readout, dim3(p.B), dim3(256), 0, st, a);
    EWS_LAUNCH_CHECK();
  }
  return EWS_OK;
}

template <bool CPLX, int N, int MAXT>
int run_backward(const Plan& p, DiagArgs a, hipStream_t st) {
  dim3 grid(p.C, p.B), blk(p.NT);
  hipLaunchKernelGGL((k_chunk_bwd_local<CPLX, N, MAXT>), grid, blk, bwd_local_lds(p), st, a);
  EWS_LAUNCH_CHECK();
  hipLaunchKernelGGL((k_adjoint_scan<CPLX, N, MAXT>), dim3(p.B), blk, 0, st, a);
  EWS_LAUNCH_CHECK();
  const size_t lds = bwd_full_lds(p);
  if (lds > 65536) {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(&k_chunk_bwd_full<CPLX, N, MAXT>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess)
      return EWS_ERR_LAUNCH;
  }
  hipLaunchKernelGGL((k_chunk_bwd_full<CPLX, N, MAXT>), grid, blk, lds, st, a);
  EWS_LAUNCH_CHECK();
  const size_t total = (size_t)p.B * p.L;
  const int nb = (int)((total + 255) / 256 < 4096 ? (total + 255) / 256 : 4096);
  hipLaunchKernelGGL(k_knot_grads, dim3(nb), dim3(256), 0, st, a);
  EWS_LAUNCH_CHECK();
  hipLaunchKernelGGL(k_param_grads, dim3(1), dim3(256), 0, st, a);
  EWS_LAUNCH_CHECK();
  return EWS_OK;
}

}  // namespace

extern "C" {

size_t ews_diag_workspace_bytes(const ews_diag_desc* desc) {
  Plan p;
  if (make_plan(desc, p) != EWS_OK) return 0;
  return ws_layout(p).total;
}

size_t ews_diag_residual_bytes(const ews_diag_desc* desc) {
  Plan p;
  if (make_plan(desc, p) != EWS_OK) return 0;
  return resid_carries_bytes(p) + align256((size_t)p.B * p.W * 4);
}

int ews_diag_forward(const ews_diag_desc* desc, const void* path, const float* clock, const float* params,
                     float* out, void* residual, void* workspace, ews_stream_t stream) {
  Plan p;
  const int rc = make_plan(desc, p);
  if (rc != EWS_OK) return rc;
  if (!path || !clock || !params || !out || !residual || !workspace) return EWS_ERR_NULL;
  DiagArgs a = make_args(desc, p, path, clock, params, residual, workspace);
  a.out = out;
  hipStream_t st = (hipStream_t)stream;
  const bool big = p.NT > 256;
  if (p.cplx) {
    if (p.N == 2) return big ? run_forward<true, 2, 1024>(desc, p, a, st) : run_forward<true, 2, 256>(desc, p, a, st);
    return run_forward<true, 1, 256>(desc, p, a, st);
  }
  if (p.N == 2) return big ? run_forward<false, 2, 1024>(desc, p, a, st) : run_forward<false, 2, 256>(desc, p, a, st);
  return run_forward<false, 1, 256>(desc, p, a, st);
}

int ews_diag_backward(const ews_diag_desc* desc, const void* path, const float* clock, const float* params,
                      const void* residual, const float* grad_out, float* grad_path, float* grad_clock,
                      float* grad_params, void* workspace, ews_stream_t stream) {
  Plan p;
  const int rc = make_plan(desc, p);
  if (rc != EWS_OK) return rc;
  if (!path || !clock || !params || !residual || !grad_out || !grad_path || !grad_clock || !grad_params ||
      !workspace)
    return EWS_ERR_NULL;
  DiagArgs a = make_args(desc, p, path, clock, params, (void*)residual, workspace);
  a.gout = grad_out;
  a.dpath = grad_path;
  a.dclock = grad_clock;
  a.dparams = grad_params;
  hipStream_t st = (hipStream_t)stream;
  const bool big = p.NT > 256;
  if (p.cplx) {
    if (p.N == 2) return big ? run_backward<true, 2, 1024>(p, a, st) : run_backward<true, 2, 256>(p, a, st);
    return run_backward<true, 1, 256>(p, a, st);
  }
  if (p.N == 2) return big ? run_backward<false, 2, 1024>(p, a, st) : run_backward<false, 2, 256>(p, a, st);
  return run_backward<false, 1, 256>(p, a, st);
}

const char* ews_error_string(int code) {
  switch (code) {
    case EWS_OK: return "ok";
    case EWS_ERR_NULL: return "a required pointer is NULL";
    case EWS_ERR_SHAPE: return "batch/length/dim out of range for this structure";
    case EWS_ERR_DEPTH: return "depth not supported by this structure";
    case EWS_ERR_OPTION: return "unknown structure, flow mode, readout or dtype";
    case EWS_ERR_LAUNCH: return "kernel launch failed";
    default: return "unknown error";
  }
}

const char* ews_version(void) { return "0.1.0"; }

}  // extern "C"
