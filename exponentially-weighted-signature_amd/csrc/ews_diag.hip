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

#include <mutex>
#include <type_traits>

#include "ews_args.h"
#include "ews_hip.h"
#include "ews_lanes.h"
#include "ews_numerics.h"
#include "ews_pairs.h"
#include "ews_seq.h"

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

// Global -> LDS copy with eight independent loads in flight per thread (a plain strided loop waits on each
// load before issuing the next).
__device__ __forceinline__ void copy_to_lds(float* dst, const float* src, int n) {
  const int st = blockDim.x;
  int i = threadIdx.x;
  for (; i + 7 * st < n; i += 8 * st) {
    float r[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) r[u] = src[i + u * st];
#pragma unroll
    for (int u = 0; u < 8; ++u) dst[i + u * st] = r[u];
  }
  for (; i < n; i += st) dst[i] = src[i];
}

// Increments v_t = X_{t+1} - X_t and clock steps h_t = theta_{t+1} - theta_t of chunk intervals [t0, t0+Tc).
__device__ __forceinline__ void load_chunk(const DiagArgs& a, int b, int t0, int Tc, float* s_v, float* s_h) {
  const size_t base = ((size_t)b * a.L + t0) * a.d;
  const int n = Tc * a.d, st = blockDim.x;
  int i = threadIdx.x;
  for (; i + 3 * st < n; i += 4 * st) {
    float x0[4], x1[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      x0[u] = load_path(a, base + i + u * st);
      x1[u] = load_path(a, base + i + u * st + a.d);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) s_v[i + u * st] = x1[u] - x0[u];
  }
  for (; i < n; i += st) s_v[i] = load_path(a, base + i + a.d) - load_path(a, base + i);
  const float* th = a.clock + (size_t)b * a.L + t0;
  for (int k = threadIdx.x; k < Tc; k += st) s_h[k] = th[k + 1] - th[k];
}
__device__ __forceinline__ void load_clock(const DiagArgs& a, int b, int t0, int Tc, float* s_h) {
  const float* th = a.clock + (size_t)b * a.L + t0;
  for (int k = threadIdx.x; k < Tc; k += blockDim.x) s_h[k] = th[k + 1] - th[k];
}

// ------------------------------------------------------------------------------------------- coefficients
template <class T> struct Coef {
  T rho, phi_j, phi_k, IA, IB, lamA, lamB;
  T rho_k;  // flow of the level-1 coordinate k (the log rows' S1_k)
};
template <class T> struct CoefD {
  T rho1, phi_j1, phi_k1, IA1, IB1, lamA1, lamB1, rho_k1;  // d/dh
  T dphi_j, dphi_k, DxA, DyA, DxB, DyB;                   // node derivatives
};

template <class T> __device__ __forceinline__ T conj_if(T x, bool) { return x; }
__device__ __forceinline__ cf conjc(cf x) { return conj(x); }
__device__ __forceinline__ float conjc(float x) { return x; }

// Coefficients at clock step h (flows at hf: h per interval, the shared step when cached). q1 / q2: series order
// of the level-1 / level-2 local terms (0: the exact closed forms; see node1q / dd3q); flows are always exact.
template <class T, bool CPLX, int N, bool DERIV>
__device__ __forceinline__ void eval_coef(int q1, int q2, float h, float hf, bool per_int, T uj, T uk, Coef<T>& c,
                                          CoefD<T>& q) {
  const T xj = h * uj;
  const Node1<T> nj = node1q(xj, q1);
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
    const Node1<T> nk = node1q(xk, q1);
    c.phi_k = nk.p;
    c.rho_k = per_int ? nk.e : expv(hf * uk);
    const T ub = uj + uk;
    const DD3<T> db = dd3q<T, DERIV>(xj, h * ub, q2);
    c.IB = db.d;
    c.lamB = expv(hf * ub);
    if (DERIV) {
      q.dphi_k = nk.dp;
      q.phi_k1 = nk.dp * uk;
      q.rho_k1 = per_int ? c.rho_k * uk : zero<T>();
      q.DxB = db.dx;
      q.DyB = db.dy;
      q.IB1 = db.dx * uj + db.dy * ub;
      q.lamB1 = per_int ? c.lamB * ub : zero<T>();
    }
    if (CPLX) {
      const T ua = uj + conjc(uk);
      const DD3<T> da = dd3q<T, DERIV>(xj, h * ua, q2);
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
    c.rho_k = per_int ? c0.rho_k + q.rho_k1 * dlt : c0.rho_k;
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
  bool inv_ok;  // stepping the recursion backwards amplifies errors by at most 2 over the chunk
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
  // with the pair-group kernels active (a.fast_ok) they own every uniform chunk; the chunks left here take exact
  // per-step coefficients, so that the FAST instantiations have no work and are not launched
  cc.fast = finite && (dmax * 2.0f * R < 1.52587890625e-5f) && !a.fast_ok;  // 2^-16
  cc.per_int = a.flow_mode == EWS_FLOW_PER_INTERVAL;
  const float* th = a.clock + (size_t)b * a.L;
  if (a.flow_mode == EWS_FLOW_CACHED) {
    cc.href = th[1] - th[0];
  } else if (a.flow_mode == EWS_FLOW_CACHED_BASEPOINT) {
    cc.href = a.L > 2 ? th[2] - th[1] : 0.0f;
  } else {
    cc.href = 0.0f;
  }
  // largest contraction rate Re(-u_j) (the damping d_j of a plane, lambda_j of a real channel); a level-2
  // element contracts at most at twice that rate, so the inverse step grows errors by e^{2 Dmax tau}
  float Dmax = 0.0f;
  for (int j = 0; j < a.K; ++j) Dmax = fmaxf(Dmax, -re(load_u(a.params, j, &dummy)));
  const float tau = cc.per_int ? s : fabsf(cc.href) * (float)Tc;
  cc.inv_ok = finite && (2.0f * Dmax * tau <= 0.69314718f);
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
// value of the lane tid ^ o of the wavefront

// Output row element indices of the lane's values (level 1 of plane j; the level-2 block (j, k)).
template <bool CPLX>
__device__ __forceinline__ void out_values(const DiagArgs& a, int j, int k, cf S1, cf SA, cf SB, int* idx,
                                           float* val, int& n1, int& n2);

// One LogEWS row of step t from the lane's states after the step (ews/layer.py:488-517 at depth 2: level 1, then
// log S at level 2 = S2 - S1 (x) S1 / 2 at the Lyndon words a < b, lexicographic; see ews_log.hip): the lane
// (j, k) writes the words of its level-2 block, the level-1 lanes the row's level 1 and its copy in s1rows (the
// backward's input for turning the log cotangent into a flat-row cotangent).
__device__ __forceinline__ int lyndon2(int i, int j, int d) { return i * (2 * d - i - 1) / 2 + (j - i - 1); }
template <bool CPLX, class T>
__device__ __forceinline__ void write_log_row(const DiagArgs& a, const LaneMap& m, int b, int t, T S1, T S1k, T SA,
                                              T SB) {
  float* row = a.out + ((size_t)b * a.n_int + t) * a.Wlog;
  const int d = a.d;
  if constexpr (CPLX) {
    const cf s1 = S1, s1k = S1k, sa = SA, sb = SB;
    if (m.plane) {
      row[2 * m.j] = s1.re;
      row[2 * m.j + 1] = s1.im;
      if (a.s1rows) {
        float* q = a.s1rows + ((size_t)b * a.n_int + t) * d + 2 * m.j;
        q[0] = s1.re;
        q[1] = s1.im;
      }
    }
    // the real 2 x 2 block (rows 2j, 2j+1; columns 2k, 2k+1) of the halved pair states, as the flat rows
    const float q00 = 0.5f * (sa.re + sb.re), q01 = 0.5f * (sb.im - sa.im);
    const float q10 = 0.5f * (sa.im + sb.im), q11 = 0.5f * (sa.re - sb.re);
    const int r0 = 2 * m.j, c0 = 2 * m.k;
    if (m.j < m.k) {
      row[d + lyndon2(r0, c0, d)] = q00 - 0.5f * s1.re * s1k.re;
      row[d + lyndon2(r0, c0 + 1, d)] = q01 - 0.5f * s1.re * s1k.im;
      row[d + lyndon2(r0 + 1, c0, d)] = q10 - 0.5f * s1.im * s1k.re;
      row[d + lyndon2(r0 + 1, c0 + 1, d)] = q11 - 0.5f * s1.im * s1k.im;
    } else if (m.j == m.k) {
      row[d + lyndon2(r0, r0 + 1, d)] = q01 - 0.5f * s1.re * s1.im;
    }
  } else {
    const float s1 = S1, s1k = S1k, sb = SB;
    if (m.plane) {
      row[m.j] = s1;
      if (a.s1rows) a.s1rows[((size_t)b * a.n_int + t) * d + m.j] = s1;
    }
    if (m.j < m.k) row[d + lyndon2(m.j, m.k, d)] = sb - 0.5f * s1 * s1k;
  }
}

// ------------------------------------------------------------------------------------------- F1 / F3
template <bool CPLX, int N, int MODE, int MAXT, bool FAST>
__global__ __launch_bounds__(MAXT) void k_chunk_fwd(DiagArgs a) {
  using T = typename Types<CPLX>::T;
  extern __shared__ float smem[];
  float* s_v = smem;
  float* s_h = s_v + a.T * a.d;
  const int c = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
  if (a.fast_ok && (a.cflag[b * a.C + c] & 1)) return;  // a pair-group kernel owns this chunk
  // generic chunks: the first summary pass (FAST) classifies every chunk and writes its class (bit 0 uniform,
  // bit 1 invertible); every later kernel reads it and leaves a chunk it does not own before staging anything
  constexpr bool kClassify = MODE == MODE_SUMMARY && FAST;
  if (!kClassify && !a.fast_ok && ((a.cflag[b * a.C + c] & 1) != 0) != FAST) return;
  const int t0 = c * a.T;
  const int Tc = min(a.T, a.n_int - t0);
  load_chunk(a, b, t0, Tc, s_v, s_h);
  __syncthreads();
  const LaneMap m = lane_map(a, tid);
  const ChunkClock cc = chunk_clock<T>(a, b, Tc, s_h);
  if (kClassify && !a.fast_ok && tid == 0) a.cflag[b * a.C + c] = (cc.fast ? 1 : 0) | (cc.inv_ok ? 2 : 0);
  if (cc.fast != FAST) return;  // the other instantiation owns this chunk
  if (!m.active) return;
  T dummy{};
  const T uj = load_u(a.params, m.j, &dummy);
  const T uk = load_u(a.params, m.k, &dummy);

  T S1 = zero<T>(), SA = zero<T>(), SB = zero<T>();
  T S1k = zero<T>();  // level 1 of coordinate k (log rows only)
  const bool logrows = MODE == MODE_PREFIX && N == 2 && a.log;
  if (MODE != MODE_SUMMARY) {
    const double* cr = a.carries + ((size_t)b * (a.C + 1) + c) * a.D;
    S1 = ldTd<CPLX, T>(cr + st1<CPLX>(m.j));
    if (logrows) S1k = ldTd<CPLX, T>(cr + st1<CPLX>(m.k));
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
  if constexpr (FAST) eval_coef<T, CPLX, N, true>(a.sq1, a.sq2, cc.hbar, cc.href, cc.per_int, uj, uk, c0, q);

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
    if constexpr (FAST) {
      lin_coef<T, CPLX, N>(c0, q, h - cc.hbar, cc.per_int, co);
    } else {
      CoefD<T> qq;
      eval_coef<T, CPLX, N, false>(a.sq1, a.sq2, h, cc.href, cc.per_int, uj, uk, co, qq);
    }
    const T pj = lds_p<T>(s_v, t, a.d, m.j);
    const T pk = (N == 2) ? lds_p<T>(s_v, t, a.d, m.k) : zero<T>();
    fwd_step<T, CPLX, N>(co, pj, pk, S1, SA, SB);
    if (MODE == MODE_SUMMARY) continue;
    if (logrows) {  // LogEWS row: level 1, then S2[a,b] - S1_a S1_b / 2 at the Lyndon words a < b
      S1k = co.rho_k * S1k + co.phi_k * pk;
      write_log_row<CPLX>(a, m, b, t0 + t, S1, S1k, SA, SB);
      continue;
    }
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

// ------------------------------------------------------------------------------------------- F3 + mixer
// The output pass with the block's mixer epilogue in it (ews/block.py:282-306, 336-357, 405-408; ews/norms.py:47-134;
// the same arithmetic as csrc/ews_mixer.hip k_mix_fwd): the chunk's prefix rows are staged in LDS kMixRB at a
// time, without their level-0 column, and contracted there against c_down on fp32 MFMA, so that only the
// hidden-wide rows and the mixer's residual (each level's products P_k, its scale and two derivative factors per
// row) reach memory; the D-wide rows are never written. The wavefronts of the workgroup split each level's 16-entry
// column blocks between them, and their partial products are summed through LDS. r = b + sum_k f_k P_k with
// P_k = W_k x_k on the unscaled row and f_k the level's prescale times its GradedRMSNorm factor.
constexpr int kMixRB = 16;  // rows staged per block (one MFMA row tile)
constexpr int kMixHT = 4;   // hidden tiles of 16: c_down up to 64 wide
constexpr int kMixNW = 4;   // wavefronts sharing the contraction (the others wait at its barriers)
typedef float mf4 __attribute__((ext_vector_type(4)));
typedef float mf4u __attribute__((ext_vector_type(4), aligned(4)));

struct MixEpi {
  const float* weight;  // (H, D) row-major: c_down's weight
  const float* bias;    // (H,)
  const float* gains;   // (N,) GradedRMSNorm gains, or (1,) lam for dilation
  float* out;           // (B, R + prepend, H)
  float* P;             // (B R, N, H) level products
  float* F;             // (B R, N, 3): scale, beta, d scale / d gain
  int H, variant, prepend, prescale;
  float eps[2];
};

__device__ __forceinline__ mf4 mix_load4(const float* p, int k, int end, bool ok) {
  if (!ok) return mf4{0.0f, 0.0f, 0.0f, 0.0f};
  if (k + 3 < end) {
    const mf4u v = *reinterpret_cast<const mf4u*>(p + k);
    return mf4{v.x, v.y, v.z, v.w};
  }
  return mf4{k < end ? p[k] : 0.0f, k + 1 < end ? p[k + 1] : 0.0f, k + 2 < end ? p[k + 2] : 0.0f,
             k + 3 < end ? p[k + 3] : 0.0f};
}

__device__ __forceinline__ int mix_pitch(int D) { return ((D + 3) & ~3) + 4; }

// x[k .. k+3] of a staged row: one 16-byte LDS read when the run starts on a 16-byte boundary (al: the level
// starts on one, as every level does when d is a multiple of 4, and the row pitch and k0 are multiples of 4); the
// row pitch (4 mod 32 words in 16-byte units: 7 mod 8) keeps the 16 rows of a read on distinct bank groups
__device__ __forceinline__ mf4 mix_lds4(const float* p, int k, int end, bool ok, bool al) {
  if (ok && al && k + 3 < end) return *reinterpret_cast<const mf4*>(p + k);
  return mix_load4(p, k, end, ok);
}

// The mixer epilogue of rows tb .. tb + nr - 1 of the chunk staged in s_rows (row pitch Dp, levels without level 0).
template <int N, int NH>
__device__ __forceinline__ void mix_block(const DiagArgs& a, const MixEpi& e, int b, int t0, int nr,
                                          const float* s_rows, float* s_red, float* s_ssq, float* s_fac) {
  const int tid = threadIdx.x, NW = min(blockDim.x >> 6, kMixNW), w = tid >> 6, l = tid & 63, i = l & 15,
            g = l >> 4;
  const int Dp = mix_pitch(a.D), NHT = (e.H + 15) >> 4, Hp = NHT * 16;
  const bool rok = i < nr, wok = w < NW, al = (a.d & 3) == 0;  // wok: uniform over the wavefront
  const float* xr = s_rows + (size_t)i * Dp;
  mf4 acc[N][NH];
  float ssq[N];
#pragma unroll
  for (int k = 0; k < N; ++k) {
    ssq[k] = 0.0f;
#pragma unroll
    for (int h = 0; h < NH; ++h) acc[k][h] = mf4{0.0f, 0.0f, 0.0f, 0.0f};
  }
#pragma unroll
  for (int k = 0; k < N; ++k) {
    const int st = k == 0 ? 0 : a.d, n = k == 0 ? a.d : a.d * a.d, en = st + n;
#pragma unroll 2
    for (int k0 = st + 16 * w; wok && k0 < en; k0 += 16 * NW) {  // the wavefront's 16-entry blocks of the level
      const int kk = k0 + 4 * g;
      const mf4 xa = mix_lds4(xr, kk, en, rok, al);
      ssq[k] = fmaf(xa.x, xa.x, fmaf(xa.y, xa.y, fmaf(xa.z, xa.z, fmaf(xa.w, xa.w, ssq[k]))));
#pragma unroll
      for (int h = 0; h < NH; ++h) {
        if (h < NHT) {  // uniform
          const int hrow = 16 * h + i;
          const bool hok = hrow < e.H;
          const mf4 wb = mix_load4(e.weight + (size_t)(hok ? hrow : 0) * a.D, kk, en, hok);
          acc[k][h] = __builtin_amdgcn_mfma_f32_16x16x4f32(xa.x, wb.x, acc[k][h], 0, 0, 0);
          acc[k][h] = __builtin_amdgcn_mfma_f32_16x16x4f32(xa.y, wb.y, acc[k][h], 0, 0, 0);
          acc[k][h] = __builtin_amdgcn_mfma_f32_16x16x4f32(xa.z, wb.z, acc[k][h], 0, 0, 0);
          acc[k][h] = __builtin_amdgcn_mfma_f32_16x16x4f32(xa.w, wb.w, acc[k][h], 0, 0, 0);
        }
      }
    }
  }
  __syncthreads();  // s_red overlays the staged rows
  // the wavefront's partial products (lane: rows 4g + r of column 16h + i) and partial sums of squares
#pragma unroll
  for (int k = 0; k < N && wok; ++k) {
#pragma unroll
    for (int h = 0; h < NH; ++h) {
      if (h < NHT) {
        float* rp = s_red + (((size_t)w * N + k) * 16) * Hp + 16 * h + i;
        rp[(4 * g + 0) * Hp] = acc[k][h].x;
        rp[(4 * g + 1) * Hp] = acc[k][h].y;
        rp[(4 * g + 2) * Hp] = acc[k][h].z;
        rp[(4 * g + 3) * Hp] = acc[k][h].w;
      }
    }
    float v = ssq[k];
    v = lanes::add_xor32(lanes::add_xor16(v));
    if (g == 0) s_ssq[((size_t)w * N + k) * 16 + i] = v;
  }
  __syncthreads();
  // per-row factors of each level (the arithmetic of k_mix_fwd)
#pragma unroll 1
  for (int q = tid; q < nr * N; q += blockDim.x) {
    const int r = q / N, k = q % N, K = k + 1;
    float v = 0.0f;
    for (int ww = 0; ww < NW; ++ww) v += s_ssq[((size_t)ww * N + k) * 16 + r];
    const int t = t0 + r;  // the row within its sample
    const size_t gr = (size_t)b * a.n_int + t;
    float c = 1.0f;
    if (e.prescale) {  // 1 / C(max(t + 1, K), K) with t counted from the levels' first row; K <= 2: the product
      const double tl = fmax((double)(t + 1 + e.prepend), (double)K);
      c = (float)(K == 1 ? 1.0 / tl : 2.0 / (tl * (tl - 1.0)));
    }
    const int nk = K == 1 ? a.d : a.d * a.d;
    float f, beta = 0.0f, dfdg;
    if (e.variant == EWS_GRADED_LIVE_RMS) {
      const float gk = e.gains[k];
      const float ms = v / (float)nk;
      const float rho = ms > 0.0f ? sqrtf(ms) : 0.0f;
      const float den = fmaf(c, rho, e.eps[k]);
      dfdg = c / den;
      f = gk * dfdg;
      if (rho > 0.0f) beta = gk * c * c / (den * den * (float)nk * rho);
    } else if (e.variant == EWS_GRADED_STATIC_GAIN) {
      dfdg = c;
      f = e.gains[k] * c;
    } else {
      const float lam = e.gains[0];
      const float lk1 = powf(lam, (float)(K - 1));
      dfdg = (float)K * lk1 * c;
      f = lk1 * lam * c;
    }
    s_fac[r * N + k] = f;
    float* fp = e.F + (gr * N + k) * 3;
    fp[0] = f;
    fp[1] = beta;
    fp[2] = dfdg;
  }
  __syncthreads();
  // output rows and the level products
#pragma unroll 1
  for (int q = tid; q < nr * e.H; q += blockDim.x) {
    const int r = q / e.H, col = q % e.H, t = t0 + r;
    const size_t gr = (size_t)b * a.n_int + t;
    float v = e.bias[col];
#pragma unroll
    for (int k = 0; k < N; ++k) {
      float pv = 0.0f;
      for (int ww = 0; ww < NW; ++ww) pv += s_red[(((size_t)ww * N + k) * 16 + r) * Hp + col];
      v = fmaf(s_fac[r * N + k], pv, v);
      e.P[(gr * N + k) * e.H + col] = pv;
    }
    e.out[((size_t)b * (a.n_int + e.prepend) + t + e.prepend) * e.H + col] = v;
  }
}

// LDS of k_chunk_mix: increments and steps, kMixRB staged rows (then, in the same space, the wavefronts' partial
// products), the partial sums of squares and the rows' factors
__host__ __device__ __forceinline__ size_t mix_rows_floats(int D, int NT, int N, int H) {
  const size_t rows = (size_t)kMixRB * (((D + 3) & ~3) + 4);
  const size_t red = (size_t)min((NT + 63) / 64, kMixNW) * N * 16 * (((H + 15) / 16) * 16);
  return rows > red ? rows : red;
}
__host__ __device__ __forceinline__ size_t mix_lds_floats(int T, int d, int D, int NT, int N, int H) {
  const int NW = min((NT + 63) / 64, kMixNW);
  return (size_t)T * d + ((T + 3) & ~3) + mix_rows_floats(D, NT, N, H) + (size_t)NW * N * 16 + (size_t)kMixRB * N;
}

template <bool CPLX, int N, int MAXT, bool FAST, int NH>
__global__ __launch_bounds__(MAXT) void k_chunk_mix(DiagArgs a, MixEpi e) {
  using T = typename Types<CPLX>::T;
  extern __shared__ float smem[];
  const int NW = min((int)(blockDim.x >> 6), kMixNW), Hp = ((e.H + 15) >> 4) * 16, Dp = mix_pitch(a.D);
  float* s_v = smem;
  float* s_h = s_v + a.T * a.d;
  float* s_rows = s_h + ((a.T + 3) & ~3);
  float* s_red = s_rows;  // after the contraction
  float* s_ssq = s_rows + mix_rows_floats(a.D, blockDim.x, N, e.H);
  float* s_fac = s_ssq + NW * N * 16;
  const int c = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
  // the chunk's class (written by the summary pass): the other instantiation owns it (uniform over the workgroup)
  if (((a.cflag[b * a.C + c] & 1) != 0) != FAST) return;
  const int t0 = c * a.T;
  const int Tc = min(a.T, a.n_int - t0);
  load_chunk(a, b, t0, Tc, s_v, s_h);
  __syncthreads();
  const LaneMap m = lane_map(a, tid);  // lanes past the pairs join the barriers of the mixer blocks
  const ChunkClock cc = chunk_clock<T>(a, b, Tc, s_h);
  T dummy{};
  const T uj = load_u(a.params, m.j, &dummy);
  const T uk = load_u(a.params, m.k, &dummy);
  T S1 = zero<T>(), SA = zero<T>(), SB = zero<T>();
  {
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
  if constexpr (FAST) eval_coef<T, CPLX, N, true>(a.sq1, a.sq2, cc.hbar, cc.href, cc.per_int, uj, uk, c0, q);
  for (int tb = 0; tb < Tc; tb += kMixRB) {
    const int nr = min(kMixRB, Tc - tb);
#pragma unroll 1
    for (int s = 0; s < nr; ++s) {
      const int t = tb + s;
      const float h = s_h[t];
      Coef<T> co;
      if constexpr (FAST) {
        lin_coef<T, CPLX, N>(c0, q, h - cc.hbar, cc.per_int, co);
      } else {
        CoefD<T> qq;
        eval_coef<T, CPLX, N, false>(a.sq1, a.sq2, h, cc.href, cc.per_int, uj, uk, co, qq);
      }
      const T pj = lds_p<T>(s_v, t, a.d, m.j);
      const T pk = (N == 2) ? lds_p<T>(s_v, t, a.d, m.k) : zero<T>();
      fwd_step<T, CPLX, N>(co, pj, pk, S1, SA, SB);
      if (!m.active) continue;
      float* row = s_rows + (size_t)s * Dp;  // levels without level 0: level 1 at 0, level 2 at d
      if (m.plane) {
        if constexpr (CPLX) {
          *reinterpret_cast<float2*>(row + st1<CPLX>(m.j)) = float2{re(S1), im(S1)};
        } else {
          row[st1<CPLX>(m.j)] = re(S1);
        }
      }
      if (N == 2) {
        if constexpr (CPLX) {  // 8-byte stores: d is even and the row pitch a multiple of 4
          const cf sa = SA, sb = SB;
          float* r0 = row + a.d + (2 * m.j) * a.d + 2 * m.k;
          *reinterpret_cast<float2*>(r0) = float2{0.5f * (sa.re + sb.re), 0.5f * (sb.im - sa.im)};
          *reinterpret_cast<float2*>(r0 + a.d) = float2{0.5f * (sa.im + sb.im), 0.5f * (sa.re - sb.re)};
        } else {
          row[a.d + m.j * a.d + m.k] = re(SB);
        }
      }
    }
    __syncthreads();
    mix_block<N, NH>(a, e, b, t0 + tb, nr, s_rows, s_red, s_ssq, s_fac);
    __syncthreads();  // the next block restages the rows
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

// Float64 Chen combine of chunk summaries, in three levels so no sequential chain is longer than a group:
//   group_agg    every group of scan_cb chunks combines its summaries from a zero state (parallel)
//   group_scan   per sample, the group aggregates are combined in order -> the state before each group
//   group_expand every group re-combines its chunks from its incoming state, writing carries[c]
// Chunk and group flows are exp(u * clock span) in float64 (per-interval flows multiply to that exactly).
__device__ __forceinline__ double span_tau(const DiagArgs& a, int b, int t_start, int t_end) {
  const float* th = a.clock + (size_t)b * a.L;
  if (a.flow_mode == EWS_FLOW_PER_INTERVAL) return (double)th[t_end] - (double)th[t_start];
  if (a.flow_mode == EWS_FLOW_CACHED) return ((double)th[1] - (double)th[0]) * (t_end - t_start);
  const double h1 = a.L > 2 ? (double)th[2] - (double)th[1] : 0.0;
  return h1 * (t_end - t_start - (t_start == 0 ? 1 : 0));
}

// S <- (flow F applied to S) (x) l, the Chen product of a state with a summary (pair lane view)
template <bool CPLX, int N, class TD>
__device__ __forceinline__ void chen_fwd_lane(TD& S1, TD& SA, TD& SB, TD Fj, TD Fk, TD l1j, TD l1k, TD l2A, TD l2B) {
  const TD cj = Fj * S1;
  if (N == 2) {
    if (CPLX) SA = (Fj * conj(Fk)) * SA + cj * conj(l1k) + l2A;
    SB = (Fj * Fk) * SB + cj * l1k + l2B;
  }
  S1 = cj + l1j;
}

template <bool CPLX, class TD>
__device__ __forceinline__ void lane_summary(const DiagArgs& a, const LaneMap& m, const float* sp, TD& l1j, TD& l1k,
                                             TD& l2A, TD& l2B) {
  TD dummy{};
  l1j = ldD(sp + st1<CPLX>(m.j), &dummy);
  l1k = ldD(sp + st1<CPLX>(m.k), &dummy);
  l2A = TD{};
  l2B = TD{};
  if (a.N == 2) {
    const float* p2 = sp + st2<CPLX>(a, m.j, m.k);
    if (CPLX) {
      l2A = ldD(p2, &dummy);
      l2B = ldD(p2 + 2, &dummy);
    } else {
      l2B = ldD(p2, &dummy);
    }
  }
}
template <bool CPLX, class TD>
__device__ __forceinline__ void lane_summary_d(const DiagArgs& a, const LaneMap& m, const double* sp, TD& l1j, TD& l1k,
                                               TD& l2A, TD& l2B) {
  TD dummy{};
  l1j = ldDD(sp + st1<CPLX>(m.j), &dummy);
  l1k = ldDD(sp + st1<CPLX>(m.k), &dummy);
  l2A = TD{};
  l2B = TD{};
  if (a.N == 2) {
    const double* p2 = sp + st2<CPLX>(a, m.j, m.k);
    if (CPLX) {
      l2A = ldDD(p2, &dummy);
      l2B = ldDD(p2 + 2, &dummy);
    } else {
      l2B = ldDD(p2, &dummy);
    }
  }
}
template <bool CPLX, int N, class TD>
__device__ __forceinline__ void store_lane_d(const DiagArgs& a, const LaneMap& m, double* row, TD S1, TD SA, TD SB) {
  if (m.plane) stD(row + st1<CPLX>(m.j), S1);
  if (N == 2) {
    double* p2 = row + st2<CPLX>(a, m.j, m.k);
    if (CPLX) {
      stD(p2, SA);
      stD(p2 + 2, SB);
    } else {
      stD(p2, SB);
    }
  }
}

// Stages a group's chunk summaries and chunk flows into LDS; returns the group's chunk range.
template <bool CPLX, class TD>
__device__ __forceinline__ int stage_group(const DiagArgs& a, int b, int g, float* s_l, double* s_F, int& c0) {
  constexpr int CW = CPLX ? 2 : 1;
  c0 = g * a.scan_cb;
  const int nb = min(a.scan_cb, a.C - c0);
  copy_to_lds(s_l, a.summ + ((size_t)b * a.C + c0) * a.D, nb * a.D);
  TD dummy{};
  for (int i = threadIdx.x; i < nb * a.K; i += blockDim.x) {
    const int cc = i / a.K, j = i % a.K, c = c0 + cc;
    const int t0 = c * a.T, t1 = min(t0 + a.T, a.n_int);
    stD(s_F + (size_t)i * CW, dexp(mul_s(load_ud(a.params, j, &dummy), span_tau(a, b, t0, t1))));
  }
  __syncthreads();
  return nb;
}

template <bool CPLX, int N, int MAXT, bool EXPAND>
__global__ __launch_bounds__(MAXT) void k_fwd_group(DiagArgs a) {
  using TD = typename Types<CPLX>::TD;
  constexpr int CW = CPLX ? 2 : 1;
  extern __shared__ double dsm[];
  double* s_F = dsm;
  float* s_l = reinterpret_cast<float*>(s_F + (size_t)a.scan_cb * a.K * CW);
  const int g = blockIdx.x, b = blockIdx.y;
  const LaneMap m = lane_map(a, threadIdx.x);
  int c0;
  const int nb = stage_group<CPLX, TD>(a, b, g, s_l, s_F, c0);
  if (!m.active) return;
  TD dummy{};
  TD S1{}, SA{}, SB{};
  // the first group starts from the zero state (its carry is not read: with one group the scan is not launched)
  if (EXPAND && g > 0) lane_summary_d<CPLX>(a, m, a.gcar + ((size_t)b * a.NG + g) * a.D, S1, dummy, SA, SB);
  for (int cc = 0; cc < nb; ++cc) {
    if (EXPAND) store_lane_d<CPLX, N>(a, m, a.carries + ((size_t)b * (a.C + 1) + c0 + cc) * a.D, S1, SA, SB);
    TD l1j, l1k, l2A, l2B;
    lane_summary<CPLX>(a, m, s_l + (size_t)cc * a.D, l1j, l1k, l2A, l2B);
    const TD Fj = ldDD(s_F + (size_t)(cc * a.K + m.j) * CW, &dummy);
    const TD Fk = ldDD(s_F + (size_t)(cc * a.K + m.k) * CW, &dummy);
    chen_fwd_lane<CPLX, N>(S1, SA, SB, Fj, Fk, l1j, l1k, l2A, l2B);
  }
  if (EXPAND) {
    if (c0 + nb == a.C) {
      store_lane_d<CPLX, N>(a, m, a.carries + ((size_t)b * (a.C + 1) + a.C) * a.D, S1, SA, SB);
      if (a.readout == EWS_READOUT_TERMINAL) write_row_d<CPLX, N>(a, m, a.out + (size_t)b * a.W, S1, SA, SB, threadIdx.x);
    }
  } else {
    store_lane_d<CPLX, N>(a, m, a.gagg + ((size_t)b * a.NG + g) * a.D, S1, SA, SB);
  }
}

template <bool CPLX, int N, int MAXT>
__global__ __launch_bounds__(MAXT) void k_fwd_group_scan(DiagArgs a) {
  using TD = typename Types<CPLX>::TD;
  const int b = blockIdx.x;
  const LaneMap m = lane_map(a, threadIdx.x);
  if (!m.active) return;
  TD dummy{};
  const TD uj = load_ud(a.params, m.j, &dummy), uk = load_ud(a.params, m.k, &dummy);
  // group g's span and aggregate are loaded one group ahead and issued before the group's carry is stored (the
  // memory counter is in order: a load issued after a store is waited for together with the store)
  struct Pre {
    double tau;
    TD l1j, l1k, l2A, l2B;
  };
  auto load = [&](int g, Pre& p) {
    const int t0 = g * a.scan_cb * a.T, t1 = min(t0 + a.scan_cb * a.T, a.n_int);
    p.tau = span_tau(a, b, t0, t1);
    lane_summary_d<CPLX>(a, m, a.gagg + ((size_t)b * a.NG + g) * a.D, p.l1j, p.l1k, p.l2A, p.l2B);
  };
  TD S1{}, SA{}, SB{};
  Pre cur{}, nxt{};
  if (a.NG > 0) load(0, cur);
  for (int g = 0; g < a.NG; ++g) {
    if (g + 1 < a.NG) load(g + 1, nxt);
    store_lane_d<CPLX, N>(a, m, a.gcar + ((size_t)b * a.NG + g) * a.D, S1, SA, SB);
    chen_fwd_lane<CPLX, N>(S1, SA, SB, dexp(mul_s(uj, cur.tau)), dexp(mul_s(uk, cur.tau)), cur.l1j, cur.l1k, cur.l2A,
                           cur.l2B);
    cur = nxt;
  }
}

// ---- backward: X(c) = mu(c) + J_c^T X(c+1) in the same three levels; mt[c] = X(c+1) (cotangent on chunk c's end
// state from later chunks). J_c^T: level 2 conj(flow) X2; level 1 conj(F_j) [X1_j + sum_k (conj(l1_k) XB_jk +
// l1_k XA_jk)], with l1 the chunk's level-1 increment carry1(c+1) - F carry1(c).
template <bool CPLX, int N, class TD>
__device__ __forceinline__ void adj_lane(const DiagArgs& a, const LaneMap& m, TD& X1, TD& XA, TD& XB, TD Fj, TD Fk,
                                         TD l1k, double* s_red) {
  constexpr int CW = CPLX ? 2 : 1;
  TD dummy{};
  TD toC{};
  if (N == 2 && m.active) {
    toC = conj(l1k) * XB;
    if (CPLX) toC = toC + l1k * XA;
    XB = conj(Fj * Fk) * XB;
    if (CPLX) XA = conj(Fj * conj(Fk)) * XA;
  }
  if (N == 2) {
    if (m.active) stD(s_red + (size_t)threadIdx.x * CW, toC);
    __syncthreads();
    if (m.plane) {
      TD s = X1;
      for (int k = 0; k < a.K; ++k) s = s + ldDD(s_red + (size_t)(m.j * a.K + k) * CW, &dummy);
      X1 = conj(Fj) * s;
    }
    __syncthreads();
  } else if (m.plane) {
    X1 = conj(Fj) * X1;
  }
}
template <bool CPLX, int N, class TD>
__device__ __forceinline__ void add_mu(const DiagArgs& a, const LaneMap& m, const float* mup, TD& X1, TD& XA, TD& XB) {
  TD dummy{};
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
}
template <bool CPLX, int N, class TD>
__device__ __forceinline__ void store_lane_f(const DiagArgs& a, const LaneMap& m, float* mp, TD X1, TD XA, TD XB) {
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

template <bool CPLX, int N, int MAXT, bool EXPAND>
__global__ __launch_bounds__(MAXT) void k_bwd_group(DiagArgs a) {
  using TD = typename Types<CPLX>::TD;
  constexpr int CW = CPLX ? 2 : 1;
  extern __shared__ double dsm[];
  const int G = a.scan_cb;
  double* s_F = dsm;                                   // G * K
  double* s_l1 = s_F + (size_t)G * a.K * CW;           // G * K
  double* s_red = s_l1 + (size_t)G * a.K * CW;         // NT
  float* s_mu = reinterpret_cast<float*>(s_red + (size_t)blockDim.x * CW);  // G * D
  const int g = blockIdx.x, b = blockIdx.y;
  const LaneMap m = lane_map(a, threadIdx.x);
  const int c0 = g * G, nb = min(G, a.C - c0);
  copy_to_lds(s_mu, a.mu + ((size_t)b * a.C + c0) * a.D, nb * a.D);
  TD dummy{};
  for (int i = threadIdx.x; i < nb * a.K; i += blockDim.x) {
    const int cc = i / a.K, j = i % a.K, c = c0 + cc;
    const int t0 = c * a.T, t1 = min(t0 + a.T, a.n_int);
    const TD F = dexp(mul_s(load_ud(a.params, j, &dummy), span_tau(a, b, t0, t1)));
    stD(s_F + (size_t)i * CW, F);
    const double* cr0 = a.carries + ((size_t)b * (a.C + 1) + c) * a.D;
    stD(s_l1 + (size_t)i * CW, ldDD(cr0 + a.D + st1<CPLX>(j), &dummy) - F * ldDD(cr0 + st1<CPLX>(j), &dummy));
  }
  __syncthreads();
  TD X1{}, XA{}, XB{};
  // the last group starts from a zero cotangent (its carry is not read: with one group the scan is not launched)
  if (EXPAND && g < a.NG - 1) lane_summary_d<CPLX>(a, m, a.gcar + ((size_t)b * a.NG + g) * a.D, X1, dummy, XA, XB);
  for (int cc = nb - 1; cc >= 0; --cc) {
    const int c = c0 + cc;
    if (EXPAND) store_lane_f<CPLX, N>(a, m, a.mt + ((size_t)b * a.C + c) * a.D, X1, XA, XB);
    const TD Fj = ldDD(s_F + (size_t)(cc * a.K + m.j) * CW, &dummy);
    const TD Fk = ldDD(s_F + (size_t)(cc * a.K + m.k) * CW, &dummy);
    const TD l1k = ldDD(s_l1 + (size_t)(cc * a.K + m.k) * CW, &dummy);
    adj_lane<CPLX, N>(a, m, X1, XA, XB, Fj, Fk, l1k, s_red);
    add_mu<CPLX, N>(a, m, s_mu + (size_t)cc * a.D, X1, XA, XB);
  }
  if (!EXPAND && m.active) store_lane_d<CPLX, N>(a, m, a.gagg + ((size_t)b * a.NG + g) * a.D, X1, XA, XB);
}

template <bool CPLX, int N, int MAXT>
__global__ __launch_bounds__(MAXT) void k_bwd_group_scan(DiagArgs a) {
  using TD = typename Types<CPLX>::TD;
  constexpr int CW = CPLX ? 2 : 1;
  __shared__ double s_red[MAXT * CW];
  const int b = blockIdx.x;
  const LaneMap m = lane_map(a, threadIdx.x);
  TD dummy{};
  const TD uj = load_ud(a.params, m.j, &dummy), uk = load_ud(a.params, m.k, &dummy);
  // Group g's operands (its span, the level-1 carries at its ends, its aggregate) are loaded one group ahead and
  // issued before the group's carry is stored: the memory counter is in order, so a load issued after a store could
  // not be waited for without waiting for the store as well.
  struct Pre {
    double tau;
    TD cek, csk, a1, aA, aB;
  };
  auto load = [&](int g, Pre& p) {
    const int c0 = g * a.scan_cb, c1 = min(c0 + a.scan_cb, a.C);
    const int t0 = c0 * a.T, t1 = min(c1 * a.T, a.n_int);
    p.tau = span_tau(a, b, t0, t1);
    const double* cs = a.carries + ((size_t)b * (a.C + 1) + c0) * a.D;
    const double* ce = a.carries + ((size_t)b * (a.C + 1) + c1) * a.D;
    p.cek = ldDD(ce + st1<CPLX>(m.k), &dummy);
    p.csk = ldDD(cs + st1<CPLX>(m.k), &dummy);
    const double* ag = a.gagg + ((size_t)b * a.NG + g) * a.D;
    p.a1 = m.plane ? ldDD(ag + st1<CPLX>(m.j), &dummy) : TD{};
    p.aA = TD{};
    p.aB = TD{};
    if (N == 2 && m.active) {
      const double* p2 = ag + st2<CPLX>(a, m.j, m.k);
      if (CPLX) {
        p.aA = ldDD(p2, &dummy);
        p.aB = ldDD(p2 + 2, &dummy);
      } else {
        p.aB = ldDD(p2, &dummy);
      }
    }
  };
  TD X1{}, XA{}, XB{};
  Pre cur{}, nxt{};
  if (a.NG > 0) load(a.NG - 1, cur);
  for (int g = a.NG - 1; g >= 0; --g) {
    if (g > 0) load(g - 1, nxt);
    if (m.active) store_lane_d<CPLX, N>(a, m, a.gcar + ((size_t)b * a.NG + g) * a.D, X1, XA, XB);
    const TD Fj = dexp(mul_s(uj, cur.tau)), Fk = dexp(mul_s(uk, cur.tau));
    const TD l1k = cur.cek - Fk * cur.csk;
    adj_lane<CPLX, N>(a, m, X1, XA, XB, Fj, Fk, l1k, s_red);
    if (m.plane) X1 = X1 + cur.a1;
    if (N == 2 && m.active) {
      if (CPLX) XA = XA + cur.aA;
      XB = XB + cur.aB;
    }
    cur = nxt;
  }
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

// ------------------------------------------------------------------------------------------- backward helpers
// Lane maps of the backward kernels. WAVE: one wavefront with lane = 8 j + k (K <= 8): row sums over k and
// column sums over j are butterflies inside the wave, and the diagonal lane (j, j) owns plane j. Otherwise
// lane = K j + k, the sums go through LDS, and lane (j, 0) owns plane j.
template <bool WAVE>
__device__ __forceinline__ LaneMap lane_map_b(const DiagArgs& a, int tid) {
  LaneMap m;
  const int S = WAVE ? 8 : a.K;
  int j, k;
  bool act;
  if (a.N == 2) {
    j = tid / S;
    k = tid % S;
    act = j < a.K && k < a.K;
  } else {
    j = tid;
    k = 0;
    act = tid < a.K;
  }
  m.active = act;
  m.j = act ? j : 0;
  m.k = act ? k : 0;
  m.plane = act && ((WAVE && a.N == 2) ? (j == k) : (k == 0));
  return m;
}

template <int I, class F> __device__ __forceinline__ void static_for_rev(F&& f) {
  if constexpr (I > 0) {
    f(std::integral_constant<int, I - 1>{});
    static_for_rev<I - 1>(f);
  }
}
template <int I, int N, class F> __device__ __forceinline__ void static_for(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for<I + 1, N>(f);
  }
}

// Cotangents of the lane's state from one cotangent row (complex convention gamma = dL/dRe + i dL/dIm).
// Level 2 (complex): the row layout's block (j, k) is q00 = (ReSA + ReSB)/2, q01 = (ImSB - ImSA)/2,
// q10 = (ImSA + ImSB)/2, q11 = (ReSA - ReSB)/2. am (max readout): only elements whose argmax is tg count.
template <bool CPLX, int N, class T>
__device__ __forceinline__ void gamma_row(const DiagArgs& a, const LaneMap& m, const float* row, float scale,
                                          const int* am, int tg, T& g1, T& gA, T& gB) {
  auto G = [&](int e) -> float {
    if (am && am[e] != tg) return 0.0f;
    return row[e] * scale;
  };
  g1 = zero<T>();
  gA = zero<T>();
  gB = zero<T>();
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

// Cotangent rows of a prefix readout are staged in LDS eight steps at a time; the next block is loaded into
// registers while the current one is processed, so no global load sits on the sequential dependency chain.
constexpr int kBLK = 8;   // checkpoint block and cotangent staging rows of the exact-coefficient adjoint (the
                          // plan halves it for wide states, whose checkpoints would not fit the LDS)
constexpr int kGB = 4;    // cotangent staging rows of the inversion adjoint
constexpr int kGBL = 2;   // and of the chunk-local adjoint (two rows suit it, four the inversion adjoint)
// Asynchronous copy of n contiguous floats into LDS (global_load_lds: each lane's dword lands at the wave's
// LDS base + 4 * lane); completion is awaited with lds_dma_wait() before a barrier.
typedef __attribute__((address_space(3))) void lds_void_t;
__device__ __forceinline__ void lds_dma(float* dst, const float* src, int n) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = (blockDim.x + 63) >> 6;
  for (int base = w * 64; base < n; base += nw * 64) {
    const int idx = base + lane;
    if (idx < n) __builtin_amdgcn_global_load_lds((const void*)(src + idx), (lds_void_t*)(dst + base), 4, 0, 0);
  }
}
__device__ __forceinline__ void lds_dma_wait() { __builtin_amdgcn_s_waitcnt(0); }

struct GammaSrc {
  const float* rows;  // prefix: staged block rows (block x W); else the per-sample cotangent (W)
  const int* am;      // max readout: per-sample argmax (W)
  float scale;
  int kind;           // readout
};

template <bool CPLX, int N, class T>
__device__ __forceinline__ void gamma_step(const DiagArgs& a, const LaneMap& m, const GammaSrc& gs, int r, int tg,
                                           T& g1, T& gA, T& gB) {
  if (!m.active) {
    g1 = gA = gB = zero<T>();
    return;
  }
  if (gs.kind == EWS_READOUT_PREFIX) {
    gamma_row<CPLX, N>(a, m, gs.rows + r * a.W, 1.0f, nullptr, tg, g1, gA, gB);
  } else if (gs.kind == EWS_READOUT_TERMINAL) {
    if (tg == a.n_int - 1) {
      gamma_row<CPLX, N>(a, m, gs.rows, 1.0f, nullptr, tg, g1, gA, gB);
    } else {
      g1 = gA = gB = zero<T>();
    }
  } else if (gs.kind == EWS_READOUT_MEAN) {
    gamma_row<CPLX, N>(a, m, gs.rows, gs.scale, nullptr, tg, g1, gA, gB);
  } else {
    gamma_row<CPLX, N>(a, m, gs.rows, 1.0f, gs.am, tg, g1, gA, gB);
  }
}

// per-sample cotangent (terminal / mean / max readouts) into LDS
__device__ __forceinline__ void stage_vec(const DiagArgs& a, int b, float* s_gv, int* s_am) {
  for (int e = threadIdx.x; e < a.W; e += blockDim.x) {
    s_gv[e] = a.gout[(size_t)b * a.W + e];
    if (a.readout == EWS_READOUT_MAX) s_am[e] = a.argmax[(size_t)b * a.W + e];
  }
}

__device__ __forceinline__ float wave_sum(float v) {
  v = lanes::sum64(v);
  return v;
}
// sums over k (lanes 8j .. 8j+7) and over j (lanes k, k+8, ..), by DPP where the lanes share a row of 16
__device__ __forceinline__ float row_sum8(float v) { return lanes::sum8(v); }
__device__ __forceinline__ float col_sum8(float v) { return lanes::colsum8(v); }
// sum over each aligned group of n lanes (n a power of two up to 64)
__device__ __forceinline__ float group_sum(float v, int n) { return lanes::sum_n(v, n); }
__device__ __forceinline__ cf group_sum(cf v, int n) { return cf{lanes::sum_n(v.re, n), lanes::sum_n(v.im, n)}; }
__device__ __forceinline__ cf row_sum8(cf v) { return cf{row_sum8(v.re), row_sum8(v.im)}; }
__device__ __forceinline__ cf col_sum8(cf v) { return cf{col_sum8(v.re), col_sum8(v.im)}; }

__device__ __forceinline__ float redot(cf a, cf b) { return a.re * b.re + a.im * b.im; }  // Re(conj(a) b)
__device__ __forceinline__ float redot(float a, float b) { return a * b; }

// parameter gradient of a node h*u with complex cotangent G (already carrying the factor h):
// x-type u = -conj(z) = -(d - i w): (dd, dw) += (-Re G, Im G); z-type u = -z: (dd, dw) += (-Re G, -Im G)
__device__ __forceinline__ void node_to_par(cf G, bool ztype, float& dd, float& dw) {
  dd += -G.re;
  dw += ztype ? -G.im : G.im;
}
__device__ __forceinline__ void node_to_par(float G, bool, float& dd, float&) { dd += -G; }

// LDS layout shared by the host sizing and the kernels
struct BwdLds {
  int v, h, gb, gv, am, ck, hist, red, dh, g, total;  // offsets in floats
};
__host__ __device__ inline BwdLds bwd_lds_layout(int T, int d, int W, int NT, int NS, bool wave, bool full,
                                                int rows = kBLK) {
  BwdLds L;
  int o = 0;
  L.v = o; o += T * d;
  L.h = o; o += T;
  L.gb = o; o += 2 * rows * W;
  L.gv = o; o += W;
  L.am = o; o += W;
  L.ck = o; o += (full && NS) ? ((T + rows - 1) / rows) * NS * NT : 0;
  L.hist = o; o += (full && NS) ? rows * NS * NT : 0;
  L.red = o; o += wave ? 0 : 8 * NT;
  L.dh = o; o += full ? T * ((NT + 63) / 64) : 0;
  L.g = o; o += 4 * NT;
  L.total = o;
  return L;
}

// ------------------------------------------------------------------------------------------- B1
// Chunk-local adjoint with zero incoming cotangent: the cotangent mu(c) on the chunk's carry-in.
// Level 1 uses linearity: each lane carries its pair's share of the plane cotangent, summed at the end.
template <bool CPLX, int N, int MAXT, bool WAVE, bool FAST>
__global__ __launch_bounds__(MAXT) void k_chunk_bwd_local(DiagArgs a) {
  using T = typename Types<CPLX>::T;
  extern __shared__ float smem[];
  const int NT = blockDim.x;
  const BwdLds Lo = bwd_lds_layout(a.T, a.d, a.W, NT, 0, WAVE, false, kGBL);
  float* s_v = smem + Lo.v;
  float* s_h = smem + Lo.h;
  float* s_gb = smem + Lo.gb;
  float* s_gv = smem + Lo.gv;
  int* s_am = reinterpret_cast<int*>(smem + Lo.am);
  float* s_red = smem + Lo.g;
  const int c = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
  if (a.fast_ok && (a.cflag[b * a.C + c] & 1)) return;  // a pair-group kernel owns this chunk
  if (!a.fast_ok && ((a.cflag[b * a.C + c] & 1) != 0) != FAST) return;  // the forward's chunk class
  const int t0 = c * a.T;
  const int Tc = min(a.T, a.n_int - t0);
  const bool prefix = a.readout == EWS_READOUT_PREFIX;
  load_clock(a, b, t0, Tc, s_h);
  __syncthreads();
  const ChunkClock cc = chunk_clock<T>(a, b, Tc, s_h);
  if (cc.fast != FAST) return;  // the other instantiation owns this chunk
  load_chunk(a, b, t0, Tc, s_v, s_h);
  if (!prefix) stage_vec(a, b, s_gv, s_am);
  const int nblk = (Tc + kGBL - 1) / kGBL;
  if (prefix) lds_dma(s_gb, a.gout + ((size_t)b * a.n_int + t0 + (nblk - 1) * kGBL) * a.W,
                      (Tc - (nblk - 1) * kGBL) * a.W);
  lds_dma_wait();
  __syncthreads();
  const LaneMap m = lane_map_b<WAVE>(a, tid);
  T dummy{};
  const T uj = load_u(a.params, m.j, &dummy);
  const T uk = load_u(a.params, m.k, &dummy);
  Coef<T> c0;
  CoefD<T> q;
  if constexpr (FAST) eval_coef<T, CPLX, N, true>(a.sq1, a.sq2, cc.hbar, cc.href, cc.per_int, uj, uk, c0, q);
  T L1 = zero<T>(), LA = zero<T>(), LB = zero<T>();
  for (int blk = nblk - 1; blk >= 0; --blk) {
    const int buf = (nblk - 1 - blk) & 1;
    const bool more = prefix && blk > 0;
    if (more) lds_dma(s_gb + (buf ^ 1) * kGBL * a.W, a.gout + ((size_t)b * a.n_int + t0 + (blk - 1) * kGBL) * a.W,
                      kGBL * a.W);
    const GammaSrc gs{prefix ? s_gb + buf * kGBL * a.W : s_gv, s_am, 1.0f / (float)a.n_int, a.readout};
    if (m.active) {
#pragma unroll 1
      for (int s = kGBL - 1; s >= 0; --s) {
        const int t = blk * kGBL + s;
        if (t < Tc) {
          T g1, gA, gB;
          gamma_step<CPLX, N>(a, m, gs, s, t0 + t, g1, gA, gB);
          L1 += g1;
          LA += gA;
          LB += gB;
          const float h = s_h[t];
          Coef<T> co;
          if constexpr (FAST) {
            lin_coef<T, CPLX, N>(c0, q, h - cc.hbar, cc.per_int, co);
          } else {
            CoefD<T> qq;
            eval_coef<T, CPLX, N, false>(a.sq1, a.sq2, h, cc.href, cc.per_int, uj, uk, co, qq);
          }
          T toC = zero<T>();
          if constexpr (N == 2) {
            const T pk = lds_p<T>(s_v, t, a.d, m.k);
            const T s1k = co.phi_k * pk;
            toC = conjc(s1k) * LB;
            if constexpr (CPLX) toC += s1k * LA;
            LB = conjc(co.lamB) * LB;
            if constexpr (CPLX) LA = conjc(co.lamA) * LA;
          }
          L1 = conjc(co.rho) * (L1 + toC);
        }
      }
    }
    if (more) {
      lds_dma_wait();
      __syncthreads();
    }
  }
  float* mp = a.mu + ((size_t)b * a.C + c) * a.D;
  if constexpr (N == 2) {
    T s1 = zero<T>();
    if constexpr (WAVE) {
      s1 = row_sum8(L1);
    } else {
      if (m.active) stT(s_red + 2 * tid, L1);
      __syncthreads();
      if (m.plane) {
        for (int k = 0; k < a.K; ++k) s1 += ldT<CPLX, T>(s_red + 2 * (m.j * a.K + k));
      }
    }
    if (m.plane) stT(mp + st1<CPLX>(m.j), s1);
    if (m.active) {
      float* p2 = mp + st2<CPLX>(a, m.j, m.k);
      if constexpr (CPLX) {
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

// Running cotangents and parameter accumulators of a backward chunk lane.
template <class T> struct BwdAcc {
  T L1, LA, LB;                    // cotangents of the state (level 1 of plane j; the pair's SA, SB)
  T Gx, GyA, GyB, Gxp;             // node cotangents times h (per-interval coefficients)
  T Sflow, SflowA, SflowB;         // summed flow cotangents (cached flows)
};
struct RedLds {
  float *rC, *rP, *cS, *cP;        // LDS row/column sums (multi-wave workgroups)
};

// One reverse step of the adjoint at interval t (global interval tg): adds the readout cotangent, then the
// adjoint of the Chen step with the state S(t-1) = (H1, HA, HB), writes dv[tg] for the plane lanes and the
// step's dh partial to s_dh, and moves acc's cotangents from S(t) to S(t-1).
// DH: the clock gradient is requested; without it the step's dh terms are not formed.
template <bool CPLX, int N, bool WAVE, bool ALLRED, bool DH, class T>
__device__ __forceinline__ void bwd_step(const DiagArgs& a, const LaneMap& m, const GammaSrc& gs, int s, int t, int tg,
                                         float h, const float* s_v, bool per_int, const Coef<T>& co,
                                         const CoefD<T>& qq, BwdAcc<T>& acc, T H1, T HA, T HB, const RedLds& red,
                                         float* s_dh) {
  const int tid = threadIdx.x, NW = (blockDim.x + 63) / 64, wid = tid / 64, b = blockIdx.y;
  float* s_rC = red.rC;
  float* s_rP = red.rP;
  float* s_cS = red.cS;
  float* s_cP = red.cP;
        T g1, gA, gB;
        gamma_step<CPLX, N>(a, m, gs, s, tg, g1, gA, gB);
        acc.L1 += g1;
        acc.LA += gA;
        acc.LB += gB;
        const T pj = lds_p<T>(s_v, t, a.d, m.j);
        const T pk = (N == 2) ? lds_p<T>(s_v, t, a.d, m.k) : zero<T>();
        const T cj = co.rho * H1;
        float dhp = 0.0f;
        T toC = zero<T>(), toS = zero<T>(), toPj = zero<T>(), toPk = zero<T>();
        if constexpr (N == 2) {
          const T s1k = co.phi_k * pk;
          toC = conjc(s1k) * acc.LB;
          toS = conjc(cj) * acc.LB;
          const T gf = conjc(co.IB) * acc.LB;
          toPj = conjc(pk) * gf;
          toPk = conjc(pj) * gf;
          const T gIB = conjc(pj * pk) * acc.LB;
          const T gLB = conjc(HB) * acc.LB;
          acc.Gx += h * (gIB * conjc(qq.DxB));
          acc.GyB += h * (gIB * conjc(qq.DyB));
          if constexpr (DH) dhp += redot(gIB, qq.IB1);
          if (per_int) {
            acc.GyB += h * (gLB * conjc(co.lamB));
            if constexpr (DH) dhp += redot(gLB, qq.lamB1);
          } else {
            acc.SflowB += gLB;
          }
          if constexpr (CPLX) {
            toC += s1k * acc.LA;
            toS += conjc(acc.LA) * cj;
            const T ge = conjc(co.IA) * acc.LA;
            toPj += pk * ge;
            toPk += conjc(ge) * pj;
            const T gIA = conjc(pj * conjc(pk)) * acc.LA;
            const T gLA = conjc(HA) * acc.LA;
            acc.Gx += h * (gIA * conjc(qq.DxA));
            acc.GyA += h * (gIA * conjc(qq.DyA));
            if constexpr (DH) dhp += redot(gIA, qq.IA1);
            if (per_int) {
              acc.GyA += h * (gLA * conjc(co.lamA));
              if constexpr (DH) dhp += redot(gLA, qq.lamA1);
            } else {
              acc.SflowA += gLA;
            }
            acc.LA = conjc(co.lamA) * acc.LA;
          }
          acc.LB = conjc(co.lamB) * acc.LB;
        }
        T rowC = zero<T>(), rowP = zero<T>(), colS = zero<T>(), colP = zero<T>();
        if constexpr (N == 2) {
          if constexpr (WAVE) {
            rowC = row_sum8(toC);
            rowP = row_sum8(toPj);
            colS = col_sum8(toS);
            colP = col_sum8(toPk);
          } else if (ALLRED && a.K == 32) {
            // (1024-lane workgroups only: compiled there, so the narrower instantiations keep their registers)
            // every lane active (K K threads) and row j on the aligned lanes j K .. j K + K - 1 of one wavefront:
            // rows by an all-reduce over those lanes; columns transposed through LDS ((k, j) order) and then the
            // same all-reduce, so that lane j K + k holds the sum of column j (the plane lane's share)
            rowC = toC;
            rowP = toPj;
            stT(s_cS + 2 * (m.k * a.K + m.j), toS);
            stT(s_cP + 2 * (m.k * a.K + m.j), toPk);
            rowC = group_sum(rowC, a.K);
            rowP = group_sum(rowP, a.K);
            __syncthreads();
            colS = ldT<CPLX, T>(s_cS + 2 * tid);
            colP = ldT<CPLX, T>(s_cP + 2 * tid);
            colS = group_sum(colS, a.K);
            colP = group_sum(colP, a.K);
          } else {
            if (m.active) {
              stT(s_rC + 2 * tid, toC);
              stT(s_rP + 2 * tid, toPj);
              // column arrays are indexed by (k, j) so a plane lane reads a contiguous run
              const int ct = m.k * a.K + m.j;
              stT(s_cS + 2 * ct, toS);
              stT(s_cP + 2 * ct, toPk);
            }
            __syncthreads();
            // the first R lanes of row j (lanes j K .. j K + R - 1: one wavefront, an aligned group as R divides K)
            // each sum every R-th entry of the plane's four runs, then combine by lane exchange; the plane lane
            // (k = 0) ends with the totals
            const int R = (a.K % 4 == 0) ? 4 : ((a.K % 2 == 0) ? 2 : 1);
            if (m.active && m.k < R) {
              for (int kk = m.k; kk < a.K; kk += R) {
                rowC += ldT<CPLX, T>(s_rC + 2 * (m.j * a.K + kk));
                rowP += ldT<CPLX, T>(s_rP + 2 * (m.j * a.K + kk));
                colS += ldT<CPLX, T>(s_cS + 2 * (m.j * a.K + kk));
                colP += ldT<CPLX, T>(s_cP + 2 * (m.j * a.K + kk));
              }
            }
            rowC = group_sum(rowC, R);
            rowP = group_sum(rowP, R);
            colS = group_sum(colS, R);
            colP = group_sum(colP, R);
          }
        }
        if (m.plane) {
          const T gc = acc.L1 + rowC;
          const T gs1 = acc.L1 + colS;
          const T gp = conjc(co.phi_j) * gs1 + rowP + colP;
          float* dvp = a.dv + ((size_t)b * a.n_int + tg) * a.d + st1<CPLX>(m.j);
          if constexpr (CPLX) {
            dvp[0] = gp.re;
            dvp[1] = gp.im;
          } else {
            dvp[0] = gp;
          }
          const T grho = conjc(H1) * gc;
          const T gphi = conjc(pj) * gs1;
          acc.Gxp += h * (gphi * conjc(qq.dphi_j));
          if constexpr (DH) dhp += redot(gphi, qq.phi_j1);
          if (per_int) {
            acc.Gxp += h * (grho * conjc(co.rho));
            if constexpr (DH) dhp += redot(grho, qq.rho1);
          } else {
            acc.Sflow += grho;
          }
          acc.L1 = conjc(co.rho) * gc;
        }
        if constexpr (DH) {
          const float ws = wave_sum(dhp);
          if ((tid & 63) == 0) s_dh[t * NW + wid] = ws;
        }
        if constexpr (!WAVE) __syncthreads();
}

// ------------------------------------------------------------------------------------------- B3
// Chunk epilogue of the full adjoint: dh of the chunk's intervals (fixed-order sum over waves) and the chunk's
// parameter partials (lane (j, k) contributes to plane j as a row and to plane k as a column).
template <bool CPLX, int N, bool WAVE, bool DH, class T>
__device__ __forceinline__ void bwd_epilogue(const DiagArgs& a, const LaneMap& m, const ChunkClock& cc, BwdAcc<T>& acc,
                                             T uj, T ua, T ub, int Tc, int t0, float* s_dh, float* s_g, int c, int b) {
  const int tid = threadIdx.x, NT = blockDim.x, NW = (NT + 63) / 64, wid = tid / 64;
  if constexpr (DH) {
    for (int t = tid; t < Tc; t += NT) {
      float s = 0.0f;
      for (int w = 0; w < NW; ++w) s += s_dh[t * NW + w];
      a.dh[(size_t)b * a.n_int + t0 + t] = s;
    }
  }
  float pj_d = 0.0f, pj_w = 0.0f, pk_d = 0.0f, pk_w = 0.0f, dhref = 0.0f;
  if (m.active) {
    if (!cc.per_int) {
      // cached flows: every step used the reference step href
      const float hr = cc.href;
      if constexpr (N == 2) {
        const T lamB = expv(hr * ub);
        acc.GyB += hr * (acc.SflowB * conjc(lamB));
        dhref += redot(acc.SflowB, lamB * ub);
        if constexpr (CPLX) {
          const T lamA = expv(hr * ua);
          acc.GyA += hr * (acc.SflowA * conjc(lamA));
          dhref += redot(acc.SflowA, lamA * ua);
        }
      }
      if (m.plane) {
        const T rho = expv(hr * uj);
        acc.Gxp += hr * (acc.Sflow * conjc(rho));
        dhref += redot(acc.Sflow, rho * uj);
      }
    }
    node_to_par(acc.Gx + acc.Gxp, false, pj_d, pj_w);
    node_to_par(acc.GyB, false, pj_d, pj_w);
    node_to_par(acc.GyB, false, pk_d, pk_w);
    if constexpr (CPLX) {
      node_to_par(acc.GyA, false, pj_d, pj_w);
      node_to_par(acc.GyA, true, pk_d, pk_w);
    }
  }
  float* gpo = a.gp + ((size_t)b * a.C + c) * a.npar;
  if constexpr (WAVE && N == 2) {
    const float sd = row_sum8(pj_d) + col_sum8(pk_d);
    const float sw = row_sum8(pj_w) + col_sum8(pk_w);
    if (m.plane) {
      if constexpr (CPLX) {
        gpo[2 * m.j] = sd;
        gpo[2 * m.j + 1] = sw;
      } else {
        gpo[m.j] = sd;
      }
    }
    if constexpr (DH) {
      const float whr = wave_sum(dhref);
      if (tid == 0) a.gph[(size_t)b * a.C + c] = whr;
    }
  } else {
    __syncthreads();
    s_g[4 * tid + 0] = pj_d;
    s_g[4 * tid + 1] = pj_w;
    s_g[4 * tid + 2] = pk_d;
    s_g[4 * tid + 3] = pk_w;
    if constexpr (DH) {
      const float whr = wave_sum(dhref);
      if ((tid & 63) == 0) s_dh[wid] = whr;  // the step partials were consumed above
    }
    __syncthreads();
    if (tid < a.K) {
      const int j = tid;
      float sd = 0.0f, sw = 0.0f;
      const int S = (WAVE && a.N == 2) ? 8 : a.K;
      const int rows = (a.N == 2) ? a.K : 1;
      for (int kk = 0; kk < rows; ++kk) {
        const int lr = (a.N == 2) ? j * S + kk : j;
        sd += s_g[4 * lr + 0];
        sw += s_g[4 * lr + 1];
        if (a.N == 2) {
          const int lc = kk * S + j;
          sd += s_g[4 * lc + 2];
          sw += s_g[4 * lc + 3];
        }
      }
      if constexpr (CPLX) {
        gpo[2 * j] = sd;
        gpo[2 * j + 1] = sw;
      } else {
        gpo[j] = sd;
      }
    }
    if (DH && tid == 0) {
      float s = 0.0f;
      for (int w = 0; w < NW; ++w) s += s_dh[w];
      a.gph[(size_t)b * a.C + c] = s;
    }
  }
}

// State loads of the lane from a float64 kernel-layout row / cotangent loads from a float32 row.
template <bool CPLX, int N, class T>
__device__ __forceinline__ void load_state_d(const DiagArgs& a, const LaneMap& m, const double* cr, T& S1, T& SA, T& SB) {
  S1 = SA = SB = zero<T>();
  if (!m.active) return;
  S1 = ldTd<CPLX, T>(cr + st1<CPLX>(m.j));
  if constexpr (N == 2) {
    const double* p2 = cr + st2<CPLX>(a, m.j, m.k);
    if constexpr (CPLX) {
      SA = ldTd<CPLX, T>(p2);
      SB = ldTd<CPLX, T>(p2 + 2);
    } else {
      SB = ldTd<CPLX, T>(p2);
    }
  }
}
template <bool CPLX, int N, class T>
__device__ __forceinline__ void load_cot(const DiagArgs& a, const LaneMap& m, const float* mp, BwdAcc<T>& acc) {
  acc = BwdAcc<T>{zero<T>(), zero<T>(), zero<T>(), zero<T>(), zero<T>(), zero<T>(), zero<T>(),
                  zero<T>(), zero<T>(), zero<T>()};
  if (m.plane) acc.L1 = ldT<CPLX, T>(mp + st1<CPLX>(m.j));
  if (N == 2 && m.active) {
    const float* p2 = mp + st2<CPLX>(a, m.j, m.k);
    if constexpr (CPLX) {
      acc.LA = ldT<CPLX, T>(p2);
      acc.LB = ldT<CPLX, T>(p2 + 2);
    } else {
      acc.LB = ldT<CPLX, T>(p2);
    }
  }
}

// Shared prologue: clock steps, ownership test, increments, per-sample cotangent, first staged block.
#define EWS_BWD_PROLOGUE(OWNS, ROWS)                                                                              \
  const int tid = threadIdx.x;                                                                             \
  if (a.fast_ok && (a.cflag[b * a.C + c] & 3) == 3) return; /* a pair-group kernel owns this chunk */      \
  if (!a.fast_ok) { /* the forward's chunk class: leave a chunk this kernel does not own before staging */ \
    const int gf = a.cflag[b * a.C + c];                                                                   \
    ChunkClock cc;                                                                                         \
    cc.fast = (gf & 1) != 0;                                                                               \
    cc.inv_ok = (gf & 2) != 0;                                                                             \
    if (!(OWNS)) return;                                                                                   \
  }                                                                                                        \
  const int t0 = c * a.T;                                                                                  \
  const int Tc = min(a.T, a.n_int - t0);                                                                   \
  const bool prefix = a.readout == EWS_READOUT_PREFIX;                                                     \
  load_clock(a, b, t0, Tc, s_h);                                                                           \
  __syncthreads();                                                                                         \
  ChunkClock cc = chunk_clock<T>(a, b, Tc, s_h);                                                           \
  if (a.fast_ok) cc.inv_ok = (a.cflag[b * a.C + c] & 2) != 0; /* one invertibility test for every kernel */ \
  if (!(OWNS)) return;                                                                                     \
  load_chunk(a, b, t0, Tc, s_v, s_h);                                                                      \
  if (!prefix) stage_vec(a, b, s_gv, s_am);                                                                \
  const int nblk = (Tc + (ROWS) - 1) / (ROWS);                                                             \
  if (prefix)                                                                                              \
    lds_dma(s_gb, a.gout + ((size_t)b * a.n_int + t0 + (nblk - 1) * (ROWS)) * a.W, (Tc - (nblk - 1) * (ROWS)) * a.W); \
  lds_dma_wait();                                                                                          \
  __syncthreads();                                                                                         \
  const LaneMap m = lane_map_b<WAVE>(a, tid);                                                              \
  T dummy{};                                                                                               \
  const T uj = load_u(a.params, m.j, &dummy);                                                              \
  const T uk = load_u(a.params, m.k, &dummy);                                                              \
  const T ua = uj + conjc(uk), ub = uj + uk;

// (a) Uniform-clock chunks whose decay allows it: the states S(t-1) come from inverting the steps backwards from
// the chunk's end state (c_j = S1(t) - s1_j(t) is exact; then divide by the flows), so nothing is recomputed
// forward and no history is kept.
template <bool CPLX, int N, int MAXT, bool WAVE, bool DH>
__global__ __launch_bounds__(MAXT) void k_chunk_bwd_inv(DiagArgs a) {
  using T = typename Types<CPLX>::T;
  extern __shared__ float smem[];
  const BwdLds Lo = bwd_lds_layout(a.T, a.d, a.W, blockDim.x, 0, WAVE, true, kGB);
  float* s_v = smem + Lo.v;
  float* s_h = smem + Lo.h;
  float* s_gb = smem + Lo.gb;
  float* s_gv = smem + Lo.gv;
  int* s_am = reinterpret_cast<int*>(smem + Lo.am);
  const RedLds red{smem + Lo.red, smem + Lo.red + 2 * blockDim.x, smem + Lo.red + 4 * blockDim.x,
                   smem + Lo.red + 6 * blockDim.x};
  float* s_dh = smem + Lo.dh;
  float* s_g = smem + Lo.g;
  const int c = blockIdx.x, b = blockIdx.y;
  EWS_BWD_PROLOGUE(cc.fast && cc.inv_ok, kGB)
  Coef<T> c0;
  CoefD<T> q0;
  eval_coef<T, CPLX, N, true>(a.sq1, a.sq2, cc.hbar, cc.href, cc.per_int, uj, uk, c0, q0);
  // d/dh of the inverse flows 1/rho = e^{-x}, 1/lambda = e^{-y} at hbar
  const T irho0 = expv(-(cc.per_int ? cc.hbar : cc.href) * uj);
  const T irho1 = cc.per_int ? -(irho0 * uj) : zero<T>();
  T ilB0 = zero<T>(), ilB1 = zero<T>(), ilA0 = zero<T>(), ilA1 = zero<T>();
  if constexpr (N == 2) {
    const float hf = cc.per_int ? cc.hbar : cc.href;
    ilB0 = expv(-hf * ub);
    ilB1 = cc.per_int ? -(ilB0 * ub) : zero<T>();
    if constexpr (CPLX) {
      ilA0 = expv(-hf * ua);
      ilA1 = cc.per_int ? -(ilA0 * ua) : zero<T>();
    }
  }
  T S1, SA, SB;
  load_state_d<CPLX, N>(a, m, a.carries + ((size_t)b * (a.C + 1) + c + 1) * a.D, S1, SA, SB);
  BwdAcc<T> acc;
  load_cot<CPLX, N>(a, m, a.mt + ((size_t)b * a.C + c) * a.D, acc);
  for (int blk = nblk - 1; blk >= 0; --blk) {
    const int buf = (nblk - 1 - blk) & 1;
    const bool more = prefix && blk > 0;
    if (more) lds_dma(s_gb + (buf ^ 1) * kGB * a.W, a.gout + ((size_t)b * a.n_int + t0 + (blk - 1) * kGB) * a.W,
                      kGB * a.W);
    const GammaSrc gs{prefix ? s_gb + buf * kGB * a.W : s_gv, s_am, 1.0f / (float)a.n_int, a.readout};
#pragma unroll 1
    for (int s = kGB - 1; s >= 0; --s) {
      const int t = blk * kGB + s;
      if (t < Tc) {
        const float dlt = s_h[t] - cc.hbar;
        Coef<T> co;
        lin_coef<T, CPLX, N>(c0, q0, dlt, cc.per_int, co);
        const T pj = lds_p<T>(s_v, t, a.d, m.j);
        const T pk = (N == 2) ? lds_p<T>(s_v, t, a.d, m.k) : zero<T>();
        // invert step t: S(t) -> S(t-1)
        const T cj = S1 - co.phi_j * pj;
        const T H1 = (irho0 + irho1 * dlt) * cj;
        T HA = zero<T>(), HB = zero<T>();
        if constexpr (N == 2) {
          const T s1k = co.phi_k * pk;
          HB = (ilB0 + ilB1 * dlt) * (SB - cj * s1k - co.IB * (pj * pk));
          if constexpr (CPLX) HA = (ilA0 + ilA1 * dlt) * (SA - cj * conjc(s1k) - co.IA * (pj * conjc(pk)));
        }
        bwd_step<CPLX, N, WAVE, MAXT == 1024, DH>(a, m, gs, s, t, t0 + t, s_h[t], s_v, cc.per_int, co, q0, acc, H1, HA,
                                                  HB, red,
                                s_dh);
        S1 = H1;
        SA = HA;
        SB = HB;
      }
    }
    if (more) lds_dma_wait();
    __syncthreads();
  }
  bwd_epilogue<CPLX, N, WAVE, DH>(a, m, cc, acc, uj, ua, ub, Tc, t0, s_dh, s_g, c, b);
}

// (b) Every other chunk: forward states recomputed from the chunk's float64 carry (checkpoints every kb steps; each
// block recomputed into a lane-private LDS history before its reverse sweep), with exact per-step coefficients, or
// the first-order model at the mean step for a uniform chunk.
// One chunk c of sample b; every early return is uniform over the workgroup.
template <bool CPLX, int N, int MAXT, bool WAVE, bool DH>
__device__ __forceinline__ void chunk_bwd_full(const DiagArgs& a, const int c, const int b) {
  using T = typename Types<CPLX>::T;
  constexpr int NS = CPLX ? 6 : 2;  // checkpoint floats per lane
  extern __shared__ float smem[];
  const int NT = blockDim.x;
  const int kb = a.kb;  // checkpoint block and cotangent staging rows
  const BwdLds Lo = bwd_lds_layout(a.T, a.d, a.W, NT, NS, WAVE, true, kb);
  float* s_v = smem + Lo.v;
  float* s_h = smem + Lo.h;
  float* s_gb = smem + Lo.gb;
  float* s_gv = smem + Lo.gv;
  int* s_am = reinterpret_cast<int*>(smem + Lo.am);
  float* s_ck = smem + Lo.ck;
  float* s_hist = smem + Lo.hist;
  const RedLds red{smem + Lo.red, smem + Lo.red + 2 * NT, smem + Lo.red + 4 * NT, smem + Lo.red + 6 * NT};
  float* s_dh = smem + Lo.dh;
  float* s_g = smem + Lo.g;
  EWS_BWD_PROLOGUE(!(cc.fast && cc.inv_ok), kb)
  // uniform chunks (too contractive to invert) take the first-order model at the mean step, as every other
  // kernel does for them; the others evaluate each step's exact coefficients
  Coef<T> c0;
  CoefD<T> q0;
  if (cc.fast) eval_coef<T, CPLX, N, true>(a.sq1, a.sq2, cc.hbar, cc.href, cc.per_int, uj, uk, c0, q0);
  auto coef_at = [&](int t, Coef<T>& co, CoefD<T>& qq) {
    if (cc.fast) {
      lin_coef<T, CPLX, N>(c0, q0, s_h[t] - cc.hbar, cc.per_int, co);
      qq = q0;
    } else {
      eval_coef<T, CPLX, N, true>(a.sq1, a.sq2, s_h[t], cc.href, cc.per_int, uj, uk, co, qq);
    }
  };
  auto st_store = [&](float* p, T x1, T xa, T xb) {
    if constexpr (CPLX) {
      p[0 * NT + tid] = x1.re;
      p[1 * NT + tid] = x1.im;
      p[2 * NT + tid] = xa.re;
      p[3 * NT + tid] = xa.im;
      p[4 * NT + tid] = xb.re;
      p[5 * NT + tid] = xb.im;
    } else {
      p[0 * NT + tid] = x1;
      p[1 * NT + tid] = xb;
    }
  };
  auto st_load = [&](const float* p, T& x1, T& xa, T& xb) {
    if constexpr (CPLX) {
      x1 = cf{p[0 * NT + tid], p[1 * NT + tid]};
      xa = cf{p[2 * NT + tid], p[3 * NT + tid]};
      xb = cf{p[4 * NT + tid], p[5 * NT + tid]};
    } else {
      x1 = p[0 * NT + tid];
      xa = 0.0f;
      xb = p[1 * NT + tid];
    }
  };
  // forward pre-pass from the carry: checkpoints of the state before every kb-th step
  T S1, SA, SB;
  load_state_d<CPLX, N>(a, m, a.carries + ((size_t)b * (a.C + 1) + c) * a.D, S1, SA, SB);
  for (int t = 0; t < Tc; ++t) {
    if ((t % kb) == 0) st_store(s_ck + (size_t)(t / kb) * NS * NT, S1, SA, SB);
    Coef<T> co;
    CoefD<T> qq;
    coef_at(t, co, qq);
    const T pj = lds_p<T>(s_v, t, a.d, m.j);
    const T pk = (N == 2) ? lds_p<T>(s_v, t, a.d, m.k) : zero<T>();
    fwd_step<T, CPLX, N>(co, pj, pk, S1, SA, SB);
  }
  BwdAcc<T> acc;
  load_cot<CPLX, N>(a, m, a.mt + ((size_t)b * a.C + c) * a.D, acc);
  __syncthreads();
  for (int blk = nblk - 1; blk >= 0; --blk) {
    const int buf = (nblk - 1 - blk) & 1;
    const bool more = prefix && blk > 0;
    if (more) lds_dma(s_gb + (buf ^ 1) * kb * a.W, a.gout + ((size_t)b * a.n_int + t0 + (blk - 1) * kb) * a.W,
                      kb * a.W);
    const GammaSrc gs{prefix ? s_gb + buf * kb * a.W : s_gv, s_am, 1.0f / (float)a.n_int, a.readout};
    st_load(s_ck + (size_t)blk * NS * NT, S1, SA, SB);
#pragma unroll 1
    for (int s = 0; s < kb; ++s) {
      const int t = blk * kb + s;
      if (t >= Tc) break;
      st_store(s_hist + (size_t)s * NS * NT, S1, SA, SB);
      Coef<T> co;
      CoefD<T> qq;
      coef_at(t, co, qq);
      const T pj = lds_p<T>(s_v, t, a.d, m.j);
      const T pk = (N == 2) ? lds_p<T>(s_v, t, a.d, m.k) : zero<T>();
      fwd_step<T, CPLX, N>(co, pj, pk, S1, SA, SB);
    }
#pragma unroll 1
    for (int s = kb - 1; s >= 0; --s) {
      const int t = blk * kb + s;
      if (t < Tc) {
        T H1, HA, HB;
        st_load(s_hist + (size_t)s * NS * NT, H1, HA, HB);
        Coef<T> co;
        CoefD<T> qq;
        coef_at(t, co, qq);
        bwd_step<CPLX, N, WAVE, MAXT == 1024, DH>(a, m, gs, s, t, t0 + t, s_h[t], s_v, cc.per_int, co, qq, acc, H1, HA, HB,
                                              red, s_dh);
      }
    }
    if (more) lds_dma_wait();
    __syncthreads();
  }
  bwd_epilogue<CPLX, N, WAVE, DH>(a, m, cc, acc, uj, ua, ub, Tc, t0, s_dh, s_g, c, b);
}
// Chunks blockIdx.x, blockIdx.x + gridDim.x, ... of sample blockIdx.y: with the pair kernels active the grid is
// small (most chunks belong to them), otherwise one chunk per workgroup. The ownership flags of 64 candidate
// chunks are read at once (one lane each: the pair kernels' flags, or the generic chunk class written by the first
// summary pass) and only the chunks left to this kernel are visited.
template <bool CPLX, int N, int MAXT, bool WAVE, bool DH>
__global__ __launch_bounds__(MAXT) void k_chunk_bwd_full(DiagArgs a) {
  const int b = blockIdx.y, lane = threadIdx.x & 63;
  for (int base = blockIdx.x; base < a.C; base += 64 * gridDim.x) {
    const int cl = base + gridDim.x * lane;
    // a pair-group kernel (fast_ok) or the inversion adjoint (generic class: uniform and invertible) owns the others
    const bool need = cl < a.C && (a.cflag[b * a.C + cl] & 3) != 3;
    unsigned long long mask = __ballot(need);  // the same in every wavefront of the workgroup
    while (mask) {
      const int i = __ffsll((long long)mask) - 1;
      mask &= mask - 1;
      chunk_bwd_full<CPLX, N, MAXT, WAVE, DH>(a, base + gridDim.x * i, b);
      __syncthreads();
    }
  }
}

// ------------------------------------------------------------------------------------------- B0 (log rows)
// The cotangent of the log rows as a cotangent of the flat rows (level 1, then level 2 row-major, no level 0):
// with L2[a,b] = S2[a,b] - S1_a S1_b / 2 at the Lyndon words a < b,
//   dS2[a,b] = dL2[a,b] (a < b, else 0),  dS1_a = dL1_a - (sum_{b > a} dL2[a,b] S1_b + sum_{b < a} dL2[b,a] S1_b) / 2,
// S1 of every step read from the forward's copy (s1rows). One wavefront per row, four rows per workgroup.
__global__ __launch_bounds__(256) void k_log_cot(DiagArgs a, const float* __restrict__ glog) {
  const size_t rows = (size_t)a.B * a.n_int;
  const size_t r = (size_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= rows) return;
  const int l = threadIdx.x & 63, d = a.d;
  const float* gl = glog + r * a.Wlog;
  const float* x = a.s1rows + r * d;
  float* go = a.gcot + r * a.D;
  for (int e = l; e < d * d; e += 64) {
    const int i = e / d, j = e - i * d;
    go[d + e] = i < j ? gl[d + lyndon2(i, j, d)] : 0.0f;
  }
  for (int i = l; i < d; i += 64) {
    float acc = 0.0f;
    for (int j = 0; j < d; ++j) {
      if (j > i) acc += gl[d + lyndon2(i, j, d)] * x[j];
      else if (j < i) acc += gl[d + lyndon2(j, i, d)] * x[j];
    }
    go[i] = gl[i] - 0.5f * acc;
  }
}

// ------------------------------------------------------------------------------------------- B4
// Knot gradients from interval gradients: dX_t = dv_{t-1} - dv_t, dtheta_t = dh_{t-1} - dh_t (+ the shared flow
// step's gradient for cached flows). One workgroup per (chunk, sample): the chunk's first knot always, its interior
// knots unless a pair-group adjoint already wrote them (it leaves dv / dh of its first and last interval for the
// boundary knots); workgroup C handles the last knot L-1.
__global__ void k_knot_grads(DiagArgs a) {
  const int c = blockIdx.x, b = blockIdx.y;
  const int dp1 = a.d + 1;
  int k0, k1;  // knot range [k0, k1)
  if (c == a.C) {
    k0 = a.n_int;
    k1 = a.L;
  } else {
    k0 = c * a.T;
    const bool owned = a.fast_ok && (a.cflag[b * a.C + c] & 3) == 3;
    k1 = owned ? k0 + 1 : min(k0 + a.T, a.n_int);
  }
  const float* dvb = a.dv + (size_t)b * a.n_int * a.d;
  const float* dhb = a.dh + (size_t)b * a.n_int;
  for (int i = threadIdx.x; i < (k1 - k0) * dp1; i += blockDim.x) {
    const int t = k0 + i / dp1, ch = i % dp1;
    const size_t bt = (size_t)b * a.L + t;
    if (ch < a.d) {
      float g = 0.0f;
      if (t >= 1) g += dvb[(size_t)(t - 1) * a.d + ch];
      if (t < a.n_int) g -= dvb[(size_t)t * a.d + ch];
      a.dpath[bt * a.d + ch] = g;
    } else if (a.dclock) {  // null: the clock gradient is not requested
      float g = 0.0f;
      if (t >= 1) g += dhb[t - 1];
      if (t < a.n_int) g -= dhb[t];
      if (a.flow_mode != EWS_FLOW_PER_INTERVAL) {
        // shared flow step href = theta[r+1] - theta[r]
        const int r = (a.flow_mode == EWS_FLOW_CACHED) ? 0 : 1;
        if (t == r || t == r + 1) {
          double hs = 0.0;
          for (int cc = 0; cc < a.C; ++cc) hs += (double)a.gph[(size_t)b * a.C + cc];
          g += (t == r + 1) ? (float)hs : -(float)hs;
        }
      }
      a.dclock[bt] = g;
    }
  }
}

// Parameter gradients in two fixed-order stages (deterministic): kParamBlocks workgroups each sum a contiguous
// range of the (B C, npar) partials in float64 (thread (r, p) takes rows r, r + R, ...: coalesced), then one
// workgroup adds the block sums in order.
constexpr int kParamBlocks = 128;
__global__ __launch_bounds__(256) void k_param_partial(DiagArgs a) {
  __shared__ double red[256];
  const int np = a.npar, R = 256 / np;
  const int r = threadIdx.x / np, p = threadIdx.x % np;
  const int n = a.B * a.C, per = (n + kParamBlocks - 1) / kParamBlocks;
  const int r0 = blockIdx.x * per, r1 = min(n, r0 + per);
  double s = 0.0;
  if (r < R) {
    int bc = r0 + r;
    for (; bc + 3 * R < r1; bc += 4 * R) {
      const float g0 = a.gp[(size_t)bc * np + p], g1 = a.gp[(size_t)(bc + R) * np + p];
      const float g2 = a.gp[(size_t)(bc + 2 * R) * np + p], g3 = a.gp[(size_t)(bc + 3 * R) * np + p];
      s += ((double)g0 + (double)g1) + ((double)g2 + (double)g3);
    }
    for (; bc < r1; bc += R) s += (double)a.gp[(size_t)bc * np + p];
  }
  red[threadIdx.x] = s;
  __syncthreads();
  if (threadIdx.x < np) {
    double t = 0.0;
    for (int rr = 0; rr < R; ++rr) t += red[rr * np + threadIdx.x];
    a.gpart[(size_t)blockIdx.x * np + threadIdx.x] = t;
  }
}
__global__ __launch_bounds__(256) void k_param_grads(DiagArgs a) {
  __shared__ double red[256];
  const int np = a.npar, R = 256 / np;
  const int r = threadIdx.x / np, p = threadIdx.x % np;
  double s = 0.0;
  if (r < R) {
    double v[kParamBlocks / 16];
#pragma unroll
    for (int u = 0; u < kParamBlocks / 16; ++u) {  // loads issued together (R >= 16 for npar <= 16)
      const int w = r + u * R;
      v[u] = w < kParamBlocks ? a.gpart[(size_t)w * np + p] : 0.0;
    }
    for (int u = 0; u < kParamBlocks / 16; ++u) s += v[u];
    for (int w = r + (kParamBlocks / 16) * R; w < kParamBlocks; w += R) s += a.gpart[(size_t)w * np + p];
  }
  red[threadIdx.x] = s;
  __syncthreads();
  if (threadIdx.x < np) {
    double t = 0.0;
    for (int rr = 0; rr < R; ++rr) t += red[rr * np + threadIdx.x];
    a.dparams[threadIdx.x] = (float)t;
  }
}

}  // namespace ews

// ================================================================================================= C ABI
namespace {

using namespace ews;

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

struct Plan {
  int B, L, n_int, d, K, N, T, C, D, W, npar, kb, readout;
  bool cplx, wave, fast;
  bool seq;  // the per-sample sequential kernels (ews_seq.hip) run the whole call
  bool log;  // log-prefix rows from the chunk kernels (W: the backward's flat-row layout, no level 0)
  int Wlog;  // floats per log row
  int NT, NTb, scan_cb, NG;
  size_t lds_bwd_local, lds_bwd_full, lds_bwd_inv, lds_carry, lds_adjoint;
};

constexpr size_t kMaxLds = 160 * 1024;  // LDS per workgroup on gfx950
constexpr size_t kScanLds = 48 * 1024;
constexpr int kMaxSeriesQ = 40;  // series order of the series leaves (the dense path's bound)

size_t bwd_lds_bytes(const Plan& p, int T, bool full, int kb) {
  const int NS = p.cplx ? 6 : 2;
  return (size_t)bwd_lds_layout(T, p.d, p.W, p.NTb, NS, p.wave, full, kb).total * 4;
}

int make_plan(const ews_diag_desc* s, Plan& p) {
  if (!s) return EWS_ERR_NULL;
  if (s->structure != EWS_STRUCT_PLANES && s->structure != EWS_STRUCT_REAL_DIAG) return EWS_ERR_OPTION;
  if (s->flow_mode < 0 || s->flow_mode > 2) return EWS_ERR_OPTION;
  if (s->readout < 0 || s->readout > EWS_READOUT_LOGPREFIX) return EWS_ERR_OPTION;
  if (s->path_dtype != EWS_DTYPE_F32 && s->path_dtype != EWS_DTYPE_BF16) return EWS_ERR_OPTION;
  if (s->depth != 1 && s->depth != 2) return EWS_ERR_DEPTH;
  if (s->batch < 1 || s->length < 2 || s->dim < 1) return EWS_ERR_SHAPE;
  p.cplx = s->structure == EWS_STRUCT_PLANES;
  if (p.cplx && (s->dim % 2 != 0 || s->dim > 32)) return EWS_ERR_SHAPE;
  if (!p.cplx && s->dim > 32) return EWS_ERR_SHAPE;
  if ((s->flow_mode == EWS_FLOW_CACHED_BASEPOINT) && s->length < 3) return EWS_ERR_SHAPE;
  if (s->chunk < 0 && s->chunk != EWS_CHUNK_SEQUENTIAL) return EWS_ERR_SHAPE;
  if (s->leaf < EWS_DIAG_LEAF_CLOSED || s->leaf > EWS_DIAG_LEAF_SERIES) return EWS_ERR_OPTION;
  if (s->leaf != EWS_DIAG_LEAF_CLOSED && (s->series_q < 0 || s->series_q > kMaxSeriesQ)) return EWS_ERR_OPTION;
  if (s->leaf == EWS_DIAG_LEAF_SERIES && s->series_q < 1) return EWS_ERR_OPTION;
  if (s->leaf == EWS_DIAG_LEAF_BLOCK_SERIES && s->depth == 2 && s->series_q < 1) return EWS_ERR_OPTION;
  p.B = s->batch;
  p.readout = s->readout;
  p.L = s->length;
  p.n_int = p.L - 1;
  p.d = s->dim;
  p.K = p.cplx ? p.d / 2 : p.d;
  p.N = s->depth;
  p.D = p.d + (p.N == 2 ? p.d * p.d : 0);
  const bool logp = s->readout == EWS_READOUT_LOGPREFIX;
  if (logp && p.N != 2) return EWS_ERR_DEPTH;
  p.W = logp ? p.D : p.D + (s->level0 ? 1 : 0);
  p.Wlog = logp ? p.d + p.d * (p.d - 1) / 2 : 0;
  p.npar = p.cplx ? 2 * p.K : p.K;
  // the per-sample sequential kernels: asked for (chunk EWS_CHUNK_SEQUENTIAL), or chosen for many samples of
  // moderate length, where one workgroup per sample fills the chip (the same rule for flat and log rows: a few long
  // samples take the chunk kernels, whose output pass writes the log rows as well)
  const bool seq_form = !p.cplx && p.N == 2 && p.d <= kSeqMaxK && s->flow_mode == EWS_FLOW_PER_INTERVAL &&
                        (s->readout == EWS_READOUT_PREFIX || s->readout == EWS_READOUT_LOGPREFIX);
  const bool seq_asked = s->chunk == EWS_CHUNK_SEQUENTIAL;
  if (seq_asked && !seq_form) return EWS_ERR_OPTION;
  p.seq = seq_form && (seq_asked || (s->chunk == 0 && p.B >= 128 && p.L <= 1025));
  p.log = logp && !p.seq;
  if (p.seq) {
    if (s->readout == EWS_READOUT_LOGPREFIX) p.W = p.d + p.d * (p.d - 1) / 2;
    p.fast = false;
    p.wave = false;
    p.T = p.n_int;
    p.C = 1;
    p.kb = 1;
    p.NT = p.NTb = seq_threads(p.K);
    p.scan_cb = 1;
    p.NG = 1;
    p.lds_bwd_local = p.lds_bwd_full = p.lds_bwd_inv = p.lds_carry = p.lds_adjoint = 0;
    return EWS_OK;
  }
  const int P = (p.N == 2) ? p.K * p.K : p.K;
  p.NT = ((P + 63) / 64) * 64;
  p.wave = p.K <= 8;  // one wavefront with lane = 8 j + k in the backward chunk kernels
  p.NTb = p.wave ? 64 : p.NT;
  // chunk length and checkpoint block of the recomputing adjoint: the longest chunk (down to 16) whose LDS fits
  // with blocks of kBLK steps, then shorter blocks (wide states: d = 32 at depth 2), then shorter chunks
  int T = s->chunk, kb = kBLK;
  if (T > 256) T = 256;
  if (T == 0) {
    T = 64;
    while (T > 16 && bwd_lds_bytes(p, T, true, kb) > kMaxLds) T /= 2;
  }
  while (kb > 2 && bwd_lds_bytes(p, T, true, kb) > kMaxLds) kb /= 2;
  if (s->chunk == 0)
    while (T > 8 && bwd_lds_bytes(p, T, true, kb) > kMaxLds) T /= 2;
  p.T = T;
  p.kb = kb;
  // the pair-group kernels evaluate the exact closed forms only
  p.fast = pairs_eligible(s->structure, s->depth, s->dim, s->readout, s->flow_mode, T) &&
           s->leaf == EWS_DIAG_LEAF_CLOSED;
  p.C = (p.n_int + T - 1) / T;
  p.lds_bwd_local = (size_t)bwd_lds_layout(T, p.d, p.W, p.NTb, 0, p.wave, false, kGBL).total * 4;
  p.lds_bwd_full = bwd_lds_bytes(p, T, true, kb);
  p.lds_bwd_inv = (size_t)bwd_lds_layout(T, p.d, p.W, p.NTb, 0, p.wave, true, kGB).total * 4;
  if (p.lds_bwd_full > kMaxLds) return EWS_ERR_SHAPE;
  const int CW = p.cplx ? 2 : 1;
  int cb = (int)((kScanLds - (size_t)p.NT * CW * 8) / ((size_t)p.D * 4 + (size_t)p.K * CW * 16));
  p.scan_cb = cb < 1 ? 1 : (cb > 16 ? 16 : cb);
  p.NG = (p.C + p.scan_cb - 1) / p.scan_cb;
  p.lds_carry = (size_t)p.scan_cb * p.K * CW * 8 + (size_t)p.scan_cb * p.D * 4;
  p.lds_adjoint = (size_t)p.scan_cb * p.K * CW * 16 + (size_t)p.NT * CW * 8 + (size_t)p.scan_cb * p.D * 4;
  return EWS_OK;
}

struct WsLayout {
  size_t summ, mu, mt, red, red_idx, dv, dh, gp, gph, gpart, gagg, gcar, qagg, qflow, ql1, cflow, gcot;
  size_t lbflag, lbagg, total;
};
// the look-back forward's status words (and ticket), quad and group aggregates (groups of 8 quads)
void lb_layout(const Plan& p, WsLayout& w, size_t& off) {
  const size_t NQ = (p.C + 3) / 4, NG = (NQ + 7) / 8, items = (size_t)p.B * (NQ + NG);
  w.lbflag = off; off += p.fast ? align256((items + (size_t)p.B * 32) * 4) : 0;  // statuses, then the tickets
  w.lbagg = off; off += p.fast ? align256(items * (p.D + 2 * p.K) * 8) : 0;
}
WsLayout ws_layout(const Plan& p) {
  WsLayout w{};
  size_t off = 0;
  if (p.seq) {  // per-sample parameter partials of the sequential backward (in the gp slot)
    w.gp = 0;
    w.total = align256((size_t)p.B * p.K * 4);
    return w;
  }
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
  w.gpart = off; off += align256((size_t)kParamBlocks * p.npar * 8);
  w.gagg = off; off += align256((size_t)p.B * p.NG * p.D * 8);
  w.gcar = off; off += align256((size_t)p.B * p.NG * p.D * 8);
  const size_t NQ = (p.C + 3) / 4;
  w.qagg = off; off += p.fast ? align256((size_t)p.B * NQ * p.D * 4) : 0;
  w.qflow = off; off += p.fast ? align256((size_t)p.B * NQ * p.K * 16) : 0;
  w.ql1 = off; off += p.fast ? align256((size_t)p.B * NQ * p.K * 16) : 0;
  w.cflow = off; off += p.fast ? align256(BC * p.K * 16) : 0;
  w.gcot = off; off += p.log ? align256((size_t)p.B * p.n_int * p.D * 4) : 0;
  lb_layout(p, w, off);
  w.total = off;
  return w;
}
// The forward's buffers only (the allocation-free forward): chunk summaries, mean/max partials, group and quad
// carries; the backward's buffers are absent.
WsLayout ws_layout_fwd(const Plan& p) {
  WsLayout w{};
  size_t off = 0;
  if (p.seq) return w;  // the sequential forward needs no scratch
  const size_t BC = (size_t)p.B * p.C;
  const bool reduce = p.readout == EWS_READOUT_MEAN || p.readout == EWS_READOUT_MAX;
  w.summ = off; off += align256(BC * p.D * 4);
  w.red = off; off += reduce ? align256(BC * p.W * 4) : 0;
  w.red_idx = off; off += reduce ? align256(BC * p.W * 4) : 0;
  w.gagg = off; off += align256((size_t)p.B * p.NG * p.D * 8);
  w.gcar = off; off += align256((size_t)p.B * p.NG * p.D * 8);
  const size_t NQ = (p.C + 3) / 4;
  w.qagg = off; off += p.fast ? align256((size_t)p.B * NQ * p.D * 4) : 0;
  w.qflow = off; off += p.fast ? align256((size_t)p.B * NQ * p.K * 16) : 0;
  w.ql1 = off; off += p.fast ? align256((size_t)p.B * NQ * p.K * 16) : 0;
  w.cflow = off; off += p.fast ? align256(BC * p.K * 16) : 0;
  lb_layout(p, w, off);
  w.total = off;
  return w;
}
size_t resid_carries_bytes(const Plan& p) { return align256((size_t)p.B * (p.C + 1) * p.D * 8); }
size_t resid_argmax_bytes(const Plan& p) { return align256((size_t)p.B * p.W * 4); }
size_t resid_chunk_bytes(const Plan& p) { return align256((size_t)p.B * p.C * 4); }
size_t resid_s1rows_bytes(const Plan& p) { return p.log ? align256((size_t)p.B * p.n_int * p.d * 4) : 0; }
size_t resid_bytes(const Plan& p) {
  if (p.seq) return align256((size_t)p.B * seq_ckpt_floats(p.K, p.n_int) * 4);  // state checkpoints
  return resid_carries_bytes(p) + resid_argmax_bytes(p) + 2 * resid_chunk_bytes(p) + align256(kCoefTabFloats * 4) +
         resid_s1rows_bytes(p);
}

// fwd_only: the workspace has the forward's layout (ws_layout_fwd); the backward's pointers are null
DiagArgs make_args(const ews_diag_desc* s, const Plan& p, const void* path, const float* clock,
                   const float* params, void* residual, void* workspace, bool fwd_only = false) {
  DiagArgs a{};
  a.B = p.B; a.L = p.L; a.n_int = p.n_int; a.d = p.d; a.K = p.K; a.N = p.N;
  a.flow_mode = s->flow_mode; a.readout = s->readout; a.T = p.T; a.C = p.C; a.scan_cb = p.scan_cb; a.kb = p.kb;
  a.W = p.W; a.lvl0 = s->level0 ? 1 : 0; a.off1 = a.lvl0; a.off2 = a.lvl0 + p.d; a.D = p.D; a.npar = p.npar;
  a.path_bf16 = s->path_dtype == EWS_DTYPE_BF16;
  a.sq1 = s->leaf == EWS_DIAG_LEAF_SERIES ? s->series_q : 0;
  a.sq2 = s->leaf == EWS_DIAG_LEAF_CLOSED ? 0 : s->series_q;
  a.path = path; a.clock = clock; a.params = params;
  if (p.seq) {
    if (s->readout == EWS_READOUT_LOGPREFIX) {  // log rows: level 1, then the Lyndon coefficients of level 2
      a.lvl0 = 0; a.off1 = 0; a.off2 = p.d;
    }
    a.seqck = fwd_only ? nullptr : (float*)residual;  // the allocation-free forward keeps no checkpoints
    a.seqgp = fwd_only ? nullptr : (float*)workspace;
    return a;
  }
  char* r = (char*)residual;
  a.carries = (double*)r;
  a.argmax = (int*)(r + resid_carries_bytes(p));
  a.cflag = (int*)(r + resid_carries_bytes(p) + resid_argmax_bytes(p));
  a.chbar = (float*)(r + resid_carries_bytes(p) + resid_argmax_bytes(p) + resid_chunk_bytes(p));
  a.ctab = (float*)(r + resid_carries_bytes(p) + resid_argmax_bytes(p) + 2 * resid_chunk_bytes(p));
  a.fast_ok = p.fast ? 1 : 0;
  if (p.log) {  // log rows: written with pitch Wlog; the backward's cotangent has the flat layout without level 0
    a.log = 1;
    a.readout = EWS_READOUT_PREFIX;  // every kernel but the output pass sees a prefix-row call
    a.Wlog = p.Wlog;
    a.lvl0 = 0; a.off1 = 0; a.off2 = p.d;
    a.s1rows = (float*)(r + resid_carries_bytes(p) + resid_argmax_bytes(p) + 2 * resid_chunk_bytes(p) +
                        align256(kCoefTabFloats * 4));
  }
  const WsLayout w = fwd_only ? ws_layout_fwd(p) : ws_layout(p);
  char* ws = (char*)workspace;
  a.summ = (float*)(ws + w.summ);
  a.red = (float*)(ws + w.red); a.red_idx = (int*)(ws + w.red_idx);
  if (!fwd_only) {
    a.mu = (float*)(ws + w.mu); a.mt = (float*)(ws + w.mt);
    a.dv = (float*)(ws + w.dv); a.dh = (float*)(ws + w.dh);
    a.gp = (float*)(ws + w.gp); a.gph = (float*)(ws + w.gph); a.gpart = (double*)(ws + w.gpart);
  }
  a.gagg = (double*)(ws + w.gagg); a.gcar = (double*)(ws + w.gcar); a.NG = p.NG;
  a.NQ = (p.C + 3) / 4;
  a.qagg = (float*)(ws + w.qagg); a.qflow = (double*)(ws + w.qflow); a.ql1 = (double*)(ws + w.ql1);
  a.cflow = (double*)(ws + w.cflow);
  a.lbflag = (int*)(ws + w.lbflag); a.lbagg = (double*)(ws + w.lbagg);
  if (p.log && !fwd_only) a.gcot = (float*)(ws + w.gcot);
  return a;
}

size_t fwd_lds(const Plan& p) { return (size_t)(p.T * p.d + p.T) * 4; }

#define EWS_LAUNCH_CHECK()                                  \
  do {                                                      \
    if (hipGetLastError() != hipSuccess) return EWS_ERR_LAUNCH; \
  } while (0)

// Forward passes: 0 chunk summaries, 1 carry scan, 2 chunk outputs (prefix rows or mean/max partials),
// 3 mean/max reduction. A pass that does not apply to the readout launches nothing.
template <bool CPLX, int N, int MAXT>
int forward_pass(const ews_diag_desc* s, const Plan& p, DiagArgs a, hipStream_t st, int pass) {
  dim3 grid(p.C, p.B), blk(p.NT);
  switch (pass) {
    case 0:
      if (p.fast) {  // the pair-group forward: the coefficient table here, everything else in pass 2
        if (pairs_forward(a, st, false) != 0) return EWS_ERR_LAUNCH;
        return EWS_OK;
      }
      hipLaunchKernelGGL((k_chunk_fwd<CPLX, N, MODE_SUMMARY, MAXT, true>), grid, blk, fwd_lds(p), st, a);
      EWS_LAUNCH_CHECK();
      hipLaunchKernelGGL((k_chunk_fwd<CPLX, N, MODE_SUMMARY, MAXT, false>), grid, blk, fwd_lds(p), st, a);
      break;
    case 1:
      if (p.fast) return EWS_OK;
      if (p.NG > 1) {  // one group: its carry is the zero state, no group aggregates or group scan
        hipLaunchKernelGGL((k_fwd_group<CPLX, N, MAXT, false>), dim3(p.NG, p.B), blk, p.lds_carry, st, a);
        EWS_LAUNCH_CHECK();
        hipLaunchKernelGGL((k_fwd_group_scan<CPLX, N, MAXT>), dim3(p.B), blk, 0, st, a);
        EWS_LAUNCH_CHECK();
      }
      hipLaunchKernelGGL((k_fwd_group<CPLX, N, MAXT, true>), dim3(p.NG, p.B), blk, p.lds_carry, st, a);
      break;
    case 2:
      if (s->readout == EWS_READOUT_PREFIX || s->readout == EWS_READOUT_LOGPREFIX) {
        if (p.fast) {  // the look-back forward: every chunk (uniform or not), carries and rows in one launch
          if (pairs_forward(a, st, true) != 0) return EWS_ERR_LAUNCH;
          return EWS_OK;
        }
        hipLaunchKernelGGL((k_chunk_fwd<CPLX, N, MODE_PREFIX, MAXT, true>), grid, blk, fwd_lds(p), st, a);
        EWS_LAUNCH_CHECK();
        hipLaunchKernelGGL((k_chunk_fwd<CPLX, N, MODE_PREFIX, MAXT, false>), grid, blk, fwd_lds(p), st, a);
      } else if (s->readout == EWS_READOUT_MEAN || s->readout == EWS_READOUT_MAX) {
        hipLaunchKernelGGL((k_chunk_fwd<CPLX, N, MODE_REDUCE, MAXT, true>), grid, blk, fwd_lds(p), st, a);
        EWS_LAUNCH_CHECK();
        hipLaunchKernelGGL((k_chunk_fwd<CPLX, N, MODE_REDUCE, MAXT, false>), grid, blk, fwd_lds(p), st, a);
      } else {
        return EWS_OK;
      }
      break;
    case 3:
      if (s->readout == EWS_READOUT_MEAN || s->readout == EWS_READOUT_MAX) {
        hipLaunchKernelGGL(k_reduce_readout, dim3(p.B), dim3(256), 0, st, a);
      } else {
        return EWS_OK;
      }
      break;
    default:
      return EWS_ERR_OPTION;
  }
  EWS_LAUNCH_CHECK();
  return EWS_OK;
}

template <class K>
int set_lds(K* kern, size_t lds) {
  if (lds > 65536 &&
      hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                          (int)lds) != hipSuccess)
    return EWS_ERR_LAUNCH;
  return EWS_OK;
}

// pass 2's generic kernels: the inverting full adjoint (FAST invertible chunks) and the recomputing one (the rest)
template <bool CPLX, int N, int MAXT, bool WAVE, bool DH>
int full_adjoints(const Plan& p, const DiagArgs& a, hipStream_t st) {
  dim3 grid(p.C, p.B), blkb(p.NTb);
  if (set_lds(&k_chunk_bwd_inv<CPLX, N, MAXT, WAVE, DH>, p.lds_bwd_inv) != EWS_OK) return EWS_ERR_LAUNCH;
  if (set_lds(&k_chunk_bwd_full<CPLX, N, MAXT, WAVE, DH>, p.lds_bwd_full) != EWS_OK) return EWS_ERR_LAUNCH;
  if (!p.fast) {  // k_chunk_bwd_inv owns only FAST chunks
    hipLaunchKernelGGL((k_chunk_bwd_inv<CPLX, N, MAXT, WAVE, DH>), grid, blkb, p.lds_bwd_inv, st, a);
    EWS_LAUNCH_CHECK();
  }
  // the recomputing adjoint's LDS leaves about one workgroup per CU, so up to eight chunks per workgroup (strided,
  // visited only when owned) cost no parallelism while 512 or more workgroups remain, and spare the launch most of
  // its exiting workgroups when the other kernels own the chunks
  const int gx = p.fast ? min(p.C, 8) : min(p.C, max((p.C + 7) / 8, (512 + p.B - 1) / p.B));
  hipLaunchKernelGGL((k_chunk_bwd_full<CPLX, N, MAXT, WAVE, DH>), dim3(gx, p.B), blkb, p.lds_bwd_full, st, a);
  EWS_LAUNCH_CHECK();
  return EWS_OK;
}

// Backward passes: 0 chunk-local adjoints, 1 reverse adjoint scan, 2 full chunk adjoints, 3 knot gradients,
// 4 parameter reduction.
template <bool CPLX, int N, int MAXT, bool WAVE>
int backward_pass(const Plan& p, DiagArgs a, hipStream_t st, int pass) {
  dim3 grid(p.C, p.B), blkb(p.NTb);
  switch (pass) {
    case 0:
      if (p.fast && pairs_backward(a, st, false) != 0) return EWS_ERR_LAUNCH;
      if (set_lds(&k_chunk_bwd_local<CPLX, N, MAXT, WAVE, true>, p.lds_bwd_local) != EWS_OK) return EWS_ERR_LAUNCH;
      if (set_lds(&k_chunk_bwd_local<CPLX, N, MAXT, WAVE, false>, p.lds_bwd_local) != EWS_OK) return EWS_ERR_LAUNCH;
      if (!p.fast) {  // with the pair kernels active no chunk is left to the FAST instantiation
        hipLaunchKernelGGL((k_chunk_bwd_local<CPLX, N, MAXT, WAVE, true>), grid, blkb, p.lds_bwd_local, st, a);
        EWS_LAUNCH_CHECK();
      }
      hipLaunchKernelGGL((k_chunk_bwd_local<CPLX, N, MAXT, WAVE, false>), grid, blkb, p.lds_bwd_local, st, a);
      break;
    case 1:
      if (p.fast) {
        if (pairs_carry_scan(a, st) != 0) return EWS_ERR_LAUNCH;
        break;
      }
      if (p.NG > 1) {  // one group: its end cotangent is zero, no group aggregates or group scan
        hipLaunchKernelGGL((k_bwd_group<CPLX, N, (MAXT < 256 ? 256 : MAXT), false>), dim3(p.NG, p.B), dim3(p.NT),
                           p.lds_adjoint, st, a);
        EWS_LAUNCH_CHECK();
        hipLaunchKernelGGL((k_bwd_group_scan<CPLX, N, (MAXT < 256 ? 256 : MAXT)>), dim3(p.B), dim3(p.NT), 0, st, a);
        EWS_LAUNCH_CHECK();
      }
      hipLaunchKernelGGL((k_bwd_group<CPLX, N, (MAXT < 256 ? 256 : MAXT), true>), dim3(p.NG, p.B), dim3(p.NT),
                         p.lds_adjoint, st, a);
      break;
    case 2:
      if (p.fast && pairs_backward(a, st, true) != 0) return EWS_ERR_LAUNCH;
      // the clock gradient's dh terms only when it is requested (grad_clock non-null)
      if (a.dclock) return full_adjoints<CPLX, N, MAXT, WAVE, true>(p, a, st);
      return full_adjoints<CPLX, N, MAXT, WAVE, false>(p, a, st);
    case 3:
      hipLaunchKernelGGL(k_knot_grads, dim3(p.C + 1, p.B), dim3(64), 0, st, a);
      break;
    case 4:
      hipLaunchKernelGGL(k_param_partial, dim3(kParamBlocks), dim3(256), 0, st, a);
      EWS_LAUNCH_CHECK();
      hipLaunchKernelGGL(k_param_grads, dim3(1), dim3(256), 0, st, a);
      break;
    default:
      return EWS_ERR_OPTION;
  }
  EWS_LAUNCH_CHECK();
  return EWS_OK;
}

int dispatch_forward(const ews_diag_desc* s, const Plan& p, const DiagArgs& a, hipStream_t st, int pass) {
  if (p.seq) {  // one pass: the whole forward (the other pass numbers launch nothing)
    if (pass < 0 || pass >= 4) return EWS_ERR_OPTION;
    if (pass == 0 && seq_forward(a, st) != 0) return EWS_ERR_LAUNCH;
    return EWS_OK;
  }
  const bool big = p.NT > 256;
  if (p.cplx) {
    if (p.N == 2) return big ? forward_pass<true, 2, 1024>(s, p, a, st, pass) : forward_pass<true, 2, 256>(s, p, a, st, pass);
    return forward_pass<true, 1, 256>(s, p, a, st, pass);
  }
  if (p.N == 2) return big ? forward_pass<false, 2, 1024>(s, p, a, st, pass) : forward_pass<false, 2, 256>(s, p, a, st, pass);
  return forward_pass<false, 1, 256>(s, p, a, st, pass);
}

int dispatch_backward(const Plan& p, const DiagArgs& a, hipStream_t st, int pass) {
  if (p.seq) {  // one pass: the whole backward and the parameter reduction
    if (pass < 0 || pass >= 5) return EWS_ERR_OPTION;
    if (pass == 0 && seq_backward(a, st) != 0) return EWS_ERR_LAUNCH;
    return EWS_OK;
  }
  const bool big = p.NT > 256;
  if (p.cplx) {
    if (p.N == 2) {
      if (p.wave) return backward_pass<true, 2, 64, true>(p, a, st, pass);
      return big ? backward_pass<true, 2, 1024, false>(p, a, st, pass) : backward_pass<true, 2, 256, false>(p, a, st, pass);
    }
    return p.wave ? backward_pass<true, 1, 64, true>(p, a, st, pass) : backward_pass<true, 1, 256, false>(p, a, st, pass);
  }
  if (p.N == 2) {
    if (p.wave) return backward_pass<false, 2, 64, true>(p, a, st, pass);
    return big ? backward_pass<false, 2, 1024, false>(p, a, st, pass) : backward_pass<false, 2, 256, false>(p, a, st, pass);
  }
  return p.wave ? backward_pass<false, 1, 64, true>(p, a, st, pass) : backward_pass<false, 1, 256, false>(p, a, st, pass);
}

constexpr int kForwardPasses = 4;
constexpr int kBackwardPasses = 5;

// ------------------------------------------------------------------------------------------- scan + mixer epilogue
// the leading zero row of a sample's levels maps to c_down's bias alone
__global__ void k_mix_bias_rows_fused(MixEpi e, int n_int) {
  for (int col = threadIdx.x; col < e.H; col += blockDim.x)
    e.out[(size_t)blockIdx.x * (n_int + 1) * e.H + col] = e.bias[col];
}

template <bool CPLX, int N, int MAXT, int NH>
int mix_launch(const Plan& p, const DiagArgs& a, const MixEpi& e, hipStream_t st) {
  const size_t lds = mix_lds_floats(p.T, p.d, p.D, p.NT, N, e.H) * 4;
  for (auto fn : {&k_chunk_mix<CPLX, N, MAXT, true, NH>, &k_chunk_mix<CPLX, N, MAXT, false, NH>}) {
    if (lds > 65536 && hipFuncSetAttribute(reinterpret_cast<const void*>(fn),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess)
      return EWS_ERR_LAUNCH;
  }
  const dim3 grid(p.C, p.B), blk(p.NT);
  hipLaunchKernelGGL((k_chunk_mix<CPLX, N, MAXT, true, NH>), grid, blk, lds, st, a, e);
  EWS_LAUNCH_CHECK();
  hipLaunchKernelGGL((k_chunk_mix<CPLX, N, MAXT, false, NH>), grid, blk, lds, st, a, e);
  EWS_LAUNCH_CHECK();
  return EWS_OK;
}

template <bool CPLX, int N, int MAXT>
int mix_pass(const Plan& p, const DiagArgs& a, const MixEpi& e, hipStream_t st) {
  // hidden tiles of 16: two when c_down is at most 32 wide, else four
  const int rc = e.H <= 32 ? mix_launch<CPLX, N, MAXT, 2>(p, a, e, st) : mix_launch<CPLX, N, MAXT, 4>(p, a, e, st);
  if (rc != EWS_OK) return rc;
  if (e.prepend) {
    hipLaunchKernelGGL(k_mix_bias_rows_fused, dim3(p.B), dim3(64), 0, st, e, p.n_int);
    EWS_LAUNCH_CHECK();
  }
  return EWS_OK;
}

// ------------------------------------------------------------------------------------------- allocation-free forward
// Scratch of ews_diag_forward_noalloc: the forward's residual and workspace in one file-scope device array, of which
// every GPU the library runs on holds its own copy until the process ends. On the host, `scratch` names a host-side
// stand-in, not device memory: host code uses only the per-device address hipGetSymbolAddress returns.
constexpr size_t kNoAllocScratchBytes = size_t(64) << 20;
__device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// the scratch address on the current device, looked up once per device with that device current
int scratch_on_current_device(void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return EWS_ERR_LAUNCH;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || !ptr) return EWS_ERR_LAUNCH;
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
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
  return resid_bytes(p);
}

int ews_diag_forward_pass(const ews_diag_desc* desc, int pass, const void* path, const float* clock,
                          const float* params, float* out, void* residual, void* workspace, ews_stream_t stream) {
  Plan p;
  const int rc = make_plan(desc, p);
  if (rc != EWS_OK) return rc;
  if (!path || !clock || !params || !out || !residual || !workspace) return EWS_ERR_NULL;
  if (pass < 0 || pass >= kForwardPasses) return EWS_ERR_OPTION;
  DiagArgs a = make_args(desc, p, path, clock, params, residual, workspace);
  a.out = out;
  return dispatch_forward(desc, p, a, (hipStream_t)stream, pass);
}

int ews_diag_forward(const ews_diag_desc* desc, const void* path, const float* clock, const float* params,
                     float* out, void* residual, void* workspace, ews_stream_t stream) {
  for (int pass = 0; pass < kForwardPasses; ++pass) {
    const int rc = ews_diag_forward_pass(desc, pass, path, clock, params, out, residual, workspace, stream);
    if (rc != EWS_OK) return rc;
  }
  return EWS_OK;
}

int ews_diag_backward_pass(const ews_diag_desc* desc, int pass, const void* path, const float* clock,
                           const float* params, const void* residual, const float* grad_out, float* grad_path,
                           float* grad_clock, float* grad_params, void* workspace, ews_stream_t stream) {
  Plan p;
  const int rc = make_plan(desc, p);
  if (rc != EWS_OK) return rc;
  if (!path || !clock || !params || !residual || !grad_out || !grad_path || !grad_params || !workspace)
    return EWS_ERR_NULL;  // grad_clock may be null: the clock gradient is then not computed
  if (pass < 0 || pass >= kBackwardPasses) return EWS_ERR_OPTION;
  DiagArgs a = make_args(desc, p, path, clock, params, (void*)residual, workspace);
  a.gout = grad_out;
  a.dpath = grad_path;
  a.dclock = grad_clock;
  a.dparams = grad_params;
  if (p.log) {  // the passes run on the flat-row cotangent, built from the log cotangent before pass 0
    if (pass == 0) {
      const size_t rows = (size_t)p.B * p.n_int;
      hipLaunchKernelGGL(k_log_cot, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, (hipStream_t)stream, a,
                         grad_out);
      if (hipGetLastError() != hipSuccess) return EWS_ERR_LAUNCH;
    }
    a.gout = a.gcot;
  }
  return dispatch_backward(p, a, (hipStream_t)stream, pass);
}

int ews_diag_backward(const ews_diag_desc* desc, const void* path, const float* clock, const float* params,
                      const void* residual, const float* grad_out, float* grad_path, float* grad_clock,
                      float* grad_params, void* workspace, ews_stream_t stream) {
  for (int pass = 0; pass < kBackwardPasses; ++pass) {
    const int rc = ews_diag_backward_pass(desc, pass, path, clock, params, residual, grad_out, grad_path,
                                          grad_clock, grad_params, workspace, stream);
    if (rc != EWS_OK) return rc;
  }
  return EWS_OK;
}

int ews_diag_num_passes(int direction) { return direction == 0 ? kForwardPasses : kBackwardPasses; }

int ews_diag_uses_chunk_kernels(const ews_diag_desc* desc) {
  Plan p;
  if (make_plan(desc, p) != EWS_OK) return 0;
  return (!p.fast && !p.seq && !p.log) ? 1 : 0;
}

int ews_diag_mixer_forward(const ews_diag_desc* desc, const ews_mixer_desc* mdesc, const void* path,
                           const float* clock, const float* params, const float* weight, const float* bias,
                           const float* gains, float* out, void* mixer_residual, void* residual, void* workspace,
                           ews_stream_t stream) {
  Plan p;
  const int rc = make_plan(desc, p);
  if (rc != EWS_OK) return rc;
  if (!mdesc) return EWS_ERR_NULL;
  if (!path || !clock || !params || !weight || !bias || !gains || !out || !mixer_residual || !residual || !workspace)
    return EWS_ERR_NULL;
  // the chunk kernels' prefix rows only (the pair-group and per-sample kernels write their rows themselves)
  if (p.fast || p.seq || p.log || desc->readout != EWS_READOUT_PREFIX) return EWS_ERR_OPTION;
  if (mdesc->batch != p.B || mdesc->rows != p.n_int || mdesc->dim != p.d || mdesc->depth != p.N) return EWS_ERR_SHAPE;
  if (mdesc->hidden < 1 || mdesc->hidden > 16 * kMixHT || mdesc->variant < 0 || mdesc->variant > 2)
    return EWS_ERR_OPTION;
  if (mix_lds_floats(p.T, p.d, p.D, p.NT, p.N, mdesc->hidden) * 4 > kMaxLds) return EWS_ERR_SHAPE;
  DiagArgs a = make_args(desc, p, path, clock, params, residual, workspace);
  hipStream_t st = (hipStream_t)stream;
  for (int pass = 0; pass < 2; ++pass) {  // chunk summaries and the float64 carries
    const int r = dispatch_forward(desc, p, a, st, pass);
    if (r != EWS_OK) return r;
  }
  MixEpi e{};
  e.weight = weight;
  e.bias = bias;
  e.gains = gains;
  e.out = out;
  const size_t M = (size_t)p.B * p.n_int;
  e.P = (float*)mixer_residual;  // the layout of ews_mixer_residual_bytes: products, then factors
  e.F = (float*)((char*)mixer_residual + align256(M * p.N * mdesc->hidden * 4));
  e.H = mdesc->hidden;
  e.variant = mdesc->variant;
  e.prepend = mdesc->prepend ? 1 : 0;
  e.prescale = mdesc->prescale ? 1 : 0;
  e.eps[0] = mdesc->eps[0];
  e.eps[1] = mdesc->eps[1];
  const bool big = p.NT > 256;
  if (p.cplx) {
    if (p.N == 2) return big ? mix_pass<true, 2, 1024>(p, a, e, st) : mix_pass<true, 2, 256>(p, a, e, st);
    return mix_pass<true, 1, 256>(p, a, e, st);
  }
  if (p.N == 2) return big ? mix_pass<false, 2, 1024>(p, a, e, st) : mix_pass<false, 2, 256>(p, a, e, st);
  return mix_pass<false, 1, 256>(p, a, e, st);
}

int ews_diag_forward_status(const ews_diag_desc* desc, const void* residual, int* status, ews_stream_t stream) {
  Plan p;
  const int rc = make_plan(desc, p);
  if (rc != EWS_OK) return rc;
  if (!residual || !status) return EWS_ERR_NULL;
  *status = 0;
  if (!p.fast) return EWS_OK;  // only the look-back forward waits on other workgroups
  const char* ctab = (const char*)residual + resid_carries_bytes(p) + resid_argmax_bytes(p) + 2 * resid_chunk_bytes(p);
  if (hipMemcpyAsync(status, ctab + kCtabStatus * sizeof(int), sizeof(int), hipMemcpyDeviceToHost,
                     (hipStream_t)stream) != hipSuccess)
    return EWS_ERR_LAUNCH;
  return hipStreamSynchronize((hipStream_t)stream) == hipSuccess ? EWS_OK : EWS_ERR_LAUNCH;
}

int ews_diag_forward_noalloc(const ews_diag_desc* desc, const void* path, const float* clock, const float* params,
                             float* out, ews_stream_t stream) {
  Plan p;
  int rc = make_plan(desc, p);
  if (rc != EWS_OK) return rc;
  if (!path || !clock || !params || !out) return EWS_ERR_NULL;
  const size_t rb = p.seq ? 0 : resid_bytes(p);  // the sequential forward keeps no checkpoints here
  if (rb + ws_layout_fwd(p).total > kNoAllocScratchBytes) return EWS_ERR_SCRATCH;
  void* base = nullptr;
  rc = scratch_on_current_device(&base);
  if (rc != EWS_OK) return rc;
  // no pass reads scratch it has not written in the same call (no zeroed state is assumed), so the contents a
  // previous call left behind are harmless
  DiagArgs a = make_args(desc, p, path, clock, params, base, (char*)base + rb, true);
  a.out = out;
  for (int pass = 0; pass < kForwardPasses; ++pass) {
    rc = dispatch_forward(desc, p, a, (hipStream_t)stream, pass);
    if (rc != EWS_OK) return rc;
  }
  return EWS_OK;
}

const char* ews_error_string(int code) {
  switch (code) {
    case EWS_OK: return "ok";
    case EWS_ERR_NULL: return "a required pointer is NULL";
    case EWS_ERR_SHAPE: return "batch/length/dim out of range for this structure";
    case EWS_ERR_DEPTH: return "depth not supported by this structure";
    case EWS_ERR_OPTION: return "unknown structure, flow mode, readout or dtype";
    case EWS_ERR_LAUNCH: return "kernel launch failed";
    case EWS_ERR_SCRATCH: return "the call needs more scratch than the allocation-free entry point holds (64 MiB)";
    default: return "unknown error";
  }
}

const char* ews_version(void) { return "0.1.0"; }

}  // extern "C"
