// Front of an EWS block on MI355X (gfx950): the clock theta and the lifted path p, computed on the device from the
// block's raw inputs, forward and backward.
//
// Clock (ews/clocks.py:164-267, 443-466). Per sample, with dx_s the driver increment between rows s - 1 and s
// (s >= 1; the driver scaled by in_scale before the difference for the gated modes; for an increment driver, whose
// path is the masked cumulative sum of its rows, dx_s = m_s x_s), incr_s is sqrt(|dx|^2 + eps), |dx|^2,
// relu(w . dx - b) or sum_k clip(w_k . dx - b_k, 0, 1), times the pair mask m_s m_{s-1}; V_r = sum_{s <= r} incr_s,
// and theta_r = alpha t_s(i) + (1 - alpha) V_s(r), t_s(i) or V(r) / c, read at i = min(r, n) (n = last real row;
// past it the increments are masked, so V is frozen already). Scalings: none, [0,1], [-1,1] through the first and
// last values (+1e-12), or a constant denominator. V is scanned in float64: a workgroup per (chunk of 256 rows,
// sample), one thread per row; chunk sums first (one pass), then each chunk adds the sums before it.
//
// Backward: dV_r from d theta_r (with the per-sample normaliser's end term dV_end = -sum_r kappa dVs_r V_r / den^2),
// dincr_s = sum_{r >= s} dV_r + dV_end (a reverse scan in the same chunk scheme), then d dx_s, the gate parameter
// gradients and the driver gradient (value driver: g_r = dx'_r - dx'_{r+1}; increment driver: g_r = m_r dx'_r).
//
// Lift (ews/params.py:1181-1191, ews/block.py:284-301, ews/paths.py:126-131). u_r = [theta_app_r | branch_r] (or
// the branch alone), the branch replaced by its masked cumulative sum under path_mode "increment"; p_r = u_i B^T
// (or [u_i0, u_i,1: B^T], or u_i) at i = min(r, n) (forward fill); a zero row in front with a basepoint. A
// workgroup per (chunk of 128 rows, sample): the rows' inputs staged in LDS, the cumulative sum as a segmented scan
// in LDS on top of a float64 chunk carry, the lift with B^T in LDS (lanes over output channels: coalesced rows).
// Backward: du = dp B, the B gradient as per-chunk partial sums of dp (x) u (reduced in a fixed order, so the
// result is deterministic), and the branch gradient as a reverse cumulative sum (increment) or with the rows
// past n summed into row n (value; the forward fill).
#include <hip/hip_runtime.h>

#include <cstdint>

#include "ews_hip.h"
#include "ews_lanes.h"

namespace ews {
namespace front {

constexpr int CR = 256;  // clock rows per workgroup (a thread per row)
constexpr int LR = 128;  // lift rows per workgroup
constexpr int MAXK = 8;  // clamped_gate rows

// ------------------------------------------------------------------------------------------------ block helpers
__device__ __forceinline__ double wave_sum(double v) { return lanes::sum64(v); }
__device__ __forceinline__ float wave_sumf(float v) { return lanes::sum64(v); }

// sum over the 256 threads, returned to all (sh: 4 doubles of LDS)
__device__ double block_sum(double v, double* sh) {
  v = wave_sum(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = v;
  __syncthreads();
  return (sh[0] + sh[1]) + (sh[2] + sh[3]);
}

// inclusive prefix sum over the 256 threads in thread order
__device__ double block_scan(double v, double* sh) {
  const int l = threadIdx.x & 63, w = threadIdx.x >> 6;
  for (int o = 1; o < 64; o <<= 1) {
    const double u = __shfl_up(v, o, 64);
    if (l >= o) v += u;
  }
  __syncthreads();
  if (l == 63) sh[w] = v;
  __syncthreads();
  double off = 0.0;
  for (int q = 0; q < w; ++q) off += sh[q];
  return v + off;
}

// inclusive suffix sum over the 256 threads (thread t: sum over t' >= t)
__device__ double block_rscan(double v, double* sh) {
  const int l = threadIdx.x & 63, w = threadIdx.x >> 6;
  for (int o = 1; o < 64; o <<= 1) {
    const double u = __shfl_down(v, o, 64);
    if (l + o < 64) v += u;
  }
  __syncthreads();
  if (l == 0) sh[w] = v;
  __syncthreads();
  double off = 0.0;
  for (int q = 3; q > w; --q) off += sh[q];
  return v + off;
}

// last real row of each sample: n = sum(mask) - 1 (a workgroup per sample)
__global__ __launch_bounds__(256) void k_last_row(const uint8_t* m, int L, int* nrow) {
  __shared__ double sh[4];
  const int b = blockIdx.x;
  double cnt = 0.0;
  for (int r = threadIdx.x; r < L; r += 256) cnt += m[(size_t)b * L + r] ? 1.0 : 0.0;
  cnt = block_sum(cnt, sh);
  if (threadIdx.x == 0) nrow[b] = (int)cnt - 1;
}

// ================================================================================================== clock
struct CArgs {
  int B, L, c, mode, scaling, constant, K, has_mask, incr, has_tden, bp, learned;
  float alpha, C, tden, eps, sc;
  int nch, P;
  const float* t;
  const float* x;
  const uint8_t* m;
  const float* prm;
  float* theta;
  int* nrow;     // (B) residual
  double* csum;  // (B, nch) residual: chunk sums of the increments
  const float* gth;
  float* gx;
  double* dsum;  // (B, nch) chunk sums of dV
  double* psum;  // (B, nch) chunk sums of kappa dVs V (per-sample normaliser)
  double* part;  // (B nch, P) parameter partials: [alpha | w | b]
  float* gprm;
};

__device__ __forceinline__ bool valid(const CArgs& a, int b, int s) {
  return !a.has_mask || a.m[(size_t)b * a.L + s] != 0;
}
__device__ __forceinline__ bool pair_ok(const CArgs& a, int b, int s) {
  return s >= 1 && s < a.L && (!a.has_mask || (valid(a, b, s) && valid(a, b, s - 1)));
}

// dx_s (1 <= s < L)
template <int CB>
__device__ __forceinline__ void row_delta(const CArgs& a, int b, int s, float (&dx)[CB]) {
  const float* xs = a.x + ((size_t)b * a.L + s) * a.c;
  if (a.incr) {
    const bool ms = valid(a, b, s);
#pragma unroll
    for (int j = 0; j < CB; ++j) dx[j] = (j < a.c && ms) ? a.sc * xs[j] : 0.0f;
  } else {
    const float* xp = xs - a.c;
#pragma unroll
    for (int j = 0; j < CB; ++j) dx[j] = j < a.c ? a.sc * xs[j] - a.sc * xp[j] : 0.0f;
  }
}

// the increment of dx (unmasked); z: gate pre-activations; sq: |dx|^2
template <int CB>
__device__ __forceinline__ float row_incr(const CArgs& a, const float (&dx)[CB], float (&z)[MAXK]) {
  if (a.mode == EWS_CLOCK_VARIATION || a.mode == EWS_CLOCK_QUAD_VARIATION) {
    float sq = 0.0f;
#pragma unroll
    for (int j = 0; j < CB; ++j) sq = fmaf(dx[j], dx[j], sq);
    return a.mode == EWS_CLOCK_VARIATION ? sqrtf(sq + a.eps) : sq;
  }
  const float* w = a.prm;
  const float* bb = a.prm + a.K * a.c;
  float acc = 0.0f;
#pragma unroll
  for (int k = 0; k < MAXK; ++k) {
    z[k] = 0.0f;
    if (k < a.K) {
      float zk = 0.0f;
#pragma unroll
      for (int j = 0; j < CB; ++j)
        if (j < a.c) zk = fmaf(w[k * a.c + j], dx[j], zk);
      zk -= bb[k];
      z[k] = zk;
      acc += a.mode == EWS_CLOCK_TOKEN_GATED ? fmaxf(zk, 0.0f) : fminf(fmaxf(zk, 0.0f), 1.0f);
    }
  }
  return acc;
}

__device__ __forceinline__ double time_part(const CArgs& a, int i) {
  const double t = a.t[i], t0 = a.t[0];
  if (a.has_tden) {
    const double z = (t - t0) / (double)a.tden;
    return a.scaling == EWS_SCALING_SYM ? 2.0 * z - 1.0 : z;
  }
  switch (a.scaling) {
    case EWS_SCALING_NONE: return t;
    case EWS_SCALING_STEPS: return (double)i;
    default: {
      const double z = (t - t0) / ((a.t[a.L - 1] - t0) + 1e-12);
      return a.scaling == EWS_SCALING_SYM ? 2.0 * z - 1.0 : z;
    }
  }
}

// V_s and its derivative factor kappa / den
__device__ __forceinline__ double var_part(const CArgs& a, double V, double Vend, double* dfac) {
  if (a.constant) {
    const double k = a.scaling == EWS_SCALING_SYM ? 2.0 : 1.0;
    *dfac = k / (double)a.C;
    return a.scaling == EWS_SCALING_SYM ? 2.0 * V / (double)a.C - 1.0 : V / (double)a.C;
  }
  if (a.scaling == EWS_SCALING_NONE) {
    *dfac = 1.0;
    return V;
  }
  const double den = Vend + 1e-12;
  const double k = a.scaling == EWS_SCALING_SYM ? 2.0 : 1.0;
  *dfac = k / den;
  return a.scaling == EWS_SCALING_SYM ? 2.0 * (V / den) - 1.0 : V / den;
}

__device__ __forceinline__ bool gated(const CArgs& a) {
  return a.mode == EWS_CLOCK_TOKEN_GATED || a.mode == EWS_CLOCK_CLAMPED_GATE;
}
__device__ __forceinline__ double alpha_of(const CArgs& a) { return a.learned ? (double)a.prm[0] : (double)a.alpha; }

// the chunk's carry (sum of the chunk sums before it) and the sample's total
__device__ __forceinline__ void chunk_carry(const double* cs, int nch, int ch, double* sh, double& carry,
                                            double& total) {
  double c = 0.0, t = 0.0;
  for (int q = threadIdx.x; q < nch; q += 256) {
    const double v = cs[q];
    t += v;
    if (q < ch) c += v;
  }
  carry = block_sum(c, sh);
  total = block_sum(t, sh);
}

template <int CB>
__global__ __launch_bounds__(256) void k_clock_sums(CArgs a) {
  __shared__ double sh[4];
  const int ch = blockIdx.x, b = blockIdx.y, s = ch * CR + threadIdx.x;
  float v = 0.0f;
  if (pair_ok(a, b, s)) {
    float dx[CB], z[MAXK];
    row_delta<CB>(a, b, s, dx);
    v = row_incr<CB>(a, dx, z);
  }
  const double tot = block_sum((double)v, sh);
  if (threadIdx.x == 0) a.csum[(size_t)b * a.nch + ch] = tot;
}

// V at row s of the chunk (carry + in-chunk inclusive scan); also the sample total
template <int CB>
__device__ __forceinline__ double row_V(const CArgs& a, int b, int ch, int s, double* sh, double& total) {
  double carry = 0.0;
  total = 0.0;
  if (a.mode == EWS_CLOCK_TIME) return 0.0;
  chunk_carry(a.csum + (size_t)b * a.nch, a.nch, ch, sh, carry, total);
  float v = 0.0f;
  if (pair_ok(a, b, s)) {
    float dx[CB], z[MAXK];
    row_delta<CB>(a, b, s, dx);
    v = row_incr<CB>(a, dx, z);
  }
  return carry + block_scan((double)v, sh);
}

template <int CB>
__global__ __launch_bounds__(256) void k_clock_rows(CArgs a) {
  __shared__ double sh[4];
  const int ch = blockIdx.x, b = blockIdx.y, s = ch * CR + threadIdx.x;
  double total;
  const double V = row_V<CB>(a, b, ch, s, sh, total);
  if (s >= a.L) return;
  const int n = a.has_mask ? a.nrow[b] : a.L - 1;
  const int i = n >= 0 ? min(s, n) : a.L - 1;
  double th;
  if (a.mode == EWS_CLOCK_TIME) {
    th = time_part(a, i);
  } else if (gated(a)) {
    th = V / (double)a.C;
  } else {
    double f;
    const double al = alpha_of(a);
    th = al * time_part(a, i) + (1.0 - al) * var_part(a, V, total, &f);
  }
  float* out = a.theta + (size_t)b * (a.L + a.bp);
  out[s + a.bp] = (float)th;
  if (a.bp && s == 0) out[0] = (float)th;
}

// d theta_r of scan row r (the basepoint copy adds to row 0)
__device__ __forceinline__ double row_g(const CArgs& a, int b, int s) {
  const float* g = a.gth + (size_t)b * (a.L + a.bp);
  double v = g[s + a.bp];
  if (a.bp && s == 0) v += g[0];
  return v;
}

// dV_r, and the per-sample normaliser term kappa dVs V / den^2 and the alpha term
template <int CB>
__device__ __forceinline__ double row_dV(const CArgs& a, int b, int ch, int s, double* sh, double& total,
                                         double& pterm, double& aterm) {
  const double V = row_V<CB>(a, b, ch, s, sh, total);
  pterm = 0.0;
  aterm = 0.0;
  if (s >= a.L) return 0.0;
  const double g = row_g(a, b, s);
  if (gated(a)) return g / (double)a.C;
  const int n = a.has_mask ? a.nrow[b] : a.L - 1;
  const int i = n >= 0 ? min(s, n) : a.L - 1;
  double f;
  const double al = alpha_of(a);
  const double Vs = var_part(a, V, total, &f);
  aterm = g * (time_part(a, i) - Vs);
  const double dVs = (1.0 - al) * g;
  if (!a.constant && a.scaling != EWS_SCALING_NONE) pterm = dVs * f * V / (total + 1e-12);
  return dVs * f;
}

template <int CB>
__global__ __launch_bounds__(256) void k_clock_bsums(CArgs a) {
  __shared__ double sh[4];
  const int ch = blockIdx.x, b = blockIdx.y, s = ch * CR + threadIdx.x;
  double total, pterm, aterm;
  const double dV = row_dV<CB>(a, b, ch, s, sh, total, pterm, aterm);
  const double d = block_sum(dV, sh);
  const double p = block_sum(pterm, sh);
  const double al = block_sum(aterm, sh);
  if (threadIdx.x == 0) {
    const size_t q = (size_t)b * a.nch + ch;
    a.dsum[q] = d;
    a.psum[q] = p;
    if (a.learned) a.part[q * a.P] = al;
  }
}

// d dx_s = coef . (dx_s for the variations, w_k rows for the gates), coef from dincr_s
template <int CB>
__device__ __forceinline__ void row_coef(const CArgs& a, int b, int s, double dincr, float (&dx)[CB],
                                         float (&coef)[MAXK]) {
#pragma unroll
  for (int k = 0; k < MAXK; ++k) coef[k] = 0.0f;
#pragma unroll
  for (int j = 0; j < CB; ++j) dx[j] = 0.0f;
  if (!pair_ok(a, b, s)) return;
  float z[MAXK];
  row_delta<CB>(a, b, s, dx);
  const float inc = row_incr<CB>(a, dx, z);
  if (a.mode == EWS_CLOCK_VARIATION) coef[0] = (float)(dincr / (double)inc);
  else if (a.mode == EWS_CLOCK_QUAD_VARIATION) coef[0] = (float)(2.0 * dincr);
  else if (a.mode == EWS_CLOCK_TOKEN_GATED) coef[0] = z[0] > 0.0f ? (float)dincr : 0.0f;
  else {
#pragma unroll
    for (int k = 0; k < MAXK; ++k) coef[k] = (k < a.K && z[k] > 0.0f && z[k] < 1.0f) ? (float)dincr : 0.0f;
  }
}

// component j of d dx given coef and dx
template <int CB>
__device__ __forceinline__ float ddx(const CArgs& a, const float (&dx)[CB], const float (&coef)[MAXK], int j) {
  if (!gated(a)) return coef[0] * dx[j];
  float v = 0.0f;
#pragma unroll
  for (int k = 0; k < MAXK; ++k)
    if (k < a.K) v = fmaf(coef[k], a.prm[k * a.c + j], v);
  return v;
}

template <int CB>
__global__ __launch_bounds__(256) void k_clock_brows(CArgs a) {
  __shared__ double sh[4];
  __shared__ float s_next[MAXK];
  __shared__ float s_coef[CR][MAXK];
  const int ch = blockIdx.x, b = blockIdx.y, s = ch * CR + threadIdx.x;
  double total, pterm, aterm;
  const double dV = row_dV<CB>(a, b, ch, s, sh, total, pterm, aterm);
  // carry from the chunks after this one and the normaliser's end term
  double rc = 0.0, pend = 0.0;
  {
    double r = 0.0, p = 0.0;
    for (int q = threadIdx.x; q < a.nch; q += 256) {
      p += a.psum[(size_t)b * a.nch + q];
      if (q > ch) r += a.dsum[(size_t)b * a.nch + q];
    }
    rc = block_sum(r, sh);
    pend = block_sum(p, sh);
  }
  const double dVend = -pend;
  const double dincr = block_rscan(dV, sh) + rc + dVend;
  float dx[CB], coef[MAXK];
  row_coef<CB>(a, b, s, dincr, dx, coef);
#pragma unroll
  for (int k = 0; k < MAXK; ++k) s_coef[threadIdx.x][k] = coef[k];
  // the first row of the next chunk: dincr = carry of the rows after this chunk + end term
  if (threadIdx.x == CR - 1) {
    float dn[CB], cn[MAXK];
    row_coef<CB>(a, b, s + 1, rc + dVend, dn, cn);
#pragma unroll
    for (int k = 0; k < MAXK; ++k) s_next[k] = cn[k];
  }
  __syncthreads();
  // gate parameter partials: dw_kj = coef_k dx_j, db_k = -coef_k
  if (gated(a)) {
    __shared__ float s_red[4][MAXK * 64 + MAXK];
    const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
    for (int k = 0; k < a.K; ++k) {
      for (int j = 0; j < a.c; ++j) {
        float v = 0.0f;
#pragma unroll
        for (int jj = 0; jj < CB; ++jj)
          if (jj == j) v = coef[k] * dx[jj];
        v = wave_sumf(v);
        if (l == 0) s_red[w][k * a.c + j] = v;
      }
      const float vb = wave_sumf(-coef[k]);
      if (l == 0) s_red[w][a.K * a.c + k] = vb;
    }
    __syncthreads();
    const size_t q = (size_t)b * a.nch + ch;
    for (int p = threadIdx.x; p < a.K * a.c + a.K; p += 256)
      a.part[q * a.P + p] = (double)((s_red[0][p] + s_red[1][p]) + (s_red[2][p] + s_red[3][p]));
  }
  if (a.gx == nullptr || s >= a.L) return;
  float* gx = a.gx + ((size_t)b * a.L + s) * a.c;
  if (a.incr) {
    // dx_s = sc m_s x_s: d x_s = sc d dx_s (the pair mask already holds m_s)
#pragma unroll
    for (int j = 0; j < CB; ++j)
      if (j < a.c) gx[j] = a.sc * ddx<CB>(a, dx, coef, j);
  } else {
    // x_s enters dx_s (+) and dx_{s+1} (-)
    float cn[MAXK], dn[CB];
    const float* cr = threadIdx.x == CR - 1 ? s_next : s_coef[threadIdx.x + 1];
#pragma unroll
    for (int k = 0; k < MAXK; ++k) cn[k] = cr[k];
#pragma unroll
    for (int j = 0; j < CB; ++j) dn[j] = 0.0f;
    if (!gated(a) && s + 1 < a.L && pair_ok(a, b, s + 1)) row_delta<CB>(a, b, s + 1, dn);
#pragma unroll
    for (int j = 0; j < CB; ++j)
      if (j < a.c) {
        const float up = s + 1 < a.L ? ddx<CB>(a, dn, cn, j) : 0.0f;
        gx[j] = a.sc * (ddx<CB>(a, dx, coef, j) - up);
      }
  }
}

// =================================================================================================== lift
struct LArgs {
  int B, L, H, app, Hin, w, lift, incr, has_mask, bp, nch, Hs;
  int wl, hl;        // the matrix: (wl, hl)
  int SU, SP, SM;    // LDS row strides (odd) of the u, dp and matrix tiles
  const float* br;
  const float* tha;
  const uint8_t* m;
  const float* M;
  float* p;
  int* nrow;
  double* csum;  // (B, nch, H) residual: chunk sums of the masked branch rows (increment)
  const float* gp;
  float* gbr;
  float* gtha;
  double* dsum;  // (B, nch, 2, Hin): sums of du over all rows / over rows past n
  float* part;   // (B nch, wl hl)
  double* part2; // (S, wl hl) first-level sums of part
  float* gM;
};

// Walks e = tid, tid + 256, ... over a row-major tile of width X as (row r, column c), with no division per step.
struct TileWalk {
  int r, c, dr, dc, X;
  __device__ explicit TileWalk(int X_) : X(X_) {
    r = (int)threadIdx.x / X;
    c = (int)threadIdx.x - r * X;
    dr = 256 / X;
    dc = 256 - dr * X;
  }
  __device__ void next() {
    r += dr;
    c += dc;
    if (c >= X) {
      c -= X;
      ++r;
    }
  }
};

__device__ __forceinline__ bool lvalid(const LArgs& a, int b, int r) {
  return !a.has_mask || a.m[(size_t)b * a.L + r] != 0;
}
__device__ __forceinline__ int lastrow(const LArgs& a, int b) { return a.has_mask ? a.nrow[b] : a.L - 1; }
__device__ __forceinline__ int fill_idx(int r, int n, int L) { return n >= 0 ? min(r, n) : L - 1; }

// LDS carve-up (in floats; the float64 region starts at an even float offset), sized by the actual widths
struct LLds {
  int DP, DU, U, Ms, seg, dbl, nfloat;
};
__host__ __device__ inline LLds lift_lds(const LArgs& a, bool dp, bool du, bool u, bool seg) {
  LLds l{};
  int o = 0;
  l.DP = o;
  o += dp ? LR * a.SP : 0;
  l.DU = o;
  o += du ? LR * a.SU : 0;
  l.U = o;
  o += u ? LR * a.SU : 0;
  l.Ms = o;
  o += a.wl * a.SM;
  l.seg = o;
  o += seg ? 256 : 0;
  o = (o + 1) & ~1;
  l.dbl = o;
  l.nfloat = o;
  return l;
}
constexpr int kFwdDoubles = 64 + 256;        // carry, reduction scratch
constexpr int kBsumDoubles = 512;            // two reductions
constexpr int kBrowDoubles = 64 + 160 + 256; // carry, 2 x 80 sums, reduction scratch

__global__ __launch_bounds__(256) void k_lift_sums(LArgs a) {
  __shared__ double red[256];
  const int ch = blockIdx.x, b = blockIdx.y;
  const int r0 = ch * LR, r1 = min(r0 + LR, a.L);
  const int j = threadIdx.x % a.Hs, part = threadIdx.x / a.Hs, np = 256 / a.Hs;
  double acc = 0.0;
  if (j < a.H)
    for (int r = r0 + part; r < r1; r += np)
      if (lvalid(a, b, r)) acc += a.br[((size_t)b * a.L + r) * a.H + j];
  red[threadIdx.x] = acc;
  __syncthreads();
  if (part == 0 && j < a.H) {
    double t = 0.0;
    for (int q = 0; q < np; ++q) t += red[q * a.Hs + j];
    a.csum[((size_t)b * a.nch + ch) * a.H + j] = t;
  }
}

// U tile: u rows of the chunk (forward-filled for the value path; the cumulative sum for the increment path).
// carry: 64 doubles, red: 256 doubles, segtot: 256 floats.
__device__ void load_u(const LArgs& a, int b, int ch, float* U, double* carry, double* red, float* segtot) {
  const int r0 = ch * LR, n = lastrow(a, b);
  for (TileWalk tw(a.Hin); tw.r < LR; tw.next()) {
    const int r = tw.r, i = tw.c, row = r0 + r;
    float v = 0.0f;
    if (row < a.L) {
      const int src = fill_idx(row, n, a.L);
      if (a.app && i == 0) {
        v = a.tha[(size_t)b * a.L + src];
      } else {
        const int j = i - a.app;
        if (a.incr) v = lvalid(a, b, row) ? a.br[((size_t)b * a.L + row) * a.H + j] : 0.0f;
        else v = a.br[((size_t)b * a.L + src) * a.H + j];
      }
    }
    U[r * a.SU + i] = v;
  }
  if (!a.incr) {
    __syncthreads();
    return;
  }
  // float64 carry of each channel: the chunk sums before this chunk
  {
    const int j = threadIdx.x % a.Hs, part = threadIdx.x / a.Hs, np = 256 / a.Hs;
    double c = 0.0;
    if (j < a.H)
      for (int q = part; q < ch; q += np) c += a.csum[((size_t)b * a.nch + q) * a.H + j];
    red[threadIdx.x] = c;
    __syncthreads();
    if (part == 0 && j < a.H) {
      double t = 0.0;
      for (int q = 0; q < np; ++q) t += red[q * a.Hs + j];
      carry[j] = t;
    }
  }
  __syncthreads();
  // segmented inclusive scan down each channel's column (nseg * Hs <= 256 segments)
  const int nseg = min(256 / a.Hs, 32), rps = LR / nseg;
  const int j = threadIdx.x % a.Hs, sg = threadIdx.x / a.Hs;
  const bool act = sg < nseg && j < a.H;
  float* col = U + a.app + j;
  if (act) {
    float t = 0.0f;
    for (int r = sg * rps; r < (sg + 1) * rps; ++r) t += col[r * a.SU];
    segtot[sg * a.Hs + j] = t;
  }
  __syncthreads();
  if (act) {
    double off = carry[j];
    for (int q = 0; q < sg; ++q) off += segtot[q * a.Hs + j];
    for (int r = sg * rps; r < (sg + 1) * rps; ++r) {
      off += col[r * a.SU];
      col[r * a.SU] = (float)off;
    }
  }
  __syncthreads();
}

// the matrix into LDS: Ms[o * SM + i] = M[o][i] (o < wl, i < hl)
__device__ void load_matrix(const LArgs& a, float* Ms) {
  if (a.lift == EWS_LIFT_NONE) return;
  for (TileWalk tw(a.hl); tw.r < a.wl; tw.next()) Ms[tw.r * a.SM + tw.c] = a.M[tw.r * a.hl + tw.c];
}

__global__ __launch_bounds__(256) void k_lift_rows(LArgs a) {
  extern __shared__ float lds[];
  const LLds l = lift_lds(a, false, false, true, true);
  float* U = lds + l.U;
  float* Ms = lds + l.Ms;
  float* segtot = lds + l.seg;
  double* carry = reinterpret_cast<double*>(lds + l.dbl);
  double* red = carry + 64;
  const int ch = blockIdx.x, b = blockIdx.y, r0 = ch * LR;
  load_matrix(a, Ms);
  load_u(a, b, ch, U, carry, red, segtot);
  float* pb = a.p + (size_t)b * (a.L + a.bp) * a.w;
  if (a.bp && ch == 0)
    for (int o = threadIdx.x; o < a.w; o += 256) pb[o] = 0.0f;
  for (TileWalk tw(a.w); tw.r < LR; tw.next()) {
    const int r = tw.r, o = tw.c, row = r0 + r;
    if (row >= a.L) break;
    const float* u = U + r * a.SU;
    float v;
    if (a.lift == EWS_LIFT_NONE) {
      v = u[o];
    } else if (a.lift == EWS_LIFT_FULL) {
      v = 0.0f;
      for (int i = 0; i < a.hl; ++i) v = fmaf(Ms[o * a.SM + i], u[i], v);
    } else if (o == 0) {
      v = u[0];
    } else {
      v = 0.0f;
      for (int i = 0; i < a.hl; ++i) v = fmaf(Ms[(o - 1) * a.SM + i], u[i + 1], v);
    }
    pb[(size_t)(row + a.bp) * a.w + o] = v;
  }
}

// dP tile (rows of grad_path) and DU = dP B (per row, the cotangent of u)
__device__ void load_du(const LArgs& a, int b, int ch, float* DP, const float* Ms, float* DU) {
  const int r0 = ch * LR;
  const float* gp = a.gp + (size_t)b * (a.L + a.bp) * a.w;
  for (TileWalk tw(a.w); tw.r < LR; tw.next()) {
    const int r = tw.r, o = tw.c, row = r0 + r;
    DP[r * a.SP + o] = row < a.L ? gp[(size_t)(row + a.bp) * a.w + o] : 0.0f;
  }
  __syncthreads();
  for (TileWalk tw(a.Hin); tw.r < LR; tw.next()) {
    const int r = tw.r, i = tw.c;
    const float* dp = DP + r * a.SP;
    float v;
    if (a.lift == EWS_LIFT_NONE) {
      v = dp[i];
    } else if (a.lift == EWS_LIFT_FULL) {
      v = 0.0f;
      for (int o = 0; o < a.wl; ++o) v = fmaf(Ms[o * a.SM + i], dp[o], v);
    } else if (i == 0) {
      v = dp[0];
    } else {
      v = 0.0f;
      for (int o = 0; o < a.wl; ++o) v = fmaf(Ms[o * a.SM + i - 1], dp[o + 1], v);
    }
    DU[r * a.SU + i] = v;
  }
  __syncthreads();
}

__device__ __forceinline__ int pow2_at_least8(int x) {
  return x > 64 ? 128 : (x > 32 ? 64 : (x > 16 ? 32 : (x > 8 ? 16 : 8)));
}

// per chunk: sums of du over every row and over the rows past the last real row (increment path or mask only)
__global__ __launch_bounds__(256) void k_lift_bsums(LArgs a) {
  extern __shared__ float lds[];
  const LLds l = lift_lds(a, true, true, false, false);
  float* DP = lds + l.DP;
  float* DU = lds + l.DU;
  float* Ms = lds + l.Ms;
  double* red = reinterpret_cast<double*>(lds + l.dbl);
  const int ch = blockIdx.x, b = blockIdx.y, r0 = ch * LR;
  load_matrix(a, Ms);
  __syncthreads();
  load_du(a, b, ch, DP, Ms, DU);
  const int n = lastrow(a, b);
  const int Hs2 = pow2_at_least8(a.Hin);
  const int i = threadIdx.x % Hs2, part = threadIdx.x / Hs2, np = 256 / Hs2;
  double all = 0.0, tail = 0.0;
  if (i < a.Hin)
    for (int r = part; r < LR; r += np) {
      const int row = r0 + r;
      if (row >= a.L) break;
      const double v = DU[r * a.SU + i];
      all += v;
      if (row > n) tail += v;
    }
  red[threadIdx.x] = all;
  red[256 + threadIdx.x] = tail;
  __syncthreads();
  if (part == 0 && i < a.Hin) {
    double s0 = 0.0, s1 = 0.0;
    for (int q = 0; q < np; ++q) {
      s0 += red[q * Hs2 + i];
      s1 += red[256 + q * Hs2 + i];
    }
    double* o = a.dsum + ((size_t)b * a.nch + ch) * 2 * a.Hin;
    o[i] = s0;
    o[a.Hin + i] = s1;
  }
}

__global__ __launch_bounds__(256) void k_lift_brows(LArgs a) {
  extern __shared__ float lds[];
  const LLds l = lift_lds(a, true, true, true, true);
  float* DP = lds + l.DP;
  float* DU = lds + l.DU;
  float* U = lds + l.U;
  float* Ms = lds + l.Ms;
  float* segtot = lds + l.seg;
  double* carry = reinterpret_cast<double*>(lds + l.dbl);  // 64
  double* acc = carry + 64;                                 // 2 x 80: sums after this chunk, sums past n
  double* red = acc + 160;                                  // 256
  const int ch = blockIdx.x, b = blockIdx.y, r0 = ch * LR;
  load_matrix(a, Ms);
  __syncthreads();
  load_du(a, b, ch, DP, Ms, DU);
  const int n = lastrow(a, b);
  const bool need_sums = a.incr || a.has_mask;
  // float64 sums over the other chunks: du after this chunk (increment path), du past n (the fill)
  if (need_sums) {
    const int Hs2 = pow2_at_least8(a.Hin);
    const int i = threadIdx.x % Hs2, part = threadIdx.x / Hs2, np = 256 / Hs2;
    for (int which = 0; which < 2; ++which) {
      double s = 0.0;
      if (i < a.Hin)
        for (int q = part; q < a.nch; q += np) {
          const double* d = a.dsum + ((size_t)b * a.nch + q) * 2 * a.Hin;
          if (which == 0 && q > ch) s += d[i];
          if (which == 1) s += d[a.Hin + i];
        }
      red[threadIdx.x] = s;
      __syncthreads();
      if (part == 0 && i < a.Hin) {
        double t = 0.0;
        for (int q = 0; q < np; ++q) t += red[q * Hs2 + i];
        acc[which * 80 + i] = t;
      }
      __syncthreads();
    }
  }
  // B gradient partial: sum over the chunk's rows of dp (x) u (u forward-filled, as the forward read it)
  if (a.lift != EWS_LIFT_NONE) {
    load_u(a, b, ch, U, carry, red, segtot);
    const int nr = min(LR, a.L - r0);
    const int oo = a.lift == EWS_LIFT_PRESERVE ? 1 : 0;
    float* pp = a.part + ((size_t)b * a.nch + ch) * a.wl * a.hl;
    for (TileWalk tw(a.hl); tw.r < a.wl; tw.next()) {
      const int o = tw.r, i = tw.c;
      float v = 0.0f;
      for (int r = 0; r < nr; ++r) v = fmaf(DP[r * a.SP + o + oo], U[r * a.SU + i + oo], v);
      pp[o * a.hl + i] = v;
    }
  }
  // branch and appended-clock gradients
  const int tr = n >= 0 ? n : a.L - 1;
  if (a.app) {
    for (int r = threadIdx.x; r < LR; r += 256) {
      const int row = r0 + r;
      if (row >= a.L) break;
      float v = row <= n ? DU[r * a.SU] : 0.0f;
      if (row == tr && a.has_mask) v += (float)acc[80];
      a.gtha[(size_t)b * a.L + row] = v;
    }
  }
  if (!a.incr) {
    for (TileWalk tw(a.H); tw.r < LR; tw.next()) {
      const int r = tw.r, j = tw.c, row = r0 + r;
      if (row >= a.L) break;
      float v = row <= n ? DU[r * a.SU + a.app + j] : 0.0f;
      if (row == tr && a.has_mask) v += (float)acc[80 + a.app + j];
      a.gbr[((size_t)b * a.L + row) * a.H + j] = v;
    }
    return;
  }
  // increment path: d branch_s = m_s sum_{r >= s} du_r, a segmented suffix scan down each column
  __syncthreads();
  const int nseg = min(256 / a.Hs, 32), rps = LR / nseg;
  const int j = threadIdx.x % a.Hs, sg = threadIdx.x / a.Hs;
  const bool act = sg < nseg && j < a.H;
  float* col = DU + a.app + j;
  if (act) {
    float t = 0.0f;
    for (int r = sg * rps; r < (sg + 1) * rps; ++r) t += r0 + r < a.L ? col[r * a.SU] : 0.0f;
    segtot[sg * a.Hs + j] = t;
  }
  __syncthreads();
  if (act) {
    double off = acc[a.app + j];
    for (int q = sg + 1; q < nseg; ++q) off += segtot[q * a.Hs + j];
    for (int r = (sg + 1) * rps - 1; r >= sg * rps; --r) {
      const int row = r0 + r;
      if (row >= a.L) continue;
      off += col[r * a.SU];
      a.gbr[((size_t)b * a.L + row) * a.H + j] = lvalid(a, b, row) ? (float)off : 0.0f;
    }
  }
}

// Deterministic two-level sum of per-chunk partials part (nq, P) -> out (P): workgroup (column block of 64,
// segment of QB partials) sums its segment with 4 wavefronts (fixed order), then one thread per column sums the
// segments.
constexpr int QB = 256;
template <class T>
__global__ __launch_bounds__(256) void k_reduce_stage1(const T* part, int nq, int P, double* out2) {
  __shared__ double red[4][64];
  const int l = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int p = blockIdx.x * 64 + l, sg = blockIdx.y;
  const int q0 = sg * QB, q1 = min(nq, q0 + QB);
  double s0 = 0.0, s1 = 0.0;
  if (p < P) {
    int q = q0 + w;
    for (; q + 4 < q1; q += 8) {
      s0 += (double)part[(size_t)q * P + p];
      s1 += (double)part[(size_t)(q + 4) * P + p];
    }
    if (q < q1) s0 += (double)part[(size_t)q * P + p];
  }
  red[w][l] = s0 + s1;
  __syncthreads();
  if (w == 0 && p < P) out2[(size_t)sg * P + p] = (red[0][l] + red[1][l]) + (red[2][l] + red[3][l]);
}

__global__ __launch_bounds__(256) void k_reduce_stage2(const double* out2, int S, int P, float* out) {
  const int p = blockIdx.x * 256 + threadIdx.x;
  if (p >= P) return;
  double acc = 0.0;
  for (int s = 0; s < S; ++s) acc += out2[(size_t)s * P + p];
  out[p] = (float)acc;
}

}  // namespace front
}  // namespace ews

// ================================================================================================= C ABI
namespace {

using namespace ews::front;

size_t al256f(size_t x) { return (x + 255) & ~(size_t)255; }

// segments of the first-level partial sums
size_t nseg(size_t nq) { return (nq + QB - 1) / QB; }

size_t lds_bytes(const LLds& l, int ndouble) { return (size_t)l.nfloat * 4 + (size_t)ndouble * 8; }

int clock_check(const ews_clock_desc* s) {
  if (!s) return EWS_ERR_NULL;
  if (s->batch < 1 || s->length < 1) return EWS_ERR_SHAPE;
  if (s->mode < EWS_CLOCK_TIME || s->mode > EWS_CLOCK_CLAMPED_GATE) return EWS_ERR_OPTION;
  if (s->scaling < EWS_SCALING_NONE || s->scaling > EWS_SCALING_STEPS) return EWS_ERR_OPTION;
  if (s->normalize < 0 || s->normalize > 1) return EWS_ERR_OPTION;
  if (s->mode != EWS_CLOCK_TIME && (s->channels < 1 || s->channels > 64)) return EWS_ERR_SHAPE;
  if (s->scaling == EWS_SCALING_STEPS && (s->mode != EWS_CLOCK_TIME || s->has_time_denominator))
    return EWS_ERR_OPTION;
  if (s->mode == EWS_CLOCK_TOKEN_GATED && s->gates != 1) return EWS_ERR_SHAPE;
  if (s->mode == EWS_CLOCK_CLAMPED_GATE && (s->gates < 1 || s->gates > MAXK)) return EWS_ERR_SHAPE;
  const bool gate = s->mode == EWS_CLOCK_TOKEN_GATED || s->mode == EWS_CLOCK_CLAMPED_GATE;
  if (gate && (s->scaling != EWS_SCALING_NONE || !s->normalize || !(s->norm_constant != 0.0f)))
    return EWS_ERR_OPTION;
  if (!gate && s->mode != EWS_CLOCK_TIME && s->normalize && !(s->norm_constant != 0.0f)) return EWS_ERR_OPTION;
  if (s->has_time_denominator && !(s->time_denominator != 0.0f)) return EWS_ERR_OPTION;
  if (s->learned_alpha && (s->mode != EWS_CLOCK_VARIATION)) return EWS_ERR_OPTION;
  return EWS_OK;
}

int clock_nparams(const ews_clock_desc* s) {
  if (s->mode == EWS_CLOCK_TOKEN_GATED || s->mode == EWS_CLOCK_CLAMPED_GATE)
    return s->gates * s->channels + s->gates;
  return s->learned_alpha ? 1 : 0;
}

CArgs clock_args(const ews_clock_desc* s) {
  CArgs a{};
  a.B = s->batch;
  a.L = s->length;
  a.c = s->mode == EWS_CLOCK_TIME ? 0 : s->channels;
  a.mode = s->mode;
  a.scaling = s->scaling;
  a.constant = s->normalize;
  a.K = (s->mode == EWS_CLOCK_TOKEN_GATED || s->mode == EWS_CLOCK_CLAMPED_GATE) ? s->gates : 0;
  a.has_mask = s->has_mask ? 1 : 0;
  a.incr = s->increment_driver ? 1 : 0;
  a.has_tden = s->has_time_denominator ? 1 : 0;
  a.bp = s->basepoint ? 1 : 0;
  a.learned = s->learned_alpha ? 1 : 0;
  a.alpha = s->alpha;
  const bool gate = a.K > 0;
  a.C = gate ? s->norm_constant : (s->normalize ? s->norm_constant : 1.0f);
  a.tden = s->time_denominator;
  a.eps = s->variation_eps;
  a.sc = gate ? s->in_scale : 1.0f;
  a.nch = (a.L + CR - 1) / CR;
  a.P = clock_nparams(s);
  return a;
}

// residual: nrow (B ints) | csum (B nch doubles)
void clock_residual(CArgs& a, void* res) {
  char* p = static_cast<char*>(res);
  a.nrow = reinterpret_cast<int*>(p);
  a.csum = reinterpret_cast<double*>(p + al256f((size_t)a.B * 4));
}

int clock_cb(int c) { return c <= 8 ? 8 : (c <= 16 ? 16 : (c <= 32 ? 32 : 64)); }

int launched() { return hipGetLastError() == hipSuccess ? EWS_OK : EWS_ERR_LAUNCH; }

#define EWS_CB_LAUNCH(kern, cb, grid, st, a)                                       \
  do {                                                                             \
    if ((cb) == 8) hipLaunchKernelGGL(kern<8>, grid, dim3(256), 0, st, a);         \
    else if ((cb) == 16) hipLaunchKernelGGL(kern<16>, grid, dim3(256), 0, st, a);  \
    else if ((cb) == 32) hipLaunchKernelGGL(kern<32>, grid, dim3(256), 0, st, a);  \
    else hipLaunchKernelGGL(kern<64>, grid, dim3(256), 0, st, a);                  \
  } while (0)

int lift_check(const ews_lift_desc* s) {
  if (!s) return EWS_ERR_NULL;
  if (s->batch < 1 || s->length < 1 || s->branch_dim < 1 || s->branch_dim > 64) return EWS_ERR_SHAPE;
  if (s->append < 0 || s->append > 1 || s->out_dim < 1 || s->out_dim > 64) return EWS_ERR_SHAPE;
  if (s->lift < EWS_LIFT_NONE || s->lift > EWS_LIFT_PRESERVE) return EWS_ERR_OPTION;
  const int Hin = s->branch_dim + s->append;
  if (s->lift == EWS_LIFT_NONE && s->out_dim != Hin) return EWS_ERR_SHAPE;
  if (s->lift == EWS_LIFT_PRESERVE && (Hin < 2 || s->out_dim < 2)) return EWS_ERR_SHAPE;
  return EWS_OK;
}

LArgs lift_args(const ews_lift_desc* s) {
  LArgs a{};
  a.B = s->batch;
  a.L = s->length;
  a.H = s->branch_dim;
  a.app = s->append ? 1 : 0;
  a.Hin = a.H + a.app;
  a.w = s->out_dim;
  a.lift = s->lift;
  a.incr = s->increment ? 1 : 0;
  a.has_mask = s->has_mask ? 1 : 0;
  a.bp = s->basepoint ? 1 : 0;
  a.nch = (a.L + LR - 1) / LR;
  a.Hs = a.H > 32 ? 64 : (a.H > 16 ? 32 : (a.H > 8 ? 16 : (a.H > 4 ? 8 : (a.H > 2 ? 4 : (a.H > 1 ? 2 : 1)))));
  a.wl = a.lift == EWS_LIFT_FULL ? a.w : (a.lift == EWS_LIFT_PRESERVE ? a.w - 1 : 0);
  a.hl = a.lift == EWS_LIFT_FULL ? a.Hin : (a.lift == EWS_LIFT_PRESERVE ? a.Hin - 1 : 0);
  a.SU = a.Hin | 1;
  a.SP = a.w | 1;
  a.SM = a.hl | 1;
  return a;
}

void lift_residual(LArgs& a, void* res) {
  char* p = static_cast<char*>(res);
  a.nrow = reinterpret_cast<int*>(p);
  a.csum = reinterpret_cast<double*>(p + al256f((size_t)a.B * 4));
}

}  // namespace

extern "C" {

size_t ews_clock_residual_bytes(const ews_clock_desc* s) {
  if (clock_check(s) != EWS_OK) return 0;
  const CArgs a = clock_args(s);
  return al256f((size_t)a.B * 4) + al256f((size_t)a.B * a.nch * 8);
}

size_t ews_clock_workspace_bytes(const ews_clock_desc* s) {
  if (clock_check(s) != EWS_OK) return 0;
  const CArgs a = clock_args(s);
  const size_t q = (size_t)a.B * a.nch;
  const size_t P = a.P > 0 ? a.P : 1;
  return 2 * al256f(q * 8) + al256f(q * P * 8) + al256f(nseg(q) * P * 8);
}

int ews_clock_num_params(const ews_clock_desc* s) {
  if (clock_check(s) != EWS_OK) return -1;
  return clock_nparams(s);
}

int ews_clock_forward(const ews_clock_desc* s, const float* times, const float* driver, const uint8_t* mask,
                      const float* params, float* theta, void* residual, ews_stream_t stream) {
  const int rc = clock_check(s);
  if (rc != EWS_OK) return rc;
  CArgs a = clock_args(s);
  if (!times || !theta || !residual || (a.has_mask && !mask) || (a.mode != EWS_CLOCK_TIME && !driver) ||
      (a.P > 0 && !params))
    return EWS_ERR_NULL;
  a.t = times;
  a.x = driver;
  a.m = mask;
  a.prm = params;
  a.theta = theta;
  clock_residual(a, residual);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const dim3 grid(a.nch, a.B);
  if (a.has_mask) hipLaunchKernelGGL(k_last_row, dim3(a.B), dim3(256), 0, st, mask, a.L, a.nrow);
  const int cb = clock_cb(a.c);
  if (a.mode != EWS_CLOCK_TIME) EWS_CB_LAUNCH(k_clock_sums, cb, grid, st, a);
  EWS_CB_LAUNCH(k_clock_rows, cb, grid, st, a);
  return launched();
}

int ews_clock_backward(const ews_clock_desc* s, const float* times, const float* driver, const uint8_t* mask,
                       const float* params, const void* residual, const float* grad_theta, float* grad_driver,
                       float* grad_params, void* workspace, ews_stream_t stream) {
  const int rc = clock_check(s);
  if (rc != EWS_OK) return rc;
  CArgs a = clock_args(s);
  if (a.mode == EWS_CLOCK_TIME) return EWS_OK;  // no inputs with a gradient
  if (!times || !driver || !residual || !grad_theta || !workspace || (a.has_mask && !mask) ||
      (a.P > 0 && (!params || !grad_params)))
    return EWS_ERR_NULL;
  a.t = times;
  a.x = driver;
  a.m = mask;
  a.prm = params;
  a.gth = grad_theta;
  a.gx = grad_driver;
  a.gprm = grad_params;
  clock_residual(a, const_cast<void*>(residual));
  char* w = static_cast<char*>(workspace);
  const size_t q = (size_t)a.B * a.nch;
  a.dsum = reinterpret_cast<double*>(w);
  a.psum = reinterpret_cast<double*>(w + al256f(q * 8));
  a.part = reinterpret_cast<double*>(w + 2 * al256f(q * 8));
  const size_t P = a.P > 0 ? a.P : 1;
  double* part2 = reinterpret_cast<double*>(w + 2 * al256f(q * 8) + al256f(q * P * 8));
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const dim3 grid(a.nch, a.B);
  const int cb = clock_cb(a.c);
  EWS_CB_LAUNCH(k_clock_bsums, cb, grid, st, a);
  EWS_CB_LAUNCH(k_clock_brows, cb, grid, st, a);
  if (a.P > 0) {
    const int S = (int)nseg(q);
    hipLaunchKernelGGL(k_reduce_stage1<double>, dim3((a.P + 63) / 64, S), dim3(256), 0, st, a.part, (int)q, a.P,
                       part2);
    hipLaunchKernelGGL(k_reduce_stage2, dim3((a.P + 255) / 256), dim3(256), 0, st, part2, S, a.P, a.gprm);
  }
  return launched();
}

size_t ews_lift_residual_bytes(const ews_lift_desc* s) {
  if (lift_check(s) != EWS_OK) return 0;
  const LArgs a = lift_args(s);
  return al256f((size_t)a.B * 4) + al256f((size_t)a.B * a.nch * a.H * 8);
}

size_t ews_lift_workspace_bytes(const ews_lift_desc* s) {
  if (lift_check(s) != EWS_OK) return 0;
  const LArgs a = lift_args(s);
  const size_t q = (size_t)a.B * a.nch;
  const size_t P = a.wl * a.hl > 0 ? a.wl * a.hl : 1;
  return al256f(q * 2 * a.Hin * 8) + al256f(q * P * 4) + al256f(nseg(q) * P * 8);
}

int ews_lift_forward(const ews_lift_desc* s, const float* branch, const float* theta_app, const uint8_t* mask,
                     const float* matrix, float* path, void* residual, ews_stream_t stream) {
  const int rc = lift_check(s);
  if (rc != EWS_OK) return rc;
  LArgs a = lift_args(s);
  if (!branch || !path || !residual || (a.app && !theta_app) || (a.has_mask && !mask) ||
      (a.lift != EWS_LIFT_NONE && !matrix))
    return EWS_ERR_NULL;
  a.br = branch;
  a.tha = theta_app;
  a.m = mask;
  a.M = matrix;
  a.p = path;
  lift_residual(a, residual);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const dim3 grid(a.nch, a.B);
  if (a.has_mask) hipLaunchKernelGGL(k_last_row, dim3(a.B), dim3(256), 0, st, mask, a.L, a.nrow);
  if (a.incr) hipLaunchKernelGGL(k_lift_sums, grid, dim3(256), 0, st, a);
  const size_t lf = lds_bytes(lift_lds(a, false, false, true, true), kFwdDoubles);
  (void)hipFuncSetAttribute(reinterpret_cast<const void*>(k_lift_rows), hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)lf);
  hipLaunchKernelGGL(k_lift_rows, grid, dim3(256), lf, st, a);
  return launched();
}

int ews_lift_backward(const ews_lift_desc* s, const float* branch, const float* theta_app, const uint8_t* mask,
                      const float* matrix, const void* residual, const float* grad_path, float* grad_branch,
                      float* grad_theta_app, float* grad_matrix, void* workspace, ews_stream_t stream) {
  const int rc = lift_check(s);
  if (rc != EWS_OK) return rc;
  LArgs a = lift_args(s);
  if (!branch || !residual || !grad_path || !grad_branch || !workspace || (a.app && (!theta_app || !grad_theta_app)) ||
      (a.has_mask && !mask) || (a.lift != EWS_LIFT_NONE && (!matrix || !grad_matrix)))
    return EWS_ERR_NULL;
  a.br = branch;
  a.tha = theta_app;
  a.m = mask;
  a.M = matrix;
  a.gp = grad_path;
  a.gbr = grad_branch;
  a.gtha = grad_theta_app;
  a.gM = grad_matrix;
  lift_residual(a, const_cast<void*>(residual));
  char* w = static_cast<char*>(workspace);
  const size_t q = (size_t)a.B * a.nch;
  a.dsum = reinterpret_cast<double*>(w);
  const size_t P = a.wl * a.hl > 0 ? a.wl * a.hl : 1;
  a.part = reinterpret_cast<float*>(w + al256f(q * 2 * a.Hin * 8));
  a.part2 = reinterpret_cast<double*>(w + al256f(q * 2 * a.Hin * 8) + al256f(q * P * 4));
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const dim3 grid(a.nch, a.B);
  const size_t lb = lds_bytes(lift_lds(a, true, true, false, false), kBsumDoubles);
  const size_t lr = lds_bytes(lift_lds(a, true, true, true, true), kBrowDoubles);
  (void)hipFuncSetAttribute(reinterpret_cast<const void*>(k_lift_bsums), hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)lb);
  (void)hipFuncSetAttribute(reinterpret_cast<const void*>(k_lift_brows), hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)lr);
  // the per-chunk sums serve the increment path's reverse carry and the fill's tail only
  if (a.incr || a.has_mask) hipLaunchKernelGGL(k_lift_bsums, grid, dim3(256), lb, st, a);
  hipLaunchKernelGGL(k_lift_brows, grid, dim3(256), lr, st, a);
  if (a.lift != EWS_LIFT_NONE) {
    const int S = (int)nseg(q), Pm = a.wl * a.hl;
    hipLaunchKernelGGL(k_reduce_stage1<float>, dim3((Pm + 63) / 64, S), dim3(256), 0, st, a.part, (int)q, Pm,
                       a.part2);
    hipLaunchKernelGGL(k_reduce_stage2, dim3((Pm + 255) / 256), dim3(256), 0, st, a.part2, S, Pm, a.gM);
  }
  return launched();
}

}  // extern "C"
